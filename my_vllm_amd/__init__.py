"""MI355X-native (gfx950) ragged-batch attention hot path for Nano-vLLM-v1.

Public surface, mirroring the reference's interfaces:

* ``attention_backend``: ``AttentionBackend`` lifecycle, ``AttentionPlan`` /
  ``AttentionRoute``, ``AttentionBackendRegistry`` and the gfx950 backend
  (``MI355XAttentionBackend``, registered as ``"mi355x"``).
* ``context``: ``CommonAttentionMetadata`` / ``BatchType`` step contract.
* ``activation.SiluAndMul`` and ``attention.KVCacheStore`` CustomOps.
* ``ops``: validated wrappers over the C ABI of ``lib/libmy_vllm_amd.so``.

Importing the package does not load the native library; the first kernel
use (or backend construction) does, and fails loudly if it is missing.
"""

from .context import BatchType, CommonAttentionMetadata  # noqa: F401

__all__ = ["BatchType", "CommonAttentionMetadata"]
