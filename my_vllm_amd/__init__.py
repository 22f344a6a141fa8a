"""MI355X-native (gfx950) ragged-batch attention hot path for Nano-vLLM-v1.

* ``contract``: the backend-neutral interface the reference's model runner
  drives (``CommonAttentionMetadata``, ``BatchType``, ``AttentionPlan``,
  ``AttentionRoute``, the ``AttentionBackend`` base).
* ``attention_backend``: the gfx950 backend (``MI355XAttentionBackend``,
  ``MI355XSplitAttentionBackend``) and ``integrate``, which registers it in
  the reference's own registry.
* ``layers`` / ``providers``: drop-in ``SiluAndMul``, ``KVCacheStore``,
  ``RMSNorm`` and ``RotaryEmbedding`` operators on the gfx950 kernels, and
  the provider names that select them.
* ``ops``: validated wrappers over the C ABI of ``lib/libmy_vllm_amd.so``.

Importing the package does not load the native library; the first kernel
use (or backend construction) does, and fails loudly if it is missing.
"""

from .contract import BatchType, CommonAttentionMetadata  # noqa: F401

__all__ = ["BatchType", "CommonAttentionMetadata"]
