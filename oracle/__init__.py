"""CPU oracle for the MI355X hot path — TEST INFRASTRUCTURE ONLY.

A restatement, in plain torch/numpy on the CPU, of the reference's native
(non-FlashInfer) arithmetic for each kernel of this repository.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may
import it, and only to check results or as the timed CPU baseline: the product
package (``my_vllm_amd``) never imports it and has no CPU fallback.

How each function is pinned (the tests under ``tests/test_oracle*.py``):

* ``kv_store``            — the reference's known-answer test
  (tests/test_custom_op_dispatch.py:75-95) plus brute force.
* ``silu_and_mul_*``      — closed form g*sigmoid(g)*u evaluated with
  ``math.exp`` in Python, and torch's ``F.silu`` (a library routine).
* ``rms_norm`` / ``fused_add_rms_norm`` — torch's ``F.rms_norm`` (a library
  routine, single rounding: within 1 ulp), closed forms (constant rows give
  sign(c) * w; a row of k copies of +-c), the fp32-sum statistics of the
  fused form, and a planted statistics-of-the-rounded-sum mistake.
* ``rope`` / ``qk_norm_rope`` — position 0 is the identity, the rotation of
  each (x_j, x_{j+64}) pair matches a float64 complex multiplication by
  e^{i p theta_j}, pair norms are preserved, and a planted interleaved
  (GPT-J) pairing is caught.
* ``paged_attention`` / ``ragged_attention`` — pure-Python brute force on tiny
  inputs, ``F.scaled_dot_product_attention`` on the cacheless causal case,
  and invariants (one-key context returns V exactly; equal scores give the
  mean of V; a split-K/LSE merge equals the unsplit result).
* ``page_csr`` / ``slot_mapping_for`` / ``classify_batch`` — integer
  known-answer vectors from the reference's tests (fixtures under
  ``tests/golden/``).
"""
