"""CPU oracle of the DeltaAttention prefill path.

TEST INFRASTRUCTURE ONLY.  This package restates the reference's algorithm
(Emruur/DeltaAttention: tritonModules.py, deltaFlashAttention.py,
flashAttention.py, deltaDecoding.py and the attention glue in
modeling_llama.py) on the CPU so that the HIP kernels can be checked against
it.  Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg
of ``bench.py`` may import it, and there only as the checker or as the timed
CPU baseline; the product package ``deltaattention_amd`` never imports it and
has no CPU fallback.

Parity pinning (what fixes each function besides this restatement):

* ``select_delta`` -- closed-form constructions whose anchor sets are known
  analytically (collinear keys with a known step, constant keys, the strict
  ``>`` at an exactly representable threshold, chunk restarts), plus the C
  restatement ``select_oracle.c`` agreeing bit for bit with the numpy one.
* ``index_map`` / ``pack`` -- integer closed forms (cumsum, run lengths that
  sum to N, timestamps strictly increasing, K-hat rows equal K at ts).
* ``hybrid_attention`` -- golden vectors written by the reference's own
  Triton kernels (``tests/golden/make_golden.py``) plus the invariants
  keep-all => dense causal and W >= N => dense causal, and an independent
  fp64 brute force.
* ``dense_attention`` -- textbook softmax(Q K^T * scale + causal mask) V.
* ``decode_update`` / ``decode_attention`` -- constructed merge/append
  sequences with known distances, count conservation, and the log-count
  identity exp(s + log c) = c * exp(s) (count-c anchor == c repeated keys).
"""
