"""CPU oracle for the Qwen3.5-4B int4 decode path. TEST INFRASTRUCTURE ONLY.

This package restates, in plain PyTorch on the CPU (and numpy for the bit-level int4
work), the arithmetic of the reference's pure-PyTorch baseline
(``/root/reference/src/deltaforge/reference.py``) and of its int4 champion expression
(``kernels/visible_int4_head.py:187-199``, ``kernels/tiled_gemv.py:242-288``). Every
function cites the reference lines it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import it, and only as the *checker* (or as the timed CPU baseline). The product path in
``deltaforge_amd`` never imports, calls or falls back to anything here.

How each part is pinned (a function with no independent pin would say "parity unpinned"):

* ``int4``: the reference's own quantiser bytes, dequant and dequant-GEMV output
  (``tests/golden/int4_gemv.safetensors``, written by the reference), a brute force over all
  256 byte values x scales in integer/float64 arithmetic, the K-major pairing, and the
  quantiser's range and round trip (``tests/test_oracle_invariants.py``).
* ``model``: bit-identical (rtol = atol = 0) to vectors the reference itself wrote with
  ``tests/golden/make_golden.py`` -- tiny and mid configs, dense and int4, prefill logits
  at every position, each greedy step's logits and token, conv history, fp32 recurrent
  state and KV cache (``tests/test_oracle_golden.py``) -- plus the reference tests' known
  answers and invariants: RMSNorm (1 + w), gated RMSNorm closed form, rotate_half, RoPE
  identity at position 0 and the untouched tail, conv history shift, delta rule against a
  float64 closed form, step == whole == chunks, beta = 0, causality.
* ``ops`` (per-config slices used as GPU checkers): each equals, bit for bit, the
  golden-pinned ``OracleModel`` layer it is cut from (``tests/test_oracle_invariants.py``).
"""
