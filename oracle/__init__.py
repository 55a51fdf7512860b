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

* ``int4``: numpy bit-level restatement vs the torch expression, brute force over all 256
  byte values x scales; the reference tests' own invariants (K-major pairing, round trip).
* ``model``: golden vectors written by ``tests/golden/make_golden.py`` from the reference
  itself (tiny and mid configs, prefill + decode logits and cache state, one GatedDeltaNet
  step, one GatedAttention step, int4 dequant-GEMV), plus the reference tests' known
  answers and invariants (RMSNorm known answer, rotate_half, RoPE identity at position 0,
  delta-rule step == whole == chunked, beta = 0, conv history shift).
"""
