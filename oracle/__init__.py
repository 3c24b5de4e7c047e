"""CPU oracle for the TurboPolar compressed-KV decode-attention path.

TEST INFRASTRUCTURE ONLY. This package is a NumPy restatement of the
reference's CPU path (the MLX-op codecs and the ``_cpu_*`` attention
fallbacks of ``rfsn_v11``).  It exists to check the HIP library, never to
stand in for it: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product package
``turbopolar_amd`` never imports it and has no CPU fallback.

Parity status per function (what pins it is listed in ``tests/test_oracle_*.py``):

* ``encode_block`` / ``quantize_block`` -- pinned by the closed-form known
  answers (axis-aligned angles, 3-4-5 radius, fp16 overflow, zero V group,
  group-max codes, half-even ties), by an independent exact-rational
  restatement (``tests/exact_f16.py``) on random and edge inputs, and by the
  packed-shape rules of the reference's own tests.  The MLX boundary itself
  (exact ulps of MLX's fp16 ``arctan2``/``log``) cannot be imported here; the
  documented policy is "correctly rounded", see ``oracle/turbopolar.py``.
* ``decode_block`` -- pinned by the invariants |k_hat pair| == radius and
  encode(decode(codes)) == codes.
* ``dequantize_block`` -- pinned by exact-rational known answers element by
  element (dim d takes the scale of group d // 32 of its own token), by the
  exact round trip of values that are code x power-of-two, and by the
  quantisation error bound |v - dequantize(quantize(v))| <= 0.53125 s + half
  an fp16 ulp on groups whose magnitudes differ by up to 2^16.
* ``cpu_fused_qk`` / ``cpu_online_attention`` /
  ``cpu_online_attention_dense_v`` / ``cpu_online_attention_dense_tail`` -- pinned against textbook softmax
  attention computed independently with torch float64 SDPA on the decoded
  K/V, and against brute-force loops on tiny inputs.
"""

from .turbopolar import *  # noqa: F401,F403
from .turbopolar import __all__  # noqa: F401
