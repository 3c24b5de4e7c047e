"""Seeded random sweep of decode-attention shapes against the oracle.

Each case draws a batch (1-3), kv heads (1-5), a GQA group (1-24: one or two
head blocks of 16), a page count (1-140), a tail (0-63 tokens), a masked
suffix, a pages-per-split (library default or 1-9) and a layout, so the
workgroup-index arithmetic meets unit counts that are not powers of two, and
split counts land on both sides of the two-tier combine's threshold (64
splits per unit) with ragged last groups.  Bar: max-abs <= 2e-3 and relative
L2 <= 1e-3 against the oracle's float64 restatement of
_cpu_online_attention_dense_tail (metal.py:293-332).
"""

import numpy as np
import pytest

from common import LAYOUTS, PAGE
from test_gpu_attention import build_case, check, oracle_out, run_gpu

pytestmark = pytest.mark.gpu


def _draw(seed):
    r = np.random.default_rng(1000 + seed)
    B = int(r.integers(1, 4))
    hkv = int(r.integers(1, 6))
    g = int(r.choice([1, 2, 3, 4, 5, 7, 8, 12, 16, 20, 24]))
    S = int(r.choice([1, 2, 5, 9, 17, 33, 65, 66, 80, 97, 129, 140]))
    tail = int(r.choice([0, 0, 1, 17, 37, 63]))
    pps = int(r.choice([0, 0, 1, 1, 2, 3, 9]))
    layout = str(r.choice(["default", "default", "fast", "deep2"]))
    total = S * PAGE + tail
    drop = int(r.choice([0, 0, 0, 1, 30, 100]))
    drop = min(drop, total - 1)
    return B, hkv, g, S, tail, pps, layout, drop


CASES = [_draw(i) for i in range(24)]


@pytest.mark.parametrize("B,hkv,g,S,tail,pps,layout_name,drop", CASES)
def test_decode_attention_random_shapes(device, B, hkv, g, S, tail, pps, layout_name, drop):
    hq = hkv * g
    print(f"[attn-sweep] B={B} hkv={hkv} hq={hq} S={S} tail={tail} pps={pps} layout={layout_name} drop={drop}",
          flush=True)
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS[layout_name], hq, hkv, S, tail,
                                            seed=7 * S + 3 * g + hkv + B, B=B)
    seq = S * PAGE + tail - drop
    out = run_gpu(device, block, qv, tk, tv, q, seq, pps)
    assert out.shape == (B, hq, 128)
    check(out, oracle_out(host, tk, tv, q, seq), f"sweep B={B} hkv={hkv} g={g} S={S} pps={pps}")
