"""The measurement library's decode-kernel variants against the oracle.

bench.py --variant times these variants of the decode kernel beside the product
kernel (libturbopolar_hip_timeline.so, tp_measure_set_decode_variant): the
product kernel with an agent-scope release fence before the split ticket, or
without the combining workgroup's acquire fence, on the product's workgroup
size (4 waves for splits of at most 8 pages, else 8), and the kernel with QK
and PV on the VALU instead of MFMA (default layout, 4 or 8 query heads per kv
head, no tail).  A timing of a variant is evidence only if
the variant computes the same attention: each is checked here against
oracle.cpu_online_attention_dense_tail (metal.py:293-332) at the same bar as
the product kernel (max-abs 2e-3, relative L2 1e-3), with several splits, a
masked last page and batch 2.
"""

import ctypes

import numpy as np
import pytest
import torch

from common import ATOL, LAYOUTS, PAGE, RTOL_L2, max_abs, rel_l2
from test_gpu_attention import SCALE16, build_case, oracle_out
from turbopolar_amd import _lib, build
from turbopolar_amd.kernels import PageSet

pytestmark = pytest.mark.gpu

VARIANT = {"release": 1, "valu": 2, "valu+release": 3, "no-acquire": 4}


@pytest.fixture(scope="module")
def mlib():
    h = _lib.open_library(build.TIMELINE_LIB_PATH)
    h.tp_measure_set_decode_variant.restype = ctypes.c_int32
    h.tp_measure_set_decode_variant.argtypes = [ctypes.c_int32]
    yield h
    h.tp_measure_set_decode_variant(0)


def run_variant(h, device, variant, block, qv, q, seq_len, pps):
    pages = PageSet(block, qv)
    qd = torch.from_numpy(q).to(device)
    B, hq, _ = q.shape
    out = torch.empty((B, hq, 128), dtype=torch.float16, device=device)
    need = int(h.tp_decode_workspace_bytes(B, hq, pages.H, pages.S, 0, pps))
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=device)
    assert h.tp_measure_set_decode_variant(VARIANT[variant]) == 0
    st = h.tp_decode_attention(qd.data_ptr(), B, hq, pages.H, ctypes.byref(pages.layout), ctypes.byref(pages.pages),
                               pages.S, None, None, 0, 0, seq_len, SCALE16, pps, ws.data_ptr(), need,
                               out.data_ptr(), torch.cuda.current_stream(device).cuda_stream)
    assert st == 0, h.tp_last_error().decode()
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


CASES = [
    # variant, layout, hq, hkv, pages, pages_per_split, masked tokens, batch
    ("valu", "default", 32, 8, 5, 2, 0, 1),
    ("valu", "default", 32, 8, 9, 4, 21, 1),
    ("valu", "default", 64, 8, 4, 1, 0, 1),
    ("valu", "default", 64, 8, 7, 3, 40, 2),
    ("valu+release", "default", 32, 8, 6, 2, 0, 1),
    ("valu+release", "default", 64, 8, 6, 2, 5, 1),
    ("release", "default", 32, 8, 5, 2, 0, 1),
    ("release", "fast", 64, 8, 6, 2, 9, 2),
    ("release", "default", 32, 8, 40, 16, 0, 1),     # 16-page splits: 8-wave workgroups
    ("no-acquire", "default", 32, 8, 9, 4, 21, 1),   # 4-wave workgroups
    ("no-acquire", "fast", 64, 8, 6, 2, 9, 2),
    ("no-acquire", "default", 32, 8, 40, 16, 3, 1),
]


@pytest.mark.parametrize("variant,layout_name,hq,hkv,S,pps,masked,B", CASES)
def test_variant_parity(device, mlib, variant, layout_name, hq, hkv, S, pps, masked, B):
    print(f"[variant] {variant} layout={layout_name} hq={hq} hkv={hkv} S={S} pps={pps} masked={masked} B={B}",
          flush=True)
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS[layout_name], hq, hkv, S, 0, seed=31 + S, B=B)
    seq = S * PAGE - masked
    out = run_variant(mlib, device, variant, block, qv, q, seq, pps)
    ref = oracle_out(host, tk, tv, q, seq)
    assert np.all(np.isfinite(out))
    ma, rl = max_abs(out, ref), rel_l2(out, ref)
    assert ma <= ATOL and rl <= RTOL_L2, f"max_abs={ma:.3g} rel_l2={rl:.3g}"


def test_valu_variant_rejects_other_shapes(device, mlib):
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS["default"], 12, 2, 2, 0, seed=3)
    with pytest.raises(AssertionError, match="VALU variant"):
        run_variant(mlib, device, "valu", block, qv, q, 2 * PAGE, 1)
