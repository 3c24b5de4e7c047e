"""tp_decode_attention_noalloc (static device scratch, no allocation) against
tp_decode_attention (caller workspace) through the C ABI.

Both run the same kernel with the same split, so their outputs must be bit
identical; two calls in a row, the second on a smaller input, check that the
scratch left by one call (records, counters) does not leak into the next.  The
first call is also checked against the oracle at the north_star tolerance."""

import ctypes

import numpy as np
import pytest
import torch

from common import LAYOUTS, PAGE
from test_gpu_attention import SCALE16, build_case, check, oracle_out
from turbopolar_amd import _lib
from turbopolar_amd.kernels import PageSet

pytestmark = pytest.mark.gpu


def _call(L, fn, case, pps, ws=None):
    ps, qt, tk, tv, hq, hkv, S, tail, out = case
    stream = torch.cuda.current_stream().cuda_stream
    common = (qt.data_ptr(), 1, hq, hkv, ctypes.byref(ps.layout), ctypes.byref(ps.pages), S,
              tk.data_ptr() if tail else None, tv.data_ptr() if tail else None, tail, tail if tail else 0,
              S * PAGE + tail, SCALE16, pps)
    if fn == "noalloc":
        st = L.tp_decode_attention_noalloc(*common, out.data_ptr(), stream)
    else:
        st = L.tp_decode_attention(*common, ws.data_ptr(), ws.numel(), out.data_ptr(), stream)
    assert st == 0, L.tp_last_error()


def _case(device, hq, hkv, S, tail, seed):
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS["default"], hq, hkv, S, tail, seed=seed)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    case = (PageSet(block, qv), t(q), t(tk), t(tv), hq, hkv, S, tail,
            torch.full((1, hq, 128), float("nan"), dtype=torch.float16, device=device))
    return case, (host, tk, tv, q)


def test_noalloc_matches_workspace_entry_point(device):
    L = _lib.lib()
    first, host1 = _case(device, 32, 8, 40, 13, seed=91)
    second, host2 = _case(device, 8, 2, 9, 3, seed=92)  # smaller: fewer units and splits
    for case, pps, host in ((first, 2, host1), (second, 1, host2)):
        hq, hkv, S, tail = case[4], case[5], case[6], case[7]
        print(f"[noalloc] hq={hq} hkv={hkv} S={S} tail={tail} pps={pps}", flush=True)
        need = int(L.tp_decode_workspace_bytes(1, hq, hkv, S, tail, pps))
        assert 0 < need <= _lib.TP_NOALLOC_SCRATCH_BYTES
        ws = torch.zeros(need, dtype=torch.uint8, device=device)
        ref = torch.empty_like(case[8])
        _call(L, "workspace", case[:8] + (ref,), pps, ws)
        _call(L, "noalloc", case, pps)
        torch.cuda.synchronize()
        assert torch.equal(case[8], ref), "noalloc output differs from the workspace entry point"
        check(case[8].float().cpu().numpy(), oracle_out(host[0], host[1], host[2], host[3], S * PAGE + tail),
              f"noalloc S={S}")
    # and again on the first input, after the smaller call left its records behind
    out_again = torch.empty_like(first[8])
    _call(L, "noalloc", first[:8] + (out_again,), 2)
    torch.cuda.synchronize()
    assert torch.equal(out_again, first[8])


def test_noalloc_rejects_calls_beyond_its_scratch(device):
    L = _lib.lib()
    lay = _lib.make_layout(False, 4, 4, 64)
    pages = _lib.TPPages(4096, 0, 8192, 12288, 16384, 20480, 4096)  # never dereferenced
    # 64 kv heads x 512 one-page splits need far more than the static scratch
    st = L.tp_decode_attention_noalloc(4096, 1, 64, 64, ctypes.byref(lay), ctypes.byref(pages), 512, None, None,
                                       0, 0, 512 * PAGE, SCALE16, 1, 8192, None)
    assert st == _lib.TP_ERR_WORKSPACE and b"static scratch" in L.tp_last_error()
