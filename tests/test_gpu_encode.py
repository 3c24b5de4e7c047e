"""Encode kernel parity: codes and scales bit-exact against the oracle.

Runs tp_encode_pages through the C ABI on the GPU and compares every output
buffer byte for byte with the NumPy restatement of
PolarQuantEncoder.encode_block / GroupedVQuantizer.quantize_block.  The scalar
fp16 helpers the kernel is built on are checked exhaustively.
"""

import ctypes
import sys

import numpy as np
import pytest
import torch

import oracle
from common import LAYOUTS, PAGE, edge_page, gen_kv, oracle_pages
from turbopolar_amd import _lib, kernels
from turbopolar_amd.codecs import PolarQuantEncoder
from turbopolar_amd.config import TurboPolarConfig

pytestmark = pytest.mark.gpu


def _encoder(layout):
    int8, l1b, deepb, split = layout
    cfg = TurboPolarConfig(
        k_angle_bits_level1=l1b, k_angle_bits_deep=deepb, split_dim=split, use_int8_radii=int8,
        num_q_heads=8, num_kv_heads=8,
    )
    return PolarQuantEncoder(cfg)


def encode_gpu(k, v, layout, device, capacity=None, page_begin=0, n_tokens=None):
    """Encode [B,H,T,128] numpy inputs on the GPU; returns numpy page buffers."""
    enc = _encoder(layout)
    B, H, T, _ = k.shape
    n_tokens = T if n_tokens is None else n_tokens
    S = (n_tokens + PAGE - 1) // PAGE
    cap = capacity or (page_begin + S)
    bufs = enc.alloc_pages(B, H, cap, device)
    codes = torch.zeros((B, H, cap, PAGE, 128), dtype=torch.int8, device=device)
    scales = torch.zeros((B, H, cap, PAGE, 4), dtype=torch.float16, device=device)
    pages = _lib.TPPages(
        _lib.ptr(bufs["radii"]), _lib.ptr(bufs["radii_scales"]), _lib.ptr(bufs["angle_codes_l1"]),
        _lib.ptr(bufs["angle_codes_deep"]), _lib.ptr(codes), _lib.ptr(scales), cap,
    )
    kernels.encode_pages(
        torch.from_numpy(k).to(device), torch.from_numpy(v).to(device), 0, n_tokens, enc.layout, pages, page_begin
    )
    torch.cuda.synchronize()
    sl = slice(page_begin, page_begin + S)
    out = {name: (t[:, :, sl].cpu().numpy() if t is not None else None) for name, t in bufs.items()}
    out["v_codes"] = codes[:, :, sl].cpu().numpy()
    out["v_scales"] = scales[:, :, sl].cpu().numpy()
    return out


def assert_bits_equal(gpu, ref, what):
    gpu = np.ascontiguousarray(gpu)
    ref = np.ascontiguousarray(ref)
    assert gpu.shape == ref.shape, (what, gpu.shape, ref.shape)
    g = gpu.view(np.uint8)
    r = ref.view(np.uint8)
    bad = np.count_nonzero(g != r)
    assert bad == 0, f"{what}: {bad} of {g.size} bytes differ"


def check_against_oracle(k, v, layout, device, **kw):
    gpu = encode_gpu(k, v, layout, device, **kw)
    blk, (vc, vs) = oracle_pages(k, v, layout)
    assert_bits_equal(gpu["radii"], blk["radii"], "radii")
    if layout[0]:
        assert_bits_equal(gpu["radii_scales"], blk["radii_scales"].reshape(gpu["radii_scales"].shape), "radii_scales")
    assert_bits_equal(gpu["angle_codes_l1"], blk["angle_codes_l1"], "angle_codes_l1")
    assert_bits_equal(gpu["angle_codes_deep"], blk["angle_codes_deep"], "angle_codes_deep")
    assert_bits_equal(gpu["v_codes"], vc, "v_codes")
    assert_bits_equal(gpu["v_scales"], vs, "v_scales")


@pytest.mark.parametrize("layout_name", sorted(LAYOUTS))
@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_encode_random_bit_exact(device, layout_name, dtype):
    print(f"[encode] layout={layout_name} dtype={np.dtype(dtype).name}", flush=True)
    k, v = gen_kv(3, 1, 2, 4 * PAGE, "normal", dtype)
    check_against_oracle(k, v, LAYOUTS[layout_name], device)


@pytest.mark.parametrize("kind", ["loguniform", "outlier", "studentt"])
@pytest.mark.parametrize("layout_name", ["default", "fast"])
def test_encode_baseline_distributions(device, kind, layout_name):
    print(f"[encode] kind={kind} layout={layout_name}", flush=True)
    k, v = gen_kv(11, 2, 3, 3 * PAGE, kind, np.float16)
    check_against_oracle(k, v, LAYOUTS[layout_name], device)


@pytest.mark.parametrize("layout_name", ["default", "fast", "deep2", "l1_8bit"])
@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_encode_edge_page(device, layout_name, dtype):
    print(f"[encode-edge] layout={layout_name} dtype={np.dtype(dtype).name}", flush=True)
    k, v = edge_page(dtype)
    check_against_oracle(k, v, LAYOUTS[layout_name], device)


@pytest.mark.parametrize("layout_name", ["default", "fast"])
def test_encode_partial_page_zero_padded(device, layout_name):
    """n_tokens < 64: the missing tokens encode as zeros (_maybe_encode_partial)."""
    print(f"[encode-partial] layout={layout_name}", flush=True)
    k, v = gen_kv(21, 1, 2, 37, "normal", np.float16)
    gpu = encode_gpu(k, v, LAYOUTS[layout_name], device)
    kp = np.zeros((1, 2, PAGE, 128), np.float16)
    vp = np.zeros((1, 2, PAGE, 128), np.float16)
    kp[:, :, :37], vp[:, :, :37] = k, v
    blk, (vc, vs) = oracle_pages(kp, vp, LAYOUTS[layout_name])
    assert_bits_equal(gpu["radii"], blk["radii"], "radii")
    assert_bits_equal(gpu["angle_codes_deep"], blk["angle_codes_deep"], "deep")
    assert_bits_equal(gpu["v_codes"], vc, "v_codes")
    assert_bits_equal(gpu["v_scales"], vs, "v_scales")


@pytest.mark.parametrize("layout_name", ["default", "fast"])
@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_encode_nan_inputs(device, layout_name, dtype):
    """NaN in x, in y and in a whole token row of K, and in one V group: the
    oracle's rules (NaN codes are 0; in the log-int8 layout a NaN radius makes
    the page's max |log r|, so its scale, NaN and every radius code 0)."""
    print(f"[encode-nan] layout={layout_name} dtype={np.dtype(dtype).name}", flush=True)
    k, v = gen_kv(31, 1, 2, 3 * PAGE, "normal", np.float32)
    k[0, 0, 5, 10] = np.nan           # page 0: x of pair 5
    k[0, 0, 40, 33] = np.nan          # page 0: y of pair 16
    k[0, 1, PAGE + 7, :] = np.nan     # page 1 of head 1: a whole token
    v[0, 0, 2 * PAGE + 3, 64 + 9] = np.nan  # page 2: one V group
    check_against_oracle(k.astype(dtype), v.astype(dtype), LAYOUTS[layout_name], device)


@pytest.mark.parametrize("layout_name", ["default", "fast"])
@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_encode_inf_inputs(device, layout_name, dtype):
    """Infinite K components in every sign combination, alone and in pairs
    (atan2(+-inf, +-inf) is an odd multiple of pi/4, atan2(+-inf, finite) is
    +-pi/2 and atan2(finite, -inf) is +-pi), and infinite V values: codes and
    scales as the oracle's (the radius is inf, so in the log-int8 layout the
    page's scale is inf and its radius codes 0)."""
    print(f"[encode-inf] layout={layout_name} dtype={np.dtype(dtype).name}", flush=True)
    k, v = gen_kv(33, 1, 2, 2 * PAGE, "normal", np.float32)
    inf = np.inf
    pairs = [(inf, inf), (-inf, inf), (inf, -inf), (-inf, -inf), (inf, 3.0), (-inf, 0.0), (inf, 0.0),
             (-2.0, inf), (5.0, -inf), (0.0, inf), (0.0, -inf), (-inf, -7.5)]
    for i, (x, y) in enumerate(pairs):
        t, j = 3 + 5 * i, (7 * i) % 64       # page 0 of head 0, scattered tokens and pairs
        k[0, 0, t, 2 * j], k[0, 0, t, 2 * j + 1] = x, y
    k[0, 1, PAGE + 11, 40] = -inf         # page 1 of head 1: one component
    v[0, 0, 9, 3] = inf                   # V groups with +inf and -inf
    v[0, 1, PAGE + 2, 100] = -inf
    check_against_oracle(k.astype(dtype), v.astype(dtype), LAYOUTS[layout_name], device)


def test_encode_into_capacity_slot(device):
    """Pages land in slots [page_begin, page_begin + S) of a larger store."""
    k, v = gen_kv(8, 2, 2, 2 * PAGE, "normal", np.float16)
    check_against_oracle(k, v, LAYOUTS["default"], device, capacity=8, page_begin=3)


def test_f16_tables_exhaustive(device):
    """sqrt, log and the angle->code rule over all 65536 fp16 bit patterns."""
    sq = torch.empty(65536, dtype=torch.int16, device=device)
    lg = torch.empty(65536, dtype=torch.int16, device=device)
    cd = torch.empty(65536 * 3, dtype=torch.uint8, device=device)
    st = _lib.lib().tp_selftest_f16_tables(sq.data_ptr(), lg.data_ptr(), cd.data_ptr(),
                                           torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "selftest tables")
    torch.cuda.synchronize()
    sq = sq.cpu().numpy().view(np.uint16)
    lg = lg.cpu().numpy().view(np.uint16)
    cd = cd.cpu().numpy().reshape(65536, 3)
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = bits.view(np.float16)
    nonneg = np.arange(0, 0x7C01)  # +0 .. +inf
    ref_sq = np.sqrt(f[nonneg]).view(np.uint16)
    assert np.array_equal(sq[nonneg], ref_sq), "sqrt table differs"
    pos = np.arange(1, 0x7C01)
    ref_lg = oracle.log_cr(np.maximum(f[pos], oracle.turbopolar.F16_RADIUS_FLOOR)).view(np.uint16)
    assert np.array_equal(lg[pos], ref_lg), f"log differs at {np.count_nonzero(lg[pos] != ref_lg)} inputs"
    angles = np.concatenate([np.arange(0, 0x4249), np.arange(0x8000, 0xC249)])  # |a| <= fp16(pi)
    for col, nb in enumerate((2, 4, 8)):
        ref = oracle.angle_codes_f16(f[angles], nb)
        bad = np.count_nonzero(cd[angles, col] != ref)
        assert bad == 0, f"{nb}-bit angle codes differ for {bad} angles"


def test_atan2_fast_path_exhaustive(device):
    """Fast fp32 atan2 + midpoint guard == float64 path, and the specialised
    encoder's 4- and 8-bit angle codes == the codes of the float64 angle, for
    every finite fp16 pair."""
    cnt = torch.zeros(1, dtype=torch.int64, device=device)
    step = 4096
    for x0 in range(0, 65536, step):
        st = _lib.lib().tp_selftest_atan2_exhaustive(cnt.data_ptr(), x0, step, torch.cuda.current_stream().cuda_stream)
        _lib.check(st, "selftest atan2")
    torch.cuda.synchronize()
    assert int(cnt.item()) == 0, f"{int(cnt.item())} fp16 pairs where the fast atan2 differs"


def test_v_quotient_fast_path_exhaustive(device):
    """Reciprocal-product fp16 division + midpoint guard == correctly rounded
    fp16(v / s) for every positive finite fp16 scale and every finite value."""
    cnt = torch.zeros(1, dtype=torch.int64, device=device)
    step = 4096
    for s0 in range(0, 32768, step):
        st = _lib.lib().tp_selftest_div_f16_exhaustive(cnt.data_ptr(), s0, step, torch.cuda.current_stream().cuda_stream)
        _lib.check(st, "selftest div")
    torch.cuda.synchronize()
    assert int(cnt.item()) == 0, f"{int(cnt.item())} (v, s) pairs where the fast quotient differs"


def test_v_code_fast_path_exhaustive(device):
    """The specialised fp16 encoder's V codes (reciprocal-product quotient,
    biased byte conversion that rounds half to even and saturates, exact redo
    near an fp16 midpoint) == int8(clip(rint(fp16(v / s)), -128, 127)) for
    every positive finite fp16 scale and every finite value."""
    cnt = torch.zeros(1, dtype=torch.int64, device=device)
    step = 4096
    for s0 in range(0, 32768, step):
        st = _lib.lib().tp_selftest_vcode_exhaustive(cnt.data_ptr(), s0, step, torch.cuda.current_stream().cuda_stream)
        _lib.check(st, "selftest vcode")
    torch.cuda.synchronize()
    assert int(cnt.item()) == 0, f"{int(cnt.item())} (v, s) pairs where the fast V code differs"


def test_log_radius_code_fast_path_exhaustive(device):
    """The specialised fp16 encoder's int8 log-radius codes (reciprocal FMA
    with the +128 bias, byte conversion that rounds half to even, exact redo
    near a half-integer) == int8(clip(rint(f32(lr / s)), -128, 127)) for every
    positive finite fp16 scale s and every finite fp16 lr the encoder can pair
    with it (|lr / s| < 127.1: lr is at most the page's max |lr|, and s is
    fp16(max |lr| / 127))."""
    cnt = torch.zeros(1, dtype=torch.int64, device=device)
    step = 4096
    for s0 in range(0, 32768, step):
        st = _lib.lib().tp_selftest_lcode_exhaustive(cnt.data_ptr(), s0, step, torch.cuda.current_stream().cuda_stream)
        _lib.check(st, "selftest lcode")
    torch.cuda.synchronize()
    assert int(cnt.item()) == 0, f"{int(cnt.item())} (lr, s) pairs where the fast log-radius code differs"
