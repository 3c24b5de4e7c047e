"""The HIP kernels against the committed golden fixtures (tests/golden).

Encode: the fixture inputs encode to the fixture's codes and scales byte for
byte (random pages for the default and fast layouts; the edge page in fp16 and
fp32 for four layouts).  Page decode: V exactly, K within one fp16 ulp.
Attention: the fixture's pages, tails and queries give the fixture's outputs
within max-abs 2e-3 and relative L2 1e-3.
"""

import numpy as np
import pytest
import torch

from common import ATOL, LAYOUTS, PAGE, RTOL_L2, load_golden, max_abs, rel_l2, within_f16_ulp
from test_gpu_encode import assert_bits_equal, encode_gpu
from turbopolar_amd import kernels
from turbopolar_amd.kernels import PageSet, fp16_scale
from turbopolar_amd.payload import PolarKeyBlock, QuantizedVBlock, layout_metadata

pytestmark = pytest.mark.gpu

SCALE16 = fp16_scale(1.0 / np.sqrt(128.0))
FIELDS = ("radii", "radii_scales", "angle_codes_l1", "angle_codes_deep", "v_codes", "v_scales")


def _layout(fix):
    int8, l1, deep, split = (int(x) for x in fix["layout"])
    return (bool(int8), l1, deep, split)


def _compare(gpu, fix, prefix, what):
    for f in FIELDS:
        if prefix + f not in fix:
            continue
        ref = fix[prefix + f]
        assert_bits_equal(gpu[f].reshape(ref.shape), ref, f"{what} {f}")


def _pageset(fix, device):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    int8, l1, deep, split = _layout(fix)
    B, H, S = fix["radii"].shape[:3]
    meta = layout_metadata(l1, deep, split, int8)
    block = PolarKeyBlock(
        radii=t(fix["radii"]), angle_codes_l1=t(fix["angle_codes_l1"]), angle_codes_deep=t(fix["angle_codes_deep"]),
        shape=(B, H, S * PAGE, 128), block_size=PAGE, head_dim=128, metadata=meta,
        radii_scales=t(fix["radii_scales"]) if int8 else None,
    )
    qv = QuantizedVBlock(codes=t(fix["v_codes"]), scales=t(fix["v_scales"]), group_size=32)
    return PageSet(block, qv)


@pytest.mark.parametrize("name", ["default", "fast"])
def test_golden_encode(device, name):
    print(f"[golden-encode] layout={name}", flush=True)
    inp, fix = load_golden("inputs.npz"), load_golden(f"layout_{name}.npz")
    gpu = encode_gpu(inp["k"], inp["v"], _layout(fix), device)
    _compare(gpu, fix, "", name)


@pytest.mark.parametrize("name", ["default", "fast", "deep2", "l1_8bit"])
@pytest.mark.parametrize("dtype", ["float16", "float32"])
def test_golden_edge_page(device, name, dtype):
    print(f"[golden-edge] layout={name} dtype={dtype}", flush=True)
    inp = load_golden("inputs.npz")
    fix = load_golden(f"layout_{name}.npz" if name in ("default", "fast") else f"edge_{name}.npz")
    gpu = encode_gpu(inp[f"edge_k_{dtype}"], inp[f"edge_v_{dtype}"], LAYOUTS[name], device)
    _compare(gpu, fix, f"{dtype}__", f"{name}/{dtype}")


@pytest.mark.parametrize("name", ["default", "fast"])
def test_golden_page_decode(device, name):
    print(f"[golden-decode] layout={name}", flush=True)
    fix = load_golden(f"layout_{name}.npz")
    kg, vg = kernels.decode_pages(_pageset(fix, device))
    torch.cuda.synchronize()
    assert np.array_equal(vg.cpu().numpy().view(np.uint16), fix["v_decoded"].view(np.uint16))
    assert within_f16_ulp(kg.cpu().numpy(), fix["k_decoded"])


@pytest.mark.parametrize("name", ["default", "fast"])
@pytest.mark.parametrize("g", [1, 4, 8])
@pytest.mark.parametrize("tail", [0, 1, 37, 63])
def test_golden_attention(device, name, g, tail):
    print(f"[golden-attn] layout={name} gqa={g} tail={tail}", flush=True)
    inp, fix = load_golden("inputs.npz"), load_golden(f"layout_{name}.npz")
    pages = _pageset(fix, device)
    q = torch.from_numpy(inp[f"q_g{g}"]).to(device)
    tk = torch.from_numpy(np.ascontiguousarray(inp["tail_k"][:, :, :tail])).to(device) if tail else None
    tv = torch.from_numpy(np.ascontiguousarray(inp["tail_v"][:, :, :tail])).to(device) if tail else None
    seq = fix["radii"].shape[2] * PAGE + tail
    for pps in (0, 1):
        out = kernels.decode_attention(q, pages, tk, tv, seq, SCALE16, pages_per_split=pps)
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        ref = fix[f"out_g{g}_t{tail}"]
        assert max_abs(got, ref) <= ATOL and rel_l2(got, ref) <= RTOL_L2, (pps, max_abs(got, ref))


@pytest.mark.parametrize("name", ["default", "fast"])
def test_golden_attention_masked(device, name):
    print(f"[golden-attn-mask] layout={name}", flush=True)
    inp, fix = load_golden("inputs.npz"), load_golden(f"layout_{name}.npz")
    out = kernels.decode_attention(torch.from_numpy(inp["q_g4"]).to(device), _pageset(fix, device), None, None,
                                   100, SCALE16)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ref = fix["out_g4_masked"]
    assert max_abs(got, ref) <= ATOL and rel_l2(got, ref) <= RTOL_L2
