"""Fused QK and split-K decode attention parity against the oracle.

The pages are encoded once on the GPU; the same pages (copied to the host)
feed the oracle's restatement of _cpu_fused_qk / _cpu_online_attention /
_cpu_online_attention_dense_tail (metal.py:254-332), evaluated in float64.
Tolerances: attention outputs max-abs <= 2e-3 and
relative L2 <= 1e-3; fused QK scores (fp16 out) max-abs <= 1e-2 and cosine
>= 0.999 (tests/benchmarks/test_turbo_polar_kernel_qk.py:57-58 of the reference).
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle
from common import ATOL, LAYOUTS, PAGE, RTOL_L2, cosine, gen_kv, gen_q, max_abs, rel_l2
from turbopolar_amd import kernels
from turbopolar_amd.kernels import PageSet, fp16_scale
from turbopolar_amd.payload import PolarKeyBlock, QuantizedVBlock
from test_gpu_encode import encode_gpu

pytestmark = pytest.mark.gpu

SCALE16 = fp16_scale(1.0 / np.sqrt(128.0))


def build_case(device, layout, hq, hkv, S, tail, seed=0, kind="normal", qscale=1.0, B=1):
    """Encode S pages on the GPU; returns GPU page views, host pages, tails, q."""
    k, v = gen_kv(seed, B, hkv, S * PAGE + tail, kind, np.float16)
    q = gen_q(seed, B, hq, qscale)
    host = None
    block = qv = None
    if S:
        host = encode_gpu(k[:, :, : S * PAGE], v[:, :, : S * PAGE], layout, device)
        meta = oracle.encode_block(k[:, :, :PAGE], l1_bits=layout[1], deep_bits=layout[2],
                                   split_dim=layout[3], use_int8_radii=layout[0])["metadata"]
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
        block = PolarKeyBlock(
            radii=t(host["radii"]), angle_codes_l1=t(host["angle_codes_l1"]),
            angle_codes_deep=t(host["angle_codes_deep"]), shape=(B, hkv, S * PAGE, 128),
            block_size=PAGE, head_dim=128, metadata=meta,
            radii_scales=t(host["radii_scales"]) if layout[0] else None,
        )
        qv = QuantizedVBlock(codes=t(host["v_codes"]), scales=t(host["v_scales"]), group_size=32)
        host["metadata"] = meta
    tk = k[:, :, S * PAGE:]
    tv = v[:, :, S * PAGE:]
    return block, qv, host, tk, tv, q


def oracle_out(host, tk, tv, q, seq_len):
    if host is None:
        return oracle.softmax_attention(q, tk, tv, SCALE16, seq_len)
    blk = {k: host[k] for k in ("radii", "radii_scales", "angle_codes_l1", "angle_codes_deep", "metadata")}
    if blk["radii_scales"] is not None:
        blk["radii_scales"] = blk["radii_scales"].reshape(blk["radii"].shape[:3] + (1, 1))
    return oracle.cpu_online_attention_dense_tail(
        q, blk, (host["v_codes"], host["v_scales"]), tk, tv, SCALE16, seq_len
    )


def run_gpu(device, block, qv, tk, tv, q, seq_len, pps=0):
    pages = PageSet(block, qv) if block is not None else None
    tkt = torch.from_numpy(tk).to(device) if tk.shape[2] else None
    tvt = torch.from_numpy(tv).to(device) if tv.shape[2] else None
    out = kernels.decode_attention(torch.from_numpy(q).to(device), pages, tkt, tvt, seq_len, SCALE16,
                                   pages_per_split=pps)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def check(out, ref, what):
    assert np.all(np.isfinite(out)), f"{what}: non-finite output"
    ma, rl = max_abs(out, ref), rel_l2(out, ref)
    assert ma <= ATOL and rl <= RTOL_L2, f"{what}: max_abs={ma:.3g} rel_l2={rl:.3g}"


CASES = [
    # layout, hq, hkv, S pages, tail tokens, pages_per_split
    ("default", 2, 2, 2, 0, 0),
    ("default", 2, 2, 2, 37, 0),
    ("default", 4, 2, 2, 0, 1),
    ("default", 4, 2, 3, 63, 1),
    ("default", 32, 8, 5, 1, 2),
    ("default", 64, 8, 4, 36, 3),
    ("default", 8, 1, 9, 0, 4),
    ("default", 4, 4, 0, 37, 0),
    ("fast", 4, 4, 2, 0, 0),
    ("fast", 4, 2, 2, 37, 1),
    ("fast", 32, 8, 6, 63, 2),
    ("fast", 64, 8, 3, 0, 1),
    ("deep2", 4, 2, 3, 5, 1),
    ("l1_8bit", 4, 2, 2, 17, 0),
    ("odd_split", 8, 4, 3, 9, 2),
    ("int8_default_angles", 4, 2, 2, 0, 1),
    ("default", 40, 2, 2, 11, 1),  # GQA 20 > 16: two head blocks
    ("default", 6, 2, 3, 5, 1),  # GQA 3: 3 live head rows in the fold; combine: 96 live items of 128, 4 split groups
    ("default", 12, 2, 4, 0, 1),  # GQA 6: combine items in 192 of 256 slots, 2 split groups
    ("default", 24, 2, 3, 9, 1),  # GQA 12: 384 combine items, 1 split group
    ("default", 2, 2, 600, 3, 1),  # 600 splits of one head: two-tier combine, 38 groups
    ("default", 32, 8, 21, 5, 8),  # 8-page splits, one tier: 4-wave workgroups, two pages per wave, ragged last split
    ("fast", 16, 4, 13, 0, 6),  # 6-page splits, one tier, 4 waves: waves with one and two pages
    ("default", 64, 8, 10, 37, 5),  # GQA 8, 5-page splits on 4 waves, a dense tail
    # exactly 16 splits on 4 waves: the kernel instance whose combine takes one straight batch of 16
    ("default", 32, 8, 16, 37, 1),
    ("fast", 16, 4, 16, 0, 1),
    ("default", 64, 8, 16, 5, 1),  # 8 heads on 4 waves: the same instance's batch loop, two heads per wave
    # exactly 32 splits: one straight batch of 32 records per head, on 4 waves and on 8
    ("default", 32, 8, 32, 11, 1),
    ("default", 8, 2, 288, 3, 9),
    ("fast", 8, 2, 288, 0, 9),
]


@pytest.mark.parametrize("layout_name,hq,hkv,S,tail,pps", CASES)
def test_decode_attention_parity(device, layout_name, hq, hkv, S, tail, pps):
    print(f"[attn] layout={layout_name} hq={hq} hkv={hkv} S={S} tail={tail} pps={pps}", flush=True)
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS[layout_name], hq, hkv, S, tail, seed=S * 7 + tail)
    seq = S * PAGE + tail
    out = run_gpu(device, block, qv, tk, tv, q, seq, pps)
    check(out, oracle_out(host, tk, tv, q, seq), layout_name)


BATCHED = [
    # B, layout, hq, hkv, S pages, tail tokens, pages_per_split, tokens masked at the end
    (2, "default", 40, 2, 3, 11, 1, 0),  # GQA 20: two head blocks per kv head, one-page splits
    (3, "default", 8, 2, 4, 37, 0, 0),
    (2, "default", 8, 2, 5, 20, 2, 70),  # masked suffix reaching into the last page
    (3, "default", 32, 8, 3, 0, 1, 0),
    (2, "fast", 16, 4, 3, 5, 1, 0),
    (2, "default", 4, 2, 0, 37, 0, 0),  # dense tail only
    (2, "default", 8, 2, 16, 20, 1, 100),  # 16 splits, the tail and part of the last page masked: a record of m = -inf
    (2, "default", 8, 2, 32, 0, 1, 70),  # 32 splits (one straight batch), a masked suffix into the last page
]


@pytest.mark.parametrize("B,layout_name,hq,hkv,S,tail,pps,drop", BATCHED)
def test_decode_attention_batched(device, B, layout_name, hq, hkv, S, tail, pps, drop):
    """Batch > 1: row b of q and out, page slots b * H_kv + kv of the store and
    tail rows b * H_kv + kv, checked against the oracle per batch row."""
    print(f"[attn-batch] B={B} layout={layout_name} hq={hq} hkv={hkv} S={S} tail={tail} pps={pps} drop={drop}",
          flush=True)
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS[layout_name], hq, hkv, S, tail, seed=60 + B + S, B=B)
    seq = S * PAGE + tail - drop
    out = run_gpu(device, block, qv, tk, tv, q, seq, pps)
    assert out.shape == (B, hq, 128)
    check(out, oracle_out(host, tk, tv, q, seq), f"batched B={B}")
    # every batch row differs, so a batch-index mix-up cannot pass by symmetry
    assert max_abs(out[0], out[1]) > 1e-2


@pytest.mark.parametrize("B,S,tail,pps,drop", [(1, 3, 37, 1, 0), (2, 2, 63, 0, 0), (2, 4, 1, 2, 0),
                                                (1, 2, 37, 1, 5), (3, 0, 20, 0, 0)])
def test_decode_attention_tail_rows_past_len(device, B, S, tail, pps, drop):
    """The dense tail as views into 64-row buffers (the runtime's tail
    layout: T valid rows per (b, kv) plane, planes 64 rows apart) whose rows
    past T hold NaN: the kernel reads the T rows only (its loads are bounded
    to them), so the output matches the oracle and stays finite; with drop > 0
    the last tail tokens are masked by actual_seq_len as well."""
    print(f"[attn-tailrows] B={B} S={S} tail={tail} pps={pps} drop={drop}", flush=True)
    hq, hkv = 8, 2
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS["default"], hq, hkv, S, tail, seed=90 + S + tail, B=B)
    seq = S * PAGE + tail - drop
    full_k = torch.full((B, hkv, PAGE, 128), float("nan"), dtype=torch.float16, device=device)
    full_v = torch.full_like(full_k, float("nan"))
    full_k[:, :, :tail] = torch.from_numpy(tk).to(device)
    full_v[:, :, :tail] = torch.from_numpy(tv).to(device)
    tk_view, tv_view = full_k[:, :, :tail], full_v[:, :, :tail]
    assert tk_view.stride(1) == PAGE * 128  # the views are passed as they are, not copied
    pages = PageSet(block, qv) if block is not None else None
    out = kernels.decode_attention(torch.from_numpy(q).to(device), pages, tk_view, tv_view, seq, SCALE16,
                                   pages_per_split=pps)
    torch.cuda.synchronize()
    check(out.float().cpu().numpy(), oracle_out(host, tk, tv, q, seq), f"tail rows past len B={B}")


@pytest.mark.parametrize("B,layout_name,hq,hkv,S", [(2, "default", 40, 2, 5), (3, "fast", 8, 2, 3)])
def test_fused_qk_batched(device, B, layout_name, hq, hkv, S):
    print(f"[qk-batch] B={B} layout={layout_name} hq={hq} hkv={hkv} S={S}", flush=True)
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS[layout_name], hq, hkv, S, 0, seed=70 + B, B=B)
    scores = kernels.fused_qk(torch.from_numpy(q).to(device), PageSet(block, None), SCALE16)
    torch.cuda.synchronize()
    got = scores.float().cpu().numpy()
    blk = {k: host[k] for k in ("radii", "radii_scales", "angle_codes_l1", "angle_codes_deep", "metadata")}
    if blk["radii_scales"] is not None:
        blk["radii_scales"] = blk["radii_scales"].reshape(blk["radii"].shape[:3] + (1, 1))
    ref = oracle.cpu_fused_qk(q, blk, SCALE16)
    assert got.shape == ref.shape == (B, hq, S * PAGE)
    assert max_abs(got, ref) <= 1e-2, max_abs(got, ref)
    assert cosine(got, ref) >= 0.999


@pytest.mark.parametrize("drop", [1, 5, 64, 100])
def test_decode_attention_masked_suffix(device, drop):
    """actual_seq_len below the stored tokens masks the suffix (metal.py:318-319)."""
    print(f"[attn-mask] drop={drop}", flush=True)
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS["default"], 8, 2, 4, 20, seed=4)
    seq = 4 * PAGE + 20 - drop
    for pps in (0, 1):
        out = run_gpu(device, block, qv, tk, tv, q, seq, pps)
        check(out, oracle_out(host, tk, tv, q, seq), f"drop={drop} pps={pps}")


def test_seq_len_beyond_stored_tokens(device):
    """actual_seq_len past the stored tokens attends every stored token, as the
    reference's mask (global index >= actual_seq_len) does
    (tqpolar_online_attention.metal:474; metal.py:318)."""
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS["default"], 8, 2, 3, 9, seed=8)
    total = 3 * PAGE + 9
    ref = oracle_out(host, tk, tv, q, total)
    for seq in (total + 1, total + 1000, 1 << 40):
        check(run_gpu(device, block, qv, tk, tv, q, seq), ref, f"seq={seq}")


@pytest.mark.parametrize("layout_name,hq,hkv,S", [
    ("default", 8, 2, 3), ("fast", 8, 2, 3), ("deep2", 8, 2, 3), ("odd_split", 8, 2, 3),
    ("default", 40, 2, 5),  # two head blocks; the second workgroup has one live wave
    ("fast", 32, 8, 9),
])
def test_fused_qk_parity(device, layout_name, hq, hkv, S):
    print(f"[qk] layout={layout_name} hq={hq} hkv={hkv} S={S}", flush=True)
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS[layout_name], hq, hkv, S, 0, seed=9)
    scores = kernels.fused_qk(torch.from_numpy(q).to(device), PageSet(block, None), SCALE16)
    torch.cuda.synchronize()
    got = scores.float().cpu().numpy()
    blk = {k: host[k] for k in ("radii", "radii_scales", "angle_codes_l1", "angle_codes_deep", "metadata")}
    if blk["radii_scales"] is not None:
        blk["radii_scales"] = blk["radii_scales"].reshape(blk["radii"].shape[:3] + (1, 1))
    ref = oracle.cpu_fused_qk(q, blk, SCALE16)
    assert got.shape == ref.shape
    assert max_abs(got, ref) <= 1e-2, max_abs(got, ref)
    assert cosine(got, ref) >= 0.999


@pytest.mark.parametrize("layout_name,kind,qscale", [
    ("default", "outlier", 1.0 / np.sqrt(128.0)),
    ("fast", "outlier", 1.0 / np.sqrt(128.0)),
    ("default", "normal", 1.0),
])
def test_north_star_shape_32k(device, layout_name, kind, qscale):
    """Llama-3-8B shape (32 q / 8 kv heads) at 32768 tokens, default split."""
    print(f"[attn-32k] layout={layout_name} kind={kind}", flush=True)
    S = 512
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS[layout_name], 32, 8, S, 0, seed=3, kind=kind, qscale=qscale)
    out = run_gpu(device, block, qv, tk, tv, q, S * PAGE)
    check(out, oracle_out(host, tk, tv, q, S * PAGE), "32k")


def test_config1_shape(device):
    """Llama-3.2-1B shape (32 q / 8 kv heads), 4096 tokens =
    64 pages, K, V and q ~ N(0,1) from seed 0, every token visible."""
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS["default"], 32, 8, 64, 0, seed=0)
    out = run_gpu(device, block, qv, tk, tv, q, 64 * PAGE)
    check(out, oracle_out(host, tk, tv, q, 64 * PAGE), "config 1")


@pytest.mark.parametrize("layout_name", ["default", "fast"])
def test_nonfinite_radii_propagate_like_reference(device, layout_name):
    """Config 5's K (Student-t(3) x per-channel scales up to 10) overflows the
    fp16 x*x of some pairs, so those radii are +inf (fast layout: the page
    scale is inf and the page's codes decode to NaN).  The reference's CPU
    path then gives NaN for every query head whose scores meet +inf or NaN and
    a finite output where the inf radii only produce -inf scores.  The kernel
    must reproduce exactly which outputs are NaN or +-inf, and the finite ones
    within tolerance, with and without the split-K combine."""
    hq, hkv, S, tail = 64, 8, 8, 5
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS[layout_name], hq, hkv, S, tail, seed=2,
                                            kind="studentt", qscale=1.0 / np.sqrt(128.0))
    seq = S * PAGE + tail
    rad = host["radii"] if layout_name == "default" else host["radii_scales"].reshape(1, hkv, S)
    hit = [h for h in range(hkv) if not np.all(np.isfinite(rad[0, h].astype(np.float32)))]
    assert hit and len(hit) < hkv, f"case must mix affected and clean kv heads, got {hit}"
    ref = oracle_out(host, tk, tv, q, seq)
    for pps in (0, 1):
        out = run_gpu(device, block, qv, tk, tv, q, seq, pps=pps)
        nan_heads = sorted({int(h) for h in np.nonzero(np.isnan(ref))[1]})
        print(f"[attn-nonfinite] {layout_name} pps={pps} kv heads with inf radii {hit}, "
              f"NaN query heads {nan_heads}", flush=True)
        assert np.array_equal(np.isnan(out), np.isnan(ref)), "NaN positions differ"
        assert np.array_equal(np.isposinf(out), np.isposinf(ref)), "+inf positions differ"
        assert np.array_equal(np.isneginf(out), np.isneginf(ref)), "-inf positions differ"
        fin = np.isfinite(ref)
        assert fin.any() and (~fin).any()
        check(out[fin], ref[fin], f"{layout_name} finite outputs")


@pytest.mark.parametrize("pps", [0, 1])
def test_page_of_minus_inf_scores_weighs_zero(device, pps):
    """Every token of page 1 of kv head 0 has pair 0 = (-300, 0): its radius
    overflows to +inf and its angle decodes to pi, so K-hat starts (-inf,
    -inf) and query heads with q0, q1 > 0 score -inf on the whole page.  The
    reference's softmax gives those tokens weight 0 and a finite output from
    the other pages; a page whose every score is -inf must not turn the
    running state into NaN."""
    from turbopolar_amd.payload import PolarKeyBlock, QuantizedVBlock

    hq, hkv, S, tail = 8, 2, 4, 0
    k, v = gen_kv(77, 1, hkv, S * PAGE, "normal", np.float16)
    k[0, 0, PAGE:2 * PAGE, 0] = -300.0
    k[0, 0, PAGE:2 * PAGE, 1] = 0.0
    q = gen_q(77, 1, hq)
    q[0, :2, 0:2] = np.float16(0.5)  # heads 0, 1: q0, q1 > 0 -> -inf scores on page 1
    q[0, 2, 0], q[0, 2, 1] = np.float16(0.5), np.float16(-0.5)  # head 2: -inf + inf -> NaN scores
    layout = LAYOUTS["default"]
    host = encode_gpu(k, v, layout, device)
    meta = oracle.encode_block(k[:, :, :PAGE], l1_bits=layout[1], deep_bits=layout[2], split_dim=layout[3],
                               use_int8_radii=layout[0])["metadata"]
    host["metadata"] = meta
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    block = PolarKeyBlock(radii=t(host["radii"]), angle_codes_l1=t(host["angle_codes_l1"]),
                          angle_codes_deep=t(host["angle_codes_deep"]), shape=(1, hkv, S * PAGE, 128),
                          block_size=PAGE, head_dim=128, metadata=meta, radii_scales=None)
    qv = QuantizedVBlock(codes=t(host["v_codes"]), scales=t(host["v_scales"]), group_size=32)
    empty = np.zeros((1, hkv, 0, 128), np.float16)
    ref = oracle_out(host, empty, empty, q, S * PAGE)
    assert np.all(np.isfinite(ref[0, :2])) and np.all(np.isnan(ref[0, 2])), "case does not exercise -inf / NaN"
    out = run_gpu(device, block, qv, empty, empty, q, S * PAGE, pps=pps)
    assert np.array_equal(np.isnan(out), np.isnan(ref)) and np.array_equal(np.isinf(out), np.isinf(ref))
    fin = np.isfinite(ref)
    check(out[fin], ref[fin], "-inf page")


def test_split_invariance(device):
    """Split-K online softmax equals the one-pass result for every split size."""
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS["default"], 32, 8, 40, 13, seed=12)
    seq = 40 * PAGE + 13
    outs = [run_gpu(device, block, qv, tk, tv, q, seq, pps) for pps in (1, 2, 3, 8, 40)]
    for o in outs[1:]:
        assert max_abs(o, outs[0]) <= 1e-3
    check(outs[0], oracle_out(host, tk, tv, q, seq), "split")


def test_max_splits_combine(device):
    """1536 one-page splits of 4 heads: two-tier combine of 96 groups of 16
    (the last combine folds 96 group records)."""
    print("[attn-maxsplits] S=1536 pps=1", flush=True)
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS["default"], 8, 2, 1536, 9, seed=21)
    seq = 1536 * PAGE + 9
    out = run_gpu(device, block, qv, tk, tv, q, seq, pps=1)
    check(out, oracle_out(host, tk, tv, q, seq), "max splits")


TIERED = [
    # layout, hq, hkv, S pages, tail, pages_per_split, B, tokens masked at the end
    ("default", 4, 1, 65, 0, 1, 1, 0),  # 5 groups of 16, 16, 16, 16, 1 splits
    ("default", 4, 1, 256, 0, 1, 1, 0),  # 16 full groups
    ("default", 8, 1, 300, 37, 1, 1, 0),  # 19 groups, the last of 12, with a tail
    ("default", 16, 2, 97, 5, 1, 2, 0),  # batch 2, GQA 8: 4 units of 7 groups
    ("default", 8, 1, 130, 11, 1, 1, 200),  # masked suffix: the last group (splits 128, 129) holds no live token
    ("fast", 32, 8, 80, 0, 1, 1, 0),  # 8 units of 5 groups
    ("default", 24, 2, 70, 9, 1, 1, 0),  # GQA 12: 384 combine items per group record
    ("default", 4, 1, 530, 9, 8, 1, 0),  # 8-page splits, 67 of them: 4-wave workgroups, two pages per wave
    ("fast", 8, 2, 600, 0, 6, 1, 0),  # 6-page splits, 100 per unit: 4-wave workgroups, ragged waves
]


@pytest.mark.parametrize("layout_name,hq,hkv,S,tail,pps,B,drop", TIERED)
def test_two_tier_combine(device, layout_name, hq, hkv, S, tail, pps, B, drop):
    """More than 64 splits per (b, kv head, head block): groups of 16 splits
    combine into group records, and the last group combines the groups."""
    print(f"[attn-tiers] layout={layout_name} hq={hq} hkv={hkv} S={S} tail={tail} pps={pps} B={B} drop={drop}",
          flush=True)
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS[layout_name], hq, hkv, S, tail, seed=90 + S, B=B)
    seq = S * PAGE + tail - drop
    out = run_gpu(device, block, qv, tk, tv, q, seq, pps)
    check(out, oracle_out(host, tk, tv, q, seq), f"tiers S={S}")


COMBINE_MAPS = [
    # hq, hkv, S pages, pages_per_split: the combine's items are (head, 8-dim
    # chunk) = GQA x 16 per head block, padded to 32 / 64 / 128 / 256 slots,
    # and the rest of the threads form 2-16 split groups; splits of <= 8 pages
    # at GQA <= 8 run on 4-wave workgroups (256 threads), longer ones on 8.
    (1, 1, 23, 2), (2, 1, 23, 9),  # GQA 1 / 2: 16 / 32 items in 32 slots, 8 / 16 split groups
    (3, 1, 19, 3), (3, 1, 19, 10),  # GQA 3: 48 items in 64 slots
    (5, 1, 33, 4), (7, 1, 33, 11),  # GQA 5 / 7: 80 / 112 items in 128 slots
    (8, 1, 40, 5), (8, 1, 40, 12),  # GQA 8: 128 items, 2 / 4 split groups
    (9, 1, 21, 2), (12, 1, 21, 1),  # GQA 9 / 12 (8 waves): 144 / 192 items in 256 slots, 2 split groups
    (16, 1, 17, 1), (16, 2, 30, 13),  # GQA 16: 256 items, 2 split groups; 3 splits per unit
]


@pytest.mark.parametrize("hq,hkv,S,pps", COMBINE_MAPS)
def test_combine_item_maps(device, hq, hkv, S, pps):
    """Every mapping of the split combine (items per head block, slot
    padding, split groups on 4- and 8-wave workgroups) against the oracle,
    with record counts that leave the split groups ragged and a dense tail."""
    print(f"[attn-combine] hq={hq} hkv={hkv} S={S} pps={pps}", flush=True)
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS["default"], hq, hkv, S, 11, seed=200 + hq + S)
    seq = S * PAGE + 11
    out = run_gpu(device, block, qv, tk, tv, q, seq, pps)
    check(out, oracle_out(host, tk, tv, q, seq), f"combine map hq={hq} hkv={hkv} pps={pps}")


def test_two_tier_launches_repeat_exactly(device):
    """200 launches alternating a two-tier and a one-tier shape on one
    workspace: every output is bit-identical to that shape's first output, so
    the group tickets, the group records and both counter resets are
    race-free."""
    cases = []
    for hq, hkv, S, seed in ((8, 1, 100, 3), (32, 8, 24, 4)):
        block, qv, host, tk, tv, q = build_case(device, LAYOUTS["default"], hq, hkv, S, 7, seed=seed)
        cases.append((PageSet(block, qv), torch.from_numpy(q).to(device), torch.from_numpy(tk).to(device),
                      torch.from_numpy(tv).to(device), S * PAGE + 7, host, tk, tv, q))
    refs = [kernels.decode_attention(c[1], c[0], c[2], c[3], c[4], SCALE16, pages_per_split=1).clone()
            for c in cases]
    torch.cuda.synchronize()
    for i, c in enumerate(cases):
        check(refs[i].float().cpu().numpy(), oracle_out(c[5], c[6], c[7], c[8], c[4]), f"case {i}")
    bad = torch.zeros((), dtype=torch.int64, device=device)
    for it in range(200):
        c = cases[it % 2]
        out = kernels.decode_attention(c[1], c[0], c[2], c[3], c[4], SCALE16, pages_per_split=1)
        bad += (out != refs[it % 2]).sum()
    torch.cuda.synchronize()
    assert int(bad.item()) == 0


def test_workspace_shared_across_shapes(device):
    """One workspace serves calls whose unit counts (batch x kv heads x head
    blocks) rise and fall: every call's records land after the fixed counter
    area, so no call finds an earlier call's records where its counters are."""
    for i, (hq, hkv, S, tail, pps) in enumerate([(4, 2, 5, 3, 1), (32, 8, 5, 1, 2), (8, 1, 6, 0, 1),
                                                 (64, 8, 4, 9, 1), (4, 1, 70, 5, 1), (4, 2, 7, 0, 2),
                                                 (32, 8, 3, 0, 1)]):
        print(f"[attn-shared-ws] hq={hq} hkv={hkv} S={S} tail={tail} pps={pps}", flush=True)
        block, qv, host, tk, tv, q = build_case(device, LAYOUTS["default"], hq, hkv, S, tail, seed=40 + i)
        seq = S * PAGE + tail
        out = run_gpu(device, block, qv, tk, tv, q, seq, pps=pps)
        check(out, oracle_out(host, tk, tv, q, seq), f"shape {i}")


def test_graph_replay_matches_eager(device):
    """Three decode launches (6 one-page splits each, so the combine and the
    ticket reset run inside the graph) captured into one HIP graph: each of
    three replays, with eager launches and syncs between them, reproduces the
    eager outputs bit for bit, and the eager outputs match the oracle."""
    from turbopolar_amd import _lib

    L = _lib.lib()
    cases = []
    for seed in (50, 51, 52):
        block, qv, host, tk, tv, q = build_case(device, LAYOUTS["default"], 32, 8, 6, 0, seed=seed)
        cases.append((PageSet(block, qv), torch.from_numpy(q).to(device),
                      torch.empty((1, 32, 128), dtype=torch.float16, device=device), host, tk, tv, q))
    seq = 6 * PAGE
    need = int(L.tp_decode_workspace_bytes(1, 32, 8, 6, 0, 1))
    ws = torch.zeros(need, dtype=torch.uint8, device=device)

    def step():
        stream = torch.cuda.current_stream(device).cuda_stream
        for ps, qt, out, *_ in cases:
            st = L.tp_decode_attention(qt.data_ptr(), 1, 32, 8, ctypes.byref(ps.layout), ctypes.byref(ps.pages), 6,
                                       None, None, 0, 0, seq, SCALE16, 1, ws.data_ptr(), need, out.data_ptr(), stream)
            assert st == 0, L.tp_last_error()

    step()
    torch.cuda.synchronize()
    eager = [c[2].clone() for c in cases]
    for (ps, qt, out, host, tk, tv, q), e in zip(cases, eager):
        check(e.float().cpu().numpy(), oracle_out(host, tk, tv, q, seq), "graph eager")
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for rep in range(3):
        for c in cases:
            c[2].fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        for c, e in zip(cases, eager):
            assert torch.equal(c[2], e), f"replay {rep} differs from eager"
        step()
        torch.cuda.synchronize()
        for c, e in zip(cases, eager):
            assert torch.equal(c[2], e), f"eager launch after replay {rep} differs"


def test_page_decode_parity(device):
    """tp_decode_pages: V exactly the dequantised codes; K within one fp16 ulp."""
    # 9 pages: the specialised default and fast kernels decode 4 pages per
    # workgroup, so this covers full and partial groups.
    for name in ("default", "fast", "deep2", "odd_split"):
        block, qv, host, tk, tv, q = build_case(device, LAYOUTS[name], 4, 2, 9, 0, seed=2)
        kg, vg = kernels.decode_pages(PageSet(block, qv))
        torch.cuda.synchronize()
        blk = {k: host[k] for k in ("radii", "radii_scales", "angle_codes_l1", "angle_codes_deep", "metadata")}
        rs = None if blk["radii_scales"] is None else blk["radii_scales"].reshape(blk["radii"].shape[:3] + (1, 1))
        kref = oracle.decode_block(blk["radii"], rs, blk["angle_codes_l1"], blk["angle_codes_deep"], blk["metadata"])
        vref = oracle.dequantize_block(host["v_codes"], host["v_scales"]).reshape(kref.shape)
        assert np.array_equal(vg.cpu().numpy().view(np.uint16), vref.view(np.uint16)), name
        kd = kg.cpu().numpy().astype(np.float64)
        ulp = np.spacing(np.abs(kref).astype(np.float16)).astype(np.float64)
        assert np.all(np.abs(kd - kref) <= ulp + 1e-12), name


def test_repeated_launches_share_workspace(device):
    """300 back-to-back launches alternating two caches on one workspace, with
    many splits: every output is bit-identical to that cache's first output, so
    the cross-workgroup exchange and the ticket reset are race-free."""
    cases = []
    for seed in (1, 2):
        block, qv, host, tk, tv, q = build_case(device, LAYOUTS["default"], 32, 8, 48, 5, seed=seed)
        cases.append((PageSet(block, qv), torch.from_numpy(q).to(device), torch.from_numpy(tk).to(device),
                      torch.from_numpy(tv).to(device), host, tk, tv, q))
    seq = 48 * PAGE + 5
    refs = [kernels.decode_attention(c[1], c[0], c[2], c[3], seq, SCALE16, pages_per_split=1).clone() for c in cases]
    torch.cuda.synchronize()
    for i, c in enumerate(cases):
        check(refs[i].float().cpu().numpy(), oracle_out(c[4], c[5], c[6], c[7], seq), f"case {i}")
    bad = torch.zeros((), dtype=torch.int64, device=device)
    for it in range(300):
        c = cases[it % 2]
        out = kernels.decode_attention(c[1], c[0], c[2], c[3], seq, SCALE16, pages_per_split=1 + (it % 3))
        bad += (out != refs[it % 2]).sum() if it % 3 == 0 else (torch.abs(out.float() - refs[it % 2].float()) > 1e-3).sum()
    torch.cuda.synchronize()
    assert int(bad.item()) == 0
