"""Compressed K with dense fp16 V on the GPU against the oracle (row a11/b:
the reference's execute_online_attention_dense_v, rfsn_v11/kernels/
turbo_polar/metal.py:586-649, kernel tqpolar_online_attention_dense_v, and its
CPU path metal.py:596-601 -> _cpu_online_attention :267-291).

tp_decode_attention_dense_v runs the decode kernel with V rows read from a
dense ``[B, H_kv, S_cap, 64, 128]`` fp16 array in place of the quantised V
pages.  Bar: max-abs 2e-3 and relative L2 1e-3 against
oracle.cpu_online_attention_dense_v in float64, over layouts, GQA groups,
split sizes (one- and two-tier combines, 4- and 8-wave workgroups), masked
suffixes, batches, a V capacity larger than the key block, and QJL.
"""

import numpy as np
import pytest
import torch

import oracle
from common import ATOL, LAYOUTS, PAGE, RTOL_L2, gen_kv, max_abs, rel_l2
from test_gpu_attention import SCALE16, build_case
from test_gpu_qjl import _qjl_case, _cfg
from turbopolar_amd import kernels
from turbopolar_amd.bridge import HipKernelBridge
from turbopolar_amd.kernels import PageSet
from turbopolar_amd.qjl import QJLPages

pytestmark = pytest.mark.gpu


def _blk(host):
    blk = {k: host[k] for k in ("radii", "radii_scales", "angle_codes_l1", "angle_codes_deep", "metadata")}
    if blk["radii_scales"] is not None:
        blk["radii_scales"] = blk["radii_scales"].reshape(blk["radii"].shape[:3] + (1, 1))
    return blk


def _dense_v(seed, B, hkv, S, cap):
    """Dense V pages [B, hkv, cap, 64, 128]: the first S pages are the case's
    V rows, the rest a different pattern that must never be read."""
    _, v = gen_kv(seed, B, hkv, S * PAGE, "normal", np.float16)
    vd = np.full((B, hkv, cap, PAGE, 128), 7.0, np.float16)
    vd[:, :, :S] = v.reshape(B, hkv, S, PAGE, 128)
    return vd


def _check(out, ref, what):
    assert np.all(np.isfinite(out)), f"{what}: non-finite output"
    ma, rl = max_abs(out, ref), rel_l2(out, ref)
    assert ma <= ATOL and rl <= RTOL_L2, f"{what}: max_abs={ma:.3g} rel_l2={rl:.3g}"


CASES = [
    # layout, hq, hkv, S, pps, masked, B, cap_extra, four_d
    ("default", 32, 8, 5, 2, 0, 1, 0, False),
    ("fast", 32, 8, 4, 1, 0, 1, 2, False),
    ("default", 8, 2, 7, 3, 21, 2, 0, True),
    ("fast", 4, 4, 3, 0, 63, 1, 0, False),
    ("deep2", 64, 8, 2, 0, 0, 1, 0, False),
    ("l1_8bit", 12, 3, 6, 4, 5, 1, 1, False),
    ("odd_split", 16, 2, 9, 0, 0, 2, 0, True),
    ("int8_default_angles", 8, 8, 1, 0, 63, 1, 0, False),
    ("default", 8, 1, 70, 1, 0, 1, 0, False),   # 70 splits: two-tier combine
    ("fast", 32, 8, 17, 6, 0, 1, 0, False),     # 6-page splits, 4-wave workgroups
    ("default", 16, 2, 16, 8, 0, 2, 3, False),  # 8-page splits, batch 2, larger V capacity
    ("default", 40, 8, 12, 0, 17, 1, 0, True),  # g = 5
    ("default", 40, 2, 3, 1, 5, 1, 1, False),   # g = 20: two head blocks, the row token order
]


@pytest.mark.parametrize("layout_name,hq,hkv,S,pps,masked,B,cap_extra,four_d", CASES)
def test_dense_v_matches_oracle(device, layout_name, hq, hkv, S, pps, masked, B, cap_extra, four_d):
    print(f"[dense_v] {layout_name} hq={hq} hkv={hkv} S={S} pps={pps} masked={masked} B={B} "
          f"cap+{cap_extra} 4d={four_d}", flush=True)
    seed = 31 + S
    block, _, host, _, _, q = build_case(device, LAYOUTS[layout_name], hq, hkv, S, 0, seed=seed, B=B)
    vd = _dense_v(seed + 1, B, hkv, S, S + cap_extra)
    vt = torch.from_numpy(vd).to(device)
    if four_d:
        vt = vt.reshape(B, hkv, (S + cap_extra) * PAGE, 128)
    seq = S * PAGE - masked
    out = kernels.decode_attention_dense_v(torch.from_numpy(q).to(device), PageSet(block, None), vt, seq,
                                           SCALE16, pages_per_split=pps)
    torch.cuda.synchronize()
    ref = oracle.cpu_online_attention_dense_v(q, _blk(host), vd[:, :, :S], SCALE16, seq)
    _check(out.float().cpu().numpy(), ref, "dense_v")


@pytest.mark.parametrize("pps", [0, 1, 2])
def test_dense_v_nonfinite_masked_rows_add_nothing(device, pps):
    """Rows of masked tokens on the last live page and the page slots past the
    key block hold NaN and inf: the output equals the oracle's over the valid
    rows (masked tokens weigh 0 and their V rows add nothing, as the
    reference's kernel skips them)."""
    S, masked = 5, 23
    block, _, host, _, _, q = build_case(device, LAYOUTS["default"], 32, 8, S, 0, seed=44)
    vd = _dense_v(45, 1, 8, S, S + 2)
    ref = oracle.cpu_online_attention_dense_v(q, _blk(host), vd[:, :, :S], SCALE16, S * PAGE - masked)
    vd[:, :, S - 1, PAGE - masked:PAGE - masked + 11] = np.nan
    vd[:, :, S - 1, PAGE - masked + 11:] = np.inf
    vd[:, :, S:] = np.nan
    out = kernels.decode_attention_dense_v(torch.from_numpy(q).to(device), PageSet(block, None),
                                           torch.from_numpy(vd).to(device), S * PAGE - masked, SCALE16,
                                           pages_per_split=pps)
    torch.cuda.synchronize()
    _check(out.float().cpu().numpy(), ref, "dense_v with non-finite masked rows")


def test_dense_v_reads_dense_rows_not_quantised_pages(device):
    """The same key block with its quantised V and with dense V: the dense
    result follows the dense oracle, which differs from the quantised one."""
    block, qv, host, _, _, q = build_case(device, LAYOUTS["default"], 8, 2, 3, 0, seed=5)
    vd = _dense_v(5, 1, 2, 3, 3)
    qd = torch.from_numpy(q).to(device)
    dense = kernels.decode_attention_dense_v(qd, PageSet(block, qv), torch.from_numpy(vd).to(device), 3 * PAGE,
                                             SCALE16).float().cpu().numpy()
    quant = kernels.decode_attention(qd, PageSet(block, qv), None, None, 3 * PAGE, SCALE16).float().cpu().numpy()
    ref = oracle.cpu_online_attention_dense_v(q, _blk(host), vd, SCALE16, 3 * PAGE)
    _check(dense, ref, "dense")
    assert max_abs(dense, quant) > 1e-3


def test_dense_v_split_invariance(device):
    block, _, host, _, _, q = build_case(device, LAYOUTS["fast"], 32, 8, 24, 0, seed=8)
    vt = torch.from_numpy(_dense_v(9, 1, 8, 24, 24)).to(device)
    qd = torch.from_numpy(q).to(device)
    outs = [kernels.decode_attention_dense_v(qd, PageSet(block, None), vt, 24 * PAGE - 3, SCALE16,
                                             pages_per_split=p).float() for p in (1, 2, 3, 8, 24)]
    for o in outs[1:]:
        assert float((o - outs[0]).abs().max()) <= 1e-3


def test_dense_v_shape_errors(device):
    block, _, _, _, _, q = build_case(device, LAYOUTS["default"], 8, 2, 3, 0, seed=6)
    qd = torch.from_numpy(q).to(device)
    pages = PageSet(block, None)
    bad = [torch.zeros((1, 2, 2, PAGE, 128), dtype=torch.float16, device=device),   # fewer pages than K
           torch.zeros((1, 4, 3, PAGE, 128), dtype=torch.float16, device=device),   # wrong H_kv
           torch.zeros((1, 2, 3 * PAGE + 5, 128), dtype=torch.float16, device=device),  # not whole pages
           torch.zeros((2, 3 * PAGE, 128), dtype=torch.float16, device=device)]     # 3-D
    for v in bad:
        with pytest.raises(ValueError):
            kernels.decode_attention_dense_v(qd, pages, v, 3 * PAGE, SCALE16)


@pytest.mark.parametrize("layout_name,hq,hkv,S,pps,masked,B", [
    ("default", 32, 8, 5, 2, 0, 1),
    ("fast", 64, 8, 4, 1, 9, 1),
    ("default", 8, 2, 7, 3, 21, 2),
    ("default", 8, 1, 70, 1, 0, 1),   # two-tier combine
    ("fast", 32, 8, 17, 6, 0, 1),     # 4-wave workgroups
    ("default", 24, 2, 4, 1, 7, 1),   # GQA 12: the row token order
])
def test_dense_v_qjl_matches_oracle(device, layout_name, hq, hkv, S, pps, masked, B):
    print(f"[dense_v qjl] {layout_name} hq={hq} hkv={hkv} S={S} pps={pps} masked={masked} B={B}", flush=True)
    block, _, host, _, _, q, qd, pay, qs, tup = _qjl_case(device, layout_name, hq, hkv, S, 0, 41 + S, B=B)
    vd = _dense_v(43 + S, B, hkv, S, S)
    seq = S * PAGE - masked
    out = kernels.decode_attention_dense_v(qd, PageSet(block, None), torch.from_numpy(vd).to(device), seq,
                                           SCALE16, pages_per_split=pps, qjl=QJLPages(pay, qs))
    ref = oracle.cpu_online_attention_dense_v(q, _blk(host), vd, SCALE16, seq, qjl=tup)
    _check(out.float().cpu().numpy(), ref, "dense_v qjl")
    plain = oracle.cpu_online_attention_dense_v(q, _blk(host), vd, SCALE16, seq)
    assert max_abs(plain, ref) > 1e-5


@pytest.mark.parametrize("P", [16, 40])
def test_dense_v_qjl_any_width(device, P):
    """Dense V with QJL sketches of a width other than 64."""
    block, _, host, _, _, q, qd, pay, qs, tup = _qjl_case(device, "default", 32, 8, 5, 0, 47, P=P)
    vd = _dense_v(48, 1, 8, 5, 5)
    seq = 5 * PAGE - 9
    out = kernels.decode_attention_dense_v(qd, PageSet(block, None), torch.from_numpy(vd).to(device), seq,
                                           SCALE16, pages_per_split=2, qjl=QJLPages(pay, qs))
    ref = oracle.cpu_online_attention_dense_v(q, _blk(host), vd, SCALE16, seq, qjl=tup)
    _check(out.float().cpu().numpy(), ref, f"dense_v qjl P={P}")


def test_bridge_dense_v(device):
    block, _, host, _, _, q, qd, pay, qs, tup = _qjl_case(device, "default", 8, 2, 3, 0, 29)
    vt = torch.from_numpy(_dense_v(30, 1, 2, 3, 3)).to(device)
    bridge = HipKernelBridge()
    cfg = _cfg(8, 2)
    out, trace = bridge.execute_online_attention_dense_v(qd, block, vt, None, None, cfg, 3 * PAGE - 4)
    assert trace["kernel_name"] == "tqpolar_online_attention_dense_v"
    assert trace["hip_kernel"] == "tp_decode_attention_dense_v" and trace["hip_used"]
    assert not trace["fallback_used"] and not trace["quant_v_used"] and not trace["qjl_used"]
    assert trace["num_queries_per_kv"] == 4 and trace["actual_seq_len"] == 3 * PAGE - 4
    direct = kernels.decode_attention_dense_v(qd, PageSet(block, None), vt, 3 * PAGE - 4, SCALE16)
    assert torch.equal(out, direct)
    with pytest.raises(ValueError, match="qjl_payload and q_proj_signs are required"):
        bridge.execute_online_attention_dense_v(qd, block, vt, None, None, cfg, 3 * PAGE, use_qjl=True)
    out_q, trace_q = bridge.execute_online_attention_dense_v(qd, block, vt, pay, qs, cfg, 3 * PAGE, use_qjl=True)
    assert trace_q["qjl_used"]
    ref = oracle.cpu_online_attention_dense_v(q, _blk(host), vt.cpu().numpy(), SCALE16, 3 * PAGE, qjl=tup)
    _check(out_q.float().cpu().numpy(), ref, "bridge dense_v qjl")


def test_dense_v_seq_len_beyond_stored_tokens(device):
    """A length past the stored tokens attends every stored token, as the
    reference's mask (global index >= actual_seq_len) does."""
    block, _, host, _, _, q = build_case(device, LAYOUTS["default"], 8, 2, 2, 0, seed=12)
    vt = torch.from_numpy(_dense_v(13, 1, 2, 2, 2)).to(device)
    qd = torch.from_numpy(q).to(device)
    full = kernels.decode_attention_dense_v(qd, PageSet(block, None), vt, 2 * PAGE, SCALE16)
    longer = kernels.decode_attention_dense_v(qd, PageSet(block, None), vt, 2 * PAGE + 100, SCALE16)
    assert torch.equal(full, longer)


def test_dense_v_graph_replay_matches_eager(device):
    """Two dense-V launches (6 one-page splits each, so the combine and the
    ticket reset run inside the graph) captured into one HIP graph: each of
    three replays, with eager launches and syncs between them, reproduces the
    eager outputs bit for bit, and the eager outputs match the oracle."""
    cases = []
    for seed in (60, 61):
        block, _, host, _, _, q = build_case(device, LAYOUTS["fast"], 32, 8, 6, 0, seed=seed)
        vd = _dense_v(seed + 7, 1, 8, 6, 6)
        cases.append((PageSet(block, None), torch.from_numpy(q).to(device), torch.from_numpy(vd).to(device),
                      torch.empty((1, 32, 128), dtype=torch.float16, device=device), host, q, vd))
    seq = 6 * PAGE - 1

    def step():
        for ps, qt, vt, out, *_ in cases:
            kernels.decode_attention_dense_v(qt, ps, vt, seq, SCALE16, pages_per_split=1, out=out)

    step()
    torch.cuda.synchronize()
    eager = [c[3].clone() for c in cases]
    for (ps, qt, vt, out, host, q, vd), e in zip(cases, eager):
        _check(e.float().cpu().numpy(), oracle.cpu_online_attention_dense_v(q, _blk(host), vd, SCALE16, seq),
               "graph eager")
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    # Captured on the warmed-up side stream: the library's per-stream
    # workspace already exists, so nothing is allocated inside the capture.
    with torch.cuda.graph(graph, stream=side):
        step()
    for rep in range(3):
        for c in cases:
            c[3].fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        for c, e in zip(cases, eager):
            assert torch.equal(c[3], e), f"replay {rep} differs from eager"
        step()
        torch.cuda.synchronize()
        for c, e in zip(cases, eager):
            assert torch.equal(c[3], e), f"eager launch after replay {rep} differs"
