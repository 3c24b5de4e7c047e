"""QJL on the GPU against the oracle (row f4: rfsn_v11/quant/qjl/encoder.py:
19-44, score_estimate.py:6-54, kernels/turbo_polar/metal.py:262-316,
tqpolar_fused_qk.metal:102-233).

* Sketches (tp_qjl_sketch): every sign bit equals the oracle's float64
  projection sign except where that projection is within 1e-5 |e| of zero (a
  summation-order tie); residual norms within one fp16 ulp.
* The estimate (tp_qjl_dot_estimate), fused QK with QJL (tp_fused_qk_qjl) and
  decode attention with QJL (tp_decode_attention_qjl) take the GPU's
  sketches, so the oracle sees the same bits: estimate within 1e-5 relative,
  QK scores at the reference's QK bar (max-abs 1e-2, cosine 0.999), attention
  at the product bar (max-abs 2e-3, relative L2 1e-3).
"""

import numpy as np
import pytest
import torch

import oracle
from common import ATOL, LAYOUTS, PAGE, RTOL_L2, cosine, max_abs, rel_l2
from test_gpu_attention import SCALE16, build_case, oracle_out
from turbopolar_amd import TurboPolarConfig, kernels
from turbopolar_amd.bridge import HipKernelBridge
from turbopolar_amd.kernels import PageSet, decode_pages
from turbopolar_amd.qjl import QJLPages, QJLResidualEncoder, qjl_dot_estimate

pytestmark = pytest.mark.gpu


def _cfg(hq=4, hkv=2, P=64):
    return TurboPolarConfig(num_q_heads=hq, num_kv_heads=hkv, qjl_proj_dim=P)


def _fp16_ulp(x):
    x = np.abs(x.astype(np.float32))
    e = np.floor(np.log2(np.maximum(x, 2.0 ** -14)))
    return 2.0 ** (e - 10)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_sketch_matches_oracle(device, dtype):
    enc = QJLResidualEncoder(_cfg())
    g = torch.Generator(device=device).manual_seed(5)
    e = (torch.randn((2, 3, 4, 64, 128), generator=g, device=device) * 0.05).to(dtype)
    e[0, 0, 0, 0] = 0.0  # zero residual: every projection 0 >= 0, norm 0
    pay = enc.compute_residual_sketch(e)
    en = e.cpu().numpy()
    packed, norms = oracle.qjl_residual_sketch(en, enc.W_host)
    proj = en.astype(np.float64) @ enc.W_host.astype(np.float64)
    tie = np.abs(proj) <= 1e-5 * np.linalg.norm(en.astype(np.float64), axis=-1, keepdims=True) + 1e-30
    gb = np.unpackbits(pay.packed_signs.cpu().numpy(), axis=-1, bitorder="little")
    ob = np.unpackbits(packed, axis=-1, bitorder="little")
    assert np.all((gb == ob) | tie), f"{int(np.sum((gb != ob) & ~tie))} sign bits differ away from a tie"
    gn = pay.norms.cpu().numpy().astype(np.float32)
    on = norms.astype(np.float32)
    assert np.all(np.abs(gn - on) <= _fp16_ulp(on))
    assert pay.norms[0, 0, 0, 0].item() == 0.0 and int(pay.packed_signs[0, 0, 0, 0].sum()) == 8 * 255
    qs = enc.query_signs(e[:, :, 0, 0])
    assert torch.equal(qs, pay.packed_signs[:, :, 0, 0])


def _residual_payload(enc, block, k_full, S):
    """Residual of the encoded pages (k - decode(encode(k)), fp16 as the
    reference's _flush_block subtracts) and its sketch."""
    dense, _ = decode_pages(PageSet(block, None), want_k=True, want_v=False)
    B, H = dense.shape[:2]
    res = (k_full - dense).reshape(B, H, S, PAGE, 128)
    return enc.compute_residual_sketch(res)


def _qjl_case(device, layout_name, hq, hkv, S, tail, seed, B=1, P=64):
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS[layout_name], hq, hkv, S, tail, seed=seed, B=B)
    from common import gen_kv
    k, _ = gen_kv(seed, B, hkv, S * PAGE + tail, "normal", np.float16)
    enc = QJLResidualEncoder(_cfg(hq, hkv, P))
    pay = _residual_payload(enc, block, torch.from_numpy(k[:, :, :S * PAGE]).to(device), S)
    qd = torch.from_numpy(q).to(device)
    qs = enc.query_signs(qd)
    tup = (pay.packed_signs.cpu().numpy(), pay.norms.cpu().numpy(), qs.cpu().numpy(), P)
    return block, qv, host, tk, tv, q, qd, pay, qs, tup


def test_dot_estimate_matches_oracle(device):
    block, qv, host, tk, tv, q, qd, pay, qs, tup = _qjl_case(device, "default", 8, 2, 3, 0, 11)
    got = qjl_dot_estimate(qd, pay, qs).cpu().numpy()
    ref = oracle.qjl_dot_estimate(q, *tup)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())


@pytest.mark.parametrize("layout_name,hq,hkv,S,P", [("default", 8, 2, 3, 64), ("fast", 32, 8, 2, 64), ("default", 64, 8, 2, 64),
                                                   ("default", 8, 2, 3, 8), ("fast", 32, 8, 2, 40),
                                                   ("default", 24, 2, 2, 256), ("deep2", 8, 2, 2, 24)])
def test_fused_qk_qjl_matches_oracle(device, layout_name, hq, hkv, S, P):
    print(f"[qjl qk] {layout_name} hq={hq} hkv={hkv} S={S} P={P}", flush=True)
    block, qv, host, tk, tv, q, qd, pay, qs, tup = _qjl_case(device, layout_name, hq, hkv, S, 0, 3 + S, P=P)
    got = kernels.fused_qk(qd, PageSet(block, None), SCALE16, qjl=QJLPages(pay, qs)).float().cpu().numpy()
    blk = {k_: host[k_] for k_ in ("radii", "radii_scales", "angle_codes_l1", "angle_codes_deep", "metadata")}
    if blk["radii_scales"] is not None:
        blk["radii_scales"] = blk["radii_scales"].reshape(blk["radii"].shape[:3] + (1, 1))
    ref = oracle.cpu_fused_qk_qjl(q, blk, tup, SCALE16)
    assert max_abs(got, ref) <= 1e-2 and cosine(got, ref) >= 0.999


@pytest.mark.parametrize("layout_name,hq,hkv,S,tail,pps,masked,B", [
    ("default", 32, 8, 5, 0, 2, 0, 1),
    ("default", 32, 8, 6, 37, 2, 0, 1),
    ("fast", 64, 8, 4, 9, 1, 0, 1),
    ("default", 8, 2, 7, 0, 3, 21, 2),
    ("fast", 4, 4, 3, 63, 0, 0, 1),
    ("default", 8, 1, 70, 5, 1, 0, 1),  # 70 splits: two-tier combine
    ("fast", 32, 8, 17, 11, 6, 0, 1),  # 6-page splits, one tier: 4-wave workgroups, two pages per wave
    ("default", 16, 2, 16, 0, 8, 0, 2),  # 8-page splits on 4 waves, batch 2
    ("default", 24, 2, 5, 9, 2, 3, 1),  # GQA 12: the row token order (head blocks above 8 heads)
])
def test_decode_attention_qjl_matches_oracle(device, layout_name, hq, hkv, S, tail, pps, masked, B):
    print(f"[qjl attn] {layout_name} hq={hq} hkv={hkv} S={S} tail={tail} pps={pps} masked={masked} B={B}", flush=True)
    block, qv, host, tk, tv, q, qd, pay, qs, tup = _qjl_case(device, layout_name, hq, hkv, S, tail, 17 + S, B=B)
    seq = S * PAGE + tail - masked
    tkt = torch.from_numpy(tk).to(device) if tail else None
    tvt = torch.from_numpy(tv).to(device) if tail else None
    out = kernels.decode_attention(qd, PageSet(block, qv), tkt, tvt, seq, SCALE16, pages_per_split=pps,
                                   qjl=QJLPages(pay, qs)).float().cpu().numpy()
    blk = {k_: host[k_] for k_ in ("radii", "radii_scales", "angle_codes_l1", "angle_codes_deep", "metadata")}
    if blk["radii_scales"] is not None:
        blk["radii_scales"] = blk["radii_scales"].reshape(blk["radii"].shape[:3] + (1, 1))
    ref = oracle.cpu_online_attention_dense_tail(q, blk, (host["v_codes"], host["v_scales"]), tk, tv, SCALE16, seq,
                                                 qjl=tup)
    assert np.all(np.isfinite(out))
    ma, rl = max_abs(out, ref), rel_l2(out, ref)
    assert ma <= ATOL and rl <= RTOL_L2, f"max_abs={ma:.3g} rel_l2={rl:.3g}"
    # The correction takes part: the oracle without it gives another output.
    plain = oracle_out(host, tk, tv, q, seq)
    assert max_abs(plain, ref) > 1e-5


@pytest.mark.parametrize("layout_name,hq,hkv,S,tail,pps,masked,P", [
    ("default", 32, 8, 5, 0, 2, 0, 8),      # half-row token order, one sketch byte per token
    ("default", 32, 8, 6, 37, 2, 5, 40),    # 5 bytes per token: sketches at every byte offset of a dword
    ("default", 24, 2, 5, 9, 2, 3, 24),     # GQA 12: row token order
    ("fast", 64, 8, 4, 9, 1, 0, 128),
    ("fast", 32, 8, 17, 11, 6, 0, 256),     # 4-wave workgroups
    ("default", 8, 1, 70, 5, 1, 0, 32),     # two-tier combine
    ("deep2", 8, 2, 3, 0, 0, 0, 56),        # generic layout kernel
])
def test_decode_attention_qjl_any_width(device, layout_name, hq, hkv, S, tail, pps, masked, P):
    """qjl_proj_dim other than 64 (turbo_polar_config.py:36-37 takes any
    positive multiple of 8): the byte-aligned sketch path against the oracle."""
    print(f"[qjl attn P] {layout_name} hq={hq} hkv={hkv} S={S} tail={tail} pps={pps} masked={masked} P={P}", flush=True)
    block, qv, host, tk, tv, q, qd, pay, qs, tup = _qjl_case(device, layout_name, hq, hkv, S, tail, 29 + S, P=P)
    assert pay.packed_signs.shape[-1] == P // 8
    seq = S * PAGE + tail - masked
    tkt = torch.from_numpy(tk).to(device) if tail else None
    tvt = torch.from_numpy(tv).to(device) if tail else None
    out = kernels.decode_attention(qd, PageSet(block, qv), tkt, tvt, seq, SCALE16, pages_per_split=pps,
                                   qjl=QJLPages(pay, qs)).float().cpu().numpy()
    blk = {k_: host[k_] for k_ in ("radii", "radii_scales", "angle_codes_l1", "angle_codes_deep", "metadata")}
    if blk["radii_scales"] is not None:
        blk["radii_scales"] = blk["radii_scales"].reshape(blk["radii"].shape[:3] + (1, 1))
    ref = oracle.cpu_online_attention_dense_tail(q, blk, (host["v_codes"], host["v_scales"]), tk, tv, SCALE16, seq,
                                                 qjl=tup)
    assert np.all(np.isfinite(out))
    ma, rl = max_abs(out, ref), rel_l2(out, ref)
    assert ma <= ATOL and rl <= RTOL_L2, f"max_abs={ma:.3g} rel_l2={rl:.3g}"
    plain = oracle_out(host, tk, tv, q, seq)
    assert max_abs(plain, ref) > 1e-5


def test_qjl_width_outside_the_kernels_rejected(device):
    from turbopolar_amd.qjl import QJLPayload
    signs = torch.zeros((1, 2, 2, 64, 33), dtype=torch.uint8, device=device)
    norms = torch.zeros((1, 2, 2, 64), dtype=torch.float16, device=device)
    qs = torch.zeros((1, 8, 33), dtype=torch.uint8, device=device)
    with pytest.raises(NotImplementedError, match="multiple of 8 up to 256"):
        QJLPages(QJLPayload(signs, norms, 264, 42, (1, 2, 2, 64, 128)), qs)


def test_bridge_qjl_paths(device):
    block, qv, host, tk, tv, q, qd, pay, qs, tup = _qjl_case(device, "default", 8, 2, 2, 5, 23)
    bridge = HipKernelBridge()
    cfg = _cfg(8, 2)
    with pytest.raises(ValueError, match="qjl_payload and q_proj_signs are required"):
        bridge.execute_online_attention_quant_v(qd, block, qv, None, None, cfg, 2 * PAGE, use_qjl=True)
    out, trace = bridge.execute_online_attention_quant_v(qd, block, qv, pay, qs, cfg, 2 * PAGE, use_qjl=True)
    assert trace["qjl_used"] and trace["hip_kernel"] == "tp_decode_attention_qjl"
    direct = kernels.decode_attention(qd, PageSet(block, qv), None, None, 2 * PAGE, SCALE16, qjl=QJLPages(pay, qs))
    assert torch.equal(out, direct)
    tkt, tvt = torch.from_numpy(tk).to(device), torch.from_numpy(tv).to(device)
    out2, trace2 = bridge.execute_online_attention_quant_v_dense_tail(qd, block, qv, tkt, tvt, pay, qs, cfg,
                                                                      2 * PAGE + 5, use_qjl=True)
    assert trace2["qjl_used"]
    # The reference's scale test (tests/kernels/test_qjl_scaled_fused_qk.py): the QJL
    # contribution to the fused-QK scores is proportional to attention_scale.
    contrib = []
    for scale in (1.0, 0.5, 0.25):
        c = TurboPolarConfig(num_q_heads=8, num_kv_heads=2, qjl_proj_dim=64, attention_scale=scale)
        with_q = bridge.execute_fused_qk_qjl(qd, block, pay, qs, c).float()
        without = bridge.execute_fused_qk(qd, block, c).float()
        contrib.append(float((with_q - without).abs().mean()) / scale)
    assert contrib[0] > 0 and np.allclose(contrib, contrib[0], rtol=2e-2)
