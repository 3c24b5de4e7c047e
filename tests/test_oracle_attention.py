"""Pins the oracle's attention restatement (metal.py:254-332 of the reference).

Independent checks: torch's float64 scaled_dot_product_attention on the same
decoded K/V, brute-force Python loops on tiny inputs, and the split-K merge
algebra (partial (m, l, acc) per split, rescaled by exp(m_i - M)) that the HIP
kernel uses, against the one-pass softmax.
"""

import math

import numpy as np
import pytest
import torch

import oracle
from common import LAYOUTS, gen_kv, gen_q, oracle_pages


def _sdpa(q, k, v, scale, seq_len=None):
    """torch float64 SDPA with the GQA broadcast done by repeat_interleave."""
    qt = torch.from_numpy(q.astype(np.float64))[:, :, None, :]
    g = q.shape[1] // k.shape[1]
    kt = torch.from_numpy(k.astype(np.float64)).repeat_interleave(g, dim=1)
    vt = torch.from_numpy(v.astype(np.float64)).repeat_interleave(g, dim=1)
    mask = None
    if seq_len is not None:
        mask = (torch.arange(k.shape[2]) < seq_len)[None, :]
    out = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=scale)
    return out[:, :, 0].numpy()


@pytest.mark.parametrize("hq,hkv,T,seq", [(4, 4, 64, 64), (8, 2, 130, 130), (32, 8, 256, 200), (6, 1, 70, 1)])
def test_softmax_attention_matches_torch_sdpa(hq, hkv, T, seq):
    rng = np.random.default_rng(T)
    q = rng.standard_normal((2, hq, 128)).astype(np.float16)
    k = rng.standard_normal((2, hkv, T, 128)).astype(np.float16)
    v = rng.standard_normal((2, hkv, T, 128)).astype(np.float16)
    scale = oracle.fp16_scale(1 / math.sqrt(128))
    got = oracle.softmax_attention(q, k, v, scale, seq)
    ref = _sdpa(q, k, v, scale, seq)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_tiny_brute_force():
    """One page, 2 q heads on 1 kv head, with a dense tail: explicit loops."""
    rng = np.random.default_rng(0)
    k, v = gen_kv(0, 1, 1, 64 + 5, "normal", np.float16)
    q = gen_q(0, 1, 2)
    blk, qv = oracle_pages(k[:, :, :64], v[:, :, :64], LAYOUTS["default"])
    scale = 0.08837890625
    got = oracle.cpu_online_attention_dense_tail(q, blk, qv, k[:, :, 64:], v[:, :, 64:], scale, 69)
    kd = oracle.decode_block(blk["radii"], None, blk["angle_codes_l1"], blk["angle_codes_deep"], blk["metadata"])
    vd = oracle.dequantize_block(*qv).reshape(1, 1, 64, 128)
    K = np.concatenate([kd, k[:, :, 64:]], 2)[0, 0].astype(float)
    V = np.concatenate([vd, v[:, :, 64:]], 2)[0, 0].astype(float)
    for h in range(2):
        s = [sum(float(q[0, h, d]) * K[t, d] for d in range(128)) * scale for t in range(69)]
        m = max(s)
        w = [math.exp(x - m) for x in s]
        z = sum(w)
        for d in range(0, 128, 17):
            assert abs(got[0, h, d] - sum(w[t] * V[t, d] for t in range(69)) / z) < 1e-12


def test_fused_qk_scores_brute_force():
    k, _ = gen_kv(5, 1, 2, 128, "normal", np.float16)
    q = gen_q(5, 1, 4)
    blk, _ = oracle_pages(k, k, LAYOUTS["fast"])
    scores = oracle.cpu_fused_qk(q, blk, 0.125)
    kd = oracle.decode_block(blk["radii"], blk["radii_scales"], blk["angle_codes_l1"], blk["angle_codes_deep"],
                             blk["metadata"]).astype(np.float64)
    for hq in range(4):
        ref = kd[0, hq // 2] @ q[0, hq].astype(np.float64) * 0.125
        assert np.allclose(scores[0, hq], ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("n_splits", [1, 2, 3, 8, 13])
def test_split_k_merge_equals_one_pass(n_splits):
    """The kernel's combine: per split (m_i, l_i, acc_i) in log2 units, merged
    with weights 2^(m_i - M) -- equal to the one-pass softmax."""
    rng = np.random.default_rng(n_splits)
    T = 640
    s = rng.standard_normal(T) * 3
    v = rng.standard_normal((T, 128))
    bounds = np.linspace(0, T, n_splits + 1).astype(int)
    parts = []
    for a, b in zip(bounds[:-1], bounds[1:]):
        x = s[a:b] * math.log2(math.e)
        m = x.max()
        p = np.exp2(x - m)
        parts.append((m, p.sum(), p @ v[a:b]))
    M = max(p[0] for p in parts)
    L = sum(p[1] * 2 ** (p[0] - M) for p in parts)
    acc = sum(p[2] * 2 ** (p[0] - M) for p in parts)
    w = np.exp(s - s.max())
    assert np.allclose(acc / L, (w @ v) / w.sum(), rtol=1e-12, atol=1e-12)


def test_lazy_rescale_reference_is_exact():
    """Any common reference max gives the same softmax (the kernel keeps a stale
    max until scores exceed it by 2^8): sum p_t v_t / sum p_t is invariant."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal(300) * 4
    v = rng.standard_normal((300, 16))
    for ref in (x.max(), x.max() - 8, x.max() - 3.5):
        p = np.exp2(x - ref)
        assert np.allclose((p @ v) / p.sum(), (np.exp2(x - x.max()) @ v) / np.exp2(x - x.max()).sum())


def test_dense_tail_equals_concatenated_attention():
    k, v = gen_kv(3, 1, 2, 2 * 64 + 37, "normal", np.float16)
    q = gen_q(3, 1, 8)
    blk, qv = oracle_pages(k[:, :, :128], v[:, :, :128], LAYOUTS["default"])
    got = oracle.cpu_online_attention_dense_tail(q, blk, qv, k[:, :, 128:], v[:, :, 128:], 0.08837890625, 165)
    kd = oracle.decode_block(blk["radii"], None, blk["angle_codes_l1"], blk["angle_codes_deep"], blk["metadata"])
    vd = oracle.dequantize_block(*qv).reshape(1, 2, 128, 128)
    ref = _sdpa(q, np.concatenate([kd, k[:, :, 128:]], 2), np.concatenate([vd, v[:, :, 128:]], 2), 0.08837890625)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)


def _sdpa_bias(q, k, v, scale, bias, seq_len):
    """torch float64 SDPA with an additive float mask: the bias on valid tokens, -inf past seq_len."""
    qt = torch.from_numpy(q.astype(np.float64))[:, :, None, :]
    g = q.shape[1] // k.shape[1]
    kt = torch.from_numpy(k.astype(np.float64)).repeat_interleave(g, dim=1)
    vt = torch.from_numpy(v.astype(np.float64)).repeat_interleave(g, dim=1)
    mask = torch.from_numpy(bias.astype(np.float64))[:, :, None, :].clone()
    mask[..., seq_len:] = -math.inf
    out = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=scale)
    return out[:, :, 0].numpy()


@pytest.mark.parametrize("hq,hkv,pages,seq", [(8, 2, 2, 128), (4, 4, 3, 150), (12, 3, 1, 1)])
def test_dense_v_matches_torch_sdpa(hq, hkv, pages, seq):
    """Decoded K pages with a dense fp16 V of shape [B, Hkv, S, 64, 128]:
    torch float64 SDPA on the same K and V, tokens past ``seq`` masked."""
    k, v = gen_kv(5 + pages, 2, hkv, pages * 64, "normal", np.float16)
    q = gen_q(5 + pages, 2, hq)
    blk, _ = oracle_pages(k, v, LAYOUTS["default"])
    v5 = v.reshape(2, hkv, pages, 64, 128)
    scale = 0.08837890625
    got = oracle.cpu_online_attention_dense_v(q, blk, v5, scale, seq)
    kd = oracle.decode_block(blk["radii"], None, blk["angle_codes_l1"], blk["angle_codes_deep"], blk["metadata"])
    ref = _sdpa(q, kd, v, scale, seq)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    # A V that differs from the quantised one: the dense values themselves are used.
    q_only = oracle.cpu_online_attention(q, blk, oracle.quantize_block(v5), scale, seq)
    assert not np.allclose(got, q_only, rtol=1e-9, atol=1e-9)


def test_dense_v_qjl_bias_is_scaled_estimate_on_every_token():
    """With QJL the estimate times ``scale`` is added to every page token's
    score: SDPA with that additive float mask."""
    k, v = gen_kv(9, 1, 2, 128, "normal", np.float16)
    q = gen_q(9, 1, 4)
    blk, _ = oracle_pages(k, v, LAYOUTS["default"])
    kd = oracle.decode_block(blk["radii"], None, blk["angle_codes_l1"], blk["angle_codes_deep"], blk["metadata"])
    w = oracle.qjl_projection(42, 128, 64)
    res = (k.astype(np.float64) - kd.astype(np.float64)).reshape(1, 2, 2, 64, 128)
    packed, norms = oracle.qjl_residual_sketch(res, w)
    qp, _ = oracle.qjl_residual_sketch(q, w)
    qjl = (packed, norms, qp, 64)
    scale = 0.125
    got = oracle.cpu_online_attention_dense_v(q, blk, v.reshape(1, 2, 2, 64, 128), scale, 100, qjl=qjl)
    bias = oracle.qjl_dot_estimate(q, *qjl) * scale
    assert np.abs(bias[..., :100]).max() > 1e-3
    ref = _sdpa_bias(q, kd, v, scale, bias, 100)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
