"""Pins of the oracle's QJL restatement (rfsn_v11/quant/qjl/encoder.py:19-44,
score_estimate.py:6-54, kernels/turbo_polar/metal.py:262-265).

Each check is independent of the formula it pins: brute-force loops, closed
forms of the estimator, and its statistical consistency (the sign-agreement
estimate converges to q . E as the projection count grows, so a wrong sign,
a wrong factor of pi or a reversed bit order fails)."""

import math

import numpy as np
import pytest

import oracle


def test_projection_unit_columns_and_seed_stream():
    w = oracle.qjl_projection(42, 128, 64)
    assert w.shape == (128, 64) and w.dtype == np.float32
    assert np.allclose(np.linalg.norm(w.astype(np.float64), axis=0), 1.0, atol=1e-6)
    raw = np.random.Generator(np.random.PCG64(42)).standard_normal((128, 64), dtype=np.float32)
    assert np.allclose(w * np.linalg.norm(raw, axis=0), raw, rtol=1e-6, atol=1e-7)  # columns scaled only
    assert not np.allclose(oracle.qjl_projection(43, 128, 64), w)


def test_pack_signs_single_bits_and_zero():
    for j in range(64):
        proj = -np.ones(64)
        proj[j] = 1.0
        packed = oracle.qjl_pack_signs(proj)
        expect = np.zeros(8, np.uint8)
        expect[j // 8] = 1 << (j % 8)
        assert np.array_equal(packed, expect), j
    assert np.array_equal(oracle.qjl_pack_signs(np.zeros(64)), np.full(8, 255, np.uint8))  # 0 >= 0
    assert np.array_equal(oracle.qjl_pack_signs(-np.zeros(64)), np.full(8, 255, np.uint8))  # -0 >= 0


def test_residual_sketch_brute_force():
    rng = np.random.default_rng(0)
    w = oracle.qjl_projection(7, 128, 32)
    e = rng.standard_normal((3, 128)).astype(np.float16)
    packed, norms = oracle.qjl_residual_sketch(e, w)
    for r in range(3):
        for p in range(32):
            dot = sum(float(e[r, d]) * float(w[d, p]) for d in range(128))
            assert ((packed[r, p // 8] >> (p % 8)) & 1) == (1 if dot >= 0 else 0)
        assert norms[r] == np.float16(math.sqrt(sum(float(x) ** 2 for x in e[r])))


def _brute_estimate(q, packed, norms, q_packed, P):
    B, Hkv, S, L, _ = packed.shape
    Hq = q_packed.shape[1]
    out = np.zeros((B, Hq, S * L))
    for b in range(B):
        for h in range(Hq):
            kv = h // (Hq // Hkv)
            qn = math.sqrt(sum(float(x) ** 2 for x in q[b, h]))
            for s in range(S):
                for t in range(L):
                    ham = sum(bin(int(packed[b, kv, s, t, j]) ^ int(q_packed[b, h, j])).count("1") for j in range(P // 8))
                    out[b, h, s * L + t] = float(norms[b, kv, s, t]) * qn * math.sin(math.pi / 2 * (P - 2 * ham) / P)
    return out


def test_estimate_brute_force_gqa():
    rng = np.random.default_rng(1)
    B, Hkv, Hq, S, L, P = 2, 2, 6, 2, 5, 64
    packed = rng.integers(0, 256, (B, Hkv, S, L, P // 8), dtype=np.uint8)
    norms = rng.uniform(0, 2, (B, Hkv, S, L)).astype(np.float16)
    q_packed = rng.integers(0, 256, (B, Hq, P // 8), dtype=np.uint8)
    q = rng.standard_normal((B, Hq, 128)).astype(np.float16)
    got = oracle.qjl_dot_estimate(q, packed, norms, q_packed, P)
    assert np.allclose(got, _brute_estimate(q, packed, norms, q_packed, P), rtol=1e-12, atol=1e-12)


def test_estimate_closed_forms():
    q = np.ones((1, 1, 128), np.float16)
    qn = math.sqrt(128.0)
    norms = np.full((1, 1, 1, 3), 0.5, np.float16)
    q_packed = np.full((1, 1, 8), 0b10110010, np.uint8)
    k = np.stack([q_packed[0, 0], ~q_packed[0, 0], q_packed[0, 0] ^ np.array([255, 255, 255, 255, 0, 0, 0, 0], np.uint8)])
    est = oracle.qjl_dot_estimate(q, k.reshape(1, 1, 1, 3, 8), norms, q_packed, 64)[0, 0]
    assert est[0] == pytest.approx(0.5 * qn, rel=1e-12)   # equal sketches
    assert est[1] == pytest.approx(-0.5 * qn, rel=1e-12)  # complementary sketches
    assert abs(est[2]) < 1e-12                             # half the bits differ


def test_estimate_converges_to_the_dot_product():
    rng = np.random.default_rng(2)
    P = 8192
    w = oracle.qjl_projection(11, 128, P)
    e = rng.standard_normal((1, 1, 1, 4, 128))
    q = rng.standard_normal((1, 1, 128))
    e[0, 0, 0, 1] = 2.0 * q[0, 0] + 0.1 * e[0, 0, 0, 1]   # nearly parallel
    e[0, 0, 0, 2] = -q[0, 0] + 0.3 * e[0, 0, 0, 2]        # nearly anti-parallel
    packed, norms = oracle.qjl_residual_sketch(e, w)
    qp, _ = oracle.qjl_residual_sketch(q, w)
    est = oracle.qjl_dot_estimate(q, packed, norms, qp, P)[0, 0]
    true = e[0, 0, 0] @ q[0, 0]
    scale = np.linalg.norm(e[0, 0, 0], axis=1) * np.linalg.norm(q[0, 0])
    assert np.all(np.abs(est - true) <= 0.03 * scale), (est, true)


def test_fused_qk_qjl_adds_scaled_estimate():
    rng = np.random.default_rng(3)
    k = rng.standard_normal((1, 2, 64, 128)).astype(np.float16)
    blk = oracle.encode_block(k, l1_bits=4, deep_bits=4, split_dim=64)
    for f in ("radii", "angle_codes_l1", "angle_codes_deep"):
        blk[f] = blk[f][:, :, None]
    w = oracle.qjl_projection(42, 128, 64)
    res = k.astype(np.float64) - oracle.decode_block(blk["radii"], None, blk["angle_codes_l1"],
                                                     blk["angle_codes_deep"], blk["metadata"]).astype(np.float64)
    packed, norms = oracle.qjl_residual_sketch(res.reshape(1, 2, 1, 64, 128), w)
    q = rng.standard_normal((1, 4, 128)).astype(np.float16)
    qp, _ = oracle.qjl_residual_sketch(q, w)
    qjl = (packed, norms, qp, 64)
    for scale in (1.0, 0.5, 0.125):
        diff = oracle.cpu_fused_qk_qjl(q, blk, qjl, scale) - oracle.cpu_fused_qk(q, blk, scale)
        assert np.allclose(diff, oracle.qjl_dot_estimate(q, *qjl) * scale, rtol=1e-12, atol=1e-12)
