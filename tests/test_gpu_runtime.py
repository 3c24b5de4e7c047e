"""Runtime API on the GPU: appends, flushes, telemetry and the decode step.

Mirrors the reference's runtime and integration suites
(tests/test_turbo_polar_cache_runtime.py, tests/benchmarks/test_turbopolar_fast_attention.py)
with the oracle standing in for MLX.
"""

import numpy as np
import pytest
import torch

import oracle
from common import ATOL, LAYOUTS, PAGE, RTOL_L2, cosine, max_abs, oracle_pages, rel_l2
from turbopolar_amd import TurboPolarConfig, TurboPolarFastCache, TurboPolarKVCacheRuntime, make_turbo_caches
from turbopolar_amd.kernels import fp16_scale

pytestmark = pytest.mark.gpu


def _cfg(layout_name, hq=4, hkv=2):
    int8, l1b, deepb, split = LAYOUTS[layout_name]
    return TurboPolarConfig(num_q_heads=hq, num_kv_heads=hkv, use_int8_radii=int8, k_angle_bits_level1=l1b,
                            k_angle_bits_deep=deepb, split_dim=split)


def _host_state(runtime):
    block, qv, tk, tv, _, seq = runtime.get_fused_attention_inputs()
    blk = None
    if block is not None:
        blk = {
            "radii": block.radii.cpu().numpy(),
            "radii_scales": block.radii_scales.cpu().numpy() if block.radii_scales is not None else None,
            "angle_codes_l1": block.angle_codes_l1.cpu().numpy(),
            "angle_codes_deep": block.angle_codes_deep.cpu().numpy(),
            "metadata": block.metadata,
        }
        qv = (qv.codes.cpu().numpy(), qv.scales.cpu().numpy())
    tk = tk.cpu().numpy() if tk is not None else np.zeros((1, runtime._num_kv_heads, 0, 128), np.float16)
    tv = tv.cpu().numpy() if tv is not None else np.zeros_like(tk)
    return blk, qv, tk, tv, seq


@pytest.mark.parametrize("layout_name", ["default", "fast"])
@pytest.mark.parametrize("total", [37, 64, 100, 130])
def test_decode_steps_match_oracle(device, layout_name, total):
    """Token-by-token decode (the reference's 37 / 100 / 64-token integration
    cases) against the oracle on the identical cache state, and the stored
    pages against the oracle encoding of the raw tokens."""
    print(f"[runtime] layout={layout_name} total={total}", flush=True)
    cfg = _cfg(layout_name)
    cache = TurboPolarFastCache(cfg)
    rng = np.random.default_rng(2026 + total)
    ks, vs = [], []
    for _ in range(total):
        q = rng.standard_normal((1, 4, 1, 128)).astype(np.float16)
        kn = rng.standard_normal((1, 2, 1, 128)).astype(np.float16)
        vn = rng.standard_normal((1, 2, 1, 128)).astype(np.float16)
        ks.append(kn)
        vs.append(vn)
        out = cache.decode_attention(torch.from_numpy(q).to(device), torch.from_numpy(kn).to(device),
                                     torch.from_numpy(vn).to(device), cfg.attention_scale)
        assert out.shape == (1, 4, 128)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    blk, qv, tk, tv, seq = _host_state(cache.runtime)
    assert seq == total
    qq = q[:, :, 0]
    scale = fp16_scale(cfg.attention_scale)
    if blk is None:
        ref = oracle.softmax_attention(qq, tk, tv, scale, seq)
    else:
        if blk["radii_scales"] is not None:
            blk["radii_scales"] = blk["radii_scales"].reshape(blk["radii"].shape[:3] + (1, 1))
        ref = oracle.cpu_online_attention_dense_tail(qq, blk, qv, tk, tv, scale, seq)
    assert max_abs(got, ref) <= ATOL and rel_l2(got, ref) <= RTOL_L2
    # Stored pages equal the oracle encoding of the raw tokens.
    S = total // PAGE
    if S:
        kk = np.concatenate(ks, axis=2)[:, :, : S * PAGE]
        vv = np.concatenate(vs, axis=2)[:, :, : S * PAGE]
        oblk, (vc, vsc) = oracle_pages(kk, vv, LAYOUTS[layout_name])
        assert np.array_equal(blk["radii"].view(np.uint8), oblk["radii"].view(np.uint8))
        assert np.array_equal(blk["angle_codes_deep"], oblk["angle_codes_deep"])
        assert np.array_equal(qv[0], vc) and np.array_equal(qv[1].view(np.uint16), vsc.view(np.uint16))
    # Against dense attention on the raw tokens (reference integration bound).
    dense = oracle.softmax_attention(qq, np.concatenate(ks, 2), np.concatenate(vs, 2), scale)
    assert cosine(got, dense) >= 0.95


def test_bulk_equals_incremental(device):
    """One 200-token append == 200 single-token appends (pages, tail, telemetry)."""
    cfg = _cfg("fast", hq=8, hkv=4)
    rng = np.random.default_rng(7)
    k = torch.from_numpy(rng.standard_normal((1, 4, 200, 128)).astype(np.float16)).to(device)
    v = torch.from_numpy(rng.standard_normal((1, 4, 200, 128)).astype(np.float16)).to(device)
    a = TurboPolarKVCacheRuntime(cfg)
    a.append(k, v)
    b = TurboPolarKVCacheRuntime(cfg)
    for t in range(200):
        b.append(k[:, :, t : t + 1], v[:, :, t : t + 1])
    for ra, rb in ((a.k_storage.radii, b.k_storage.radii), (a.v_storage.codes, b.v_storage.codes),
                   (a.k_storage.radii_scales, b.k_storage.radii_scales),
                   (a.k_storage.angle_codes_deep, b.k_storage.angle_codes_deep)):
        assert torch.equal(ra, rb)
    assert torch.equal(a.partial_k, b.partial_k)
    ta, tb = a.get_io_telemetry(), b.get_io_telemetry()
    assert ta == tb
    assert ta["total_blocks"] == 3 and ta["partial_tokens"] == 8
    assert ta["k_storage_capacity"] == 4 and ta["k_storage_reallocs"] == 0


@pytest.mark.parametrize("T", [1, 32, 63, 64, 65, 127, 128, 129])
@pytest.mark.parametrize("gqa", [1, 4])
def test_milestone_shapes(device, T, gqa):
    """turbo_polar_cache_runtime.py:42-56 shape matrix of the reference."""
    cfg = TurboPolarConfig(head_dim=128, qjl_proj_dim=64, block_size=64, split_dim=0, num_q_heads=4,
                           num_kv_heads=4 // gqa, use_qjl=False, seed=7)
    cache = TurboPolarKVCacheRuntime(cfg)
    hkv = cfg.num_kv_heads
    g = torch.Generator(device="cpu").manual_seed(T)
    k = torch.randn((1, hkv, T, 128), generator=g).to(device)
    v = torch.randn((1, hkv, T, 128), generator=g).to(device)
    cache.append(k, v)
    block, quant_v, dense_v, qjl, actual = cache.get_blocks_for_attention()
    assert actual == T and block is not None and quant_v is not None and dense_v is None and qjl is None
    S = block.radii.shape[2]
    assert S * 64 >= T > (S - 1) * 64
    tel = cache.get_io_telemetry()
    assert tel["partial_tokens"] == T % 64 and tel["total_blocks"] == T // 64


def test_telemetry_closed_forms(device):
    """Compression ratios 512/296 (default) and 512/264.03 (fast) at page multiples;
    capacity doubling 4 -> 8 -> 16 with the reference's copy accounting."""
    for name, ratio in (("default", 512 / 296), ("fast", 512 / (128 + 136 + 2 / 64))):
        cfg = _cfg(name, hq=8, hkv=8)
        rt = TurboPolarKVCacheRuntime(cfg)
        x = torch.randn((1, 8, 256, 128), device=device, dtype=torch.float16)
        rt.append(x, x)
        tel = rt.get_io_telemetry()
        assert abs(tel["compression_ratio"] - ratio) < 1e-9, (name, tel)
    rt = TurboPolarKVCacheRuntime(_cfg("default", hq=8, hkv=8))
    for _ in range(9):
        x = torch.randn((1, 8, 64, 128), device=device, dtype=torch.float16)
        rt.append(x, x)
    tel = rt.get_io_telemetry()
    assert tel["k_storage_capacity"] == 16 and tel["k_storage_reallocs"] == 2
    per_slot_k = 8 * 64 * (64 * 2 + 16 + 16)
    assert rt.k_storage.bytes_copied_during_growth == per_slot_k * (4 + 8)
    per_slot_v = 8 * 64 * (128 + 8)
    assert rt.v_storage.bytes_copied_during_growth == per_slot_v * (4 + 8)


def test_update_and_fetch_prefill(device):
    """Prefill returns decompressed K/V of every token, incl. the padded tail page."""
    cfg = _cfg("fast", hq=4, hkv=2)
    cache = make_turbo_caches(1, 4, 2, 128)[0]
    rng = np.random.default_rng(1)
    k = rng.standard_normal((1, 2, 100, 128)).astype(np.float16)
    v = rng.standard_normal((1, 2, 100, 128)).astype(np.float16)
    kd, vd = cache.update_and_fetch(torch.from_numpy(k).to(device), torch.from_numpy(v).to(device))
    assert kd.shape == (1, 2, 100, 128) and vd.shape == (1, 2, 100, 128)
    kp = np.zeros((1, 2, 128, 128), np.float16)
    vp = np.zeros((1, 2, 128, 128), np.float16)
    kp[:, :, :100], vp[:, :, :100] = k, v
    blk, (vc, vsc) = oracle_pages(kp, vp, LAYOUTS["fast"])
    kref = oracle.decode_block(blk["radii"], blk["radii_scales"].reshape(1, 2, 2, 1, 1), blk["angle_codes_l1"],
                               blk["angle_codes_deep"], blk["metadata"])[:, :, :100]
    vref = oracle.dequantize_block(vc, vsc).reshape(1, 2, 128, 128)[:, :, :100]
    assert np.array_equal(vd.cpu().numpy().view(np.uint16), vref.view(np.uint16))
    ulp = np.spacing(np.abs(kref).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(kd.cpu().numpy().astype(np.float64) - kref) <= ulp)
    assert cosine(kd.cpu().numpy(), k) >= 0.99


def test_append_rejects_nonfinite_and_changes(device):
    rt = TurboPolarKVCacheRuntime(_cfg("default", hq=4, hkv=4))
    good = torch.randn((1, 4, 64, 128), device=device, dtype=torch.float16)
    rt.append(good, good)
    assert rt.partial_k is None
    with pytest.raises(ValueError, match="batch size changed"):
        x = torch.randn((2, 4, 1, 128), device=device, dtype=torch.float16)
        rt.append(x, x)
    with pytest.raises(ValueError, match="dtype changed"):
        x = torch.randn((1, 4, 1, 128), device=device, dtype=torch.float32)
        rt.append(x, x)
    bad = good[:, :, :2].clone()
    bad[0, 0, 0, 0] = float("inf")
    with pytest.raises(ValueError, match="finite"):
        rt.append(bad, good[:, :, :2])


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("where,value", [("k", float("inf")), ("v", float("nan")), ("k", float("-inf"))])
def test_append_stage_rejects_without_state_change(device, dtype, where, value):
    """tp_append_stage scans every element: a non-finite value anywhere raises
    the reference's ValueError and leaves length, tail and storage unchanged."""
    print(f"[append-stage] dtype={dtype} {where}={value}", flush=True)
    rt = TurboPolarKVCacheRuntime(_cfg("default", hq=8, hkv=4))
    base_k = torch.randn((1, 4, 100, 128), device=device).to(dtype)
    base_v = torch.randn((1, 4, 100, 128), device=device).to(dtype)
    rt.append(base_k, base_v)  # one page + 36 tail tokens
    tail_before = rt.partial_k.clone()
    tel_before = rt.get_io_telemetry()
    for T, pos in ((1, 0), (30, 29), (200, 137)):
        k = torch.randn((1, 4, T, 128), device=device).to(dtype)
        v = torch.randn((1, 4, T, 128), device=device).to(dtype)
        (k if where == "k" else v)[0, 3, pos, 127] = value
        with pytest.raises(ValueError, match="finite"):
            rt.append(k, v)
        assert rt.actual_seq_len == 100 and rt.total_blocks == 1
        assert torch.equal(rt.partial_k, tail_before)
        assert rt.get_io_telemetry() == tel_before
    # the cache still works afterwards
    k = torch.randn((1, 4, 28, 128), device=device).to(dtype)
    rt.append(k, k)
    assert rt.actual_seq_len == 128 and rt.total_blocks == 2 and rt.partial_k is None


def test_append_error_order_matches_reference(device):
    """Non-finite input together with a changed batch size: the finiteness
    error comes first, as in turbo_polar_cache.py:69-75."""
    rt = TurboPolarKVCacheRuntime(_cfg("default", hq=4, hkv=4))
    x = torch.randn((1, 4, 3, 128), device=device, dtype=torch.float16)
    rt.append(x, x)
    y = torch.randn((2, 4, 1, 128), device=device, dtype=torch.float16)
    y[1, 0, 0, 0] = float("nan")
    with pytest.raises(ValueError, match="finite"):
        rt.append(y, y)
    with pytest.raises(ValueError, match="batch size changed"):
        rt.append(y.nan_to_num(), y.nan_to_num())


def test_single_token_appends_match_bulk(device):
    """4096 single-token appends (BASELINE configs[3] workload 2, shortened to
    200 + a page boundary mix) give the storage and tail of one bulk append."""
    cfg = _cfg("default", hq=8, hkv=2)
    k = torch.randn((1, 2, 200, 128), device=device, dtype=torch.float16)
    v = torch.randn((1, 2, 200, 128), device=device, dtype=torch.float16)
    a = TurboPolarKVCacheRuntime(cfg)
    for t in range(200):
        a.append(k[:, :, t:t + 1], v[:, :, t:t + 1])
    b = TurboPolarKVCacheRuntime(cfg)
    for lo, hi in ((0, 7), (7, 64), (64, 65), (65, 200)):
        b.append(k[:, :, lo:hi], v[:, :, lo:hi])
    c = TurboPolarKVCacheRuntime(cfg)
    c.append(k, v)
    for r in (a, b):
        assert r.actual_seq_len == c.actual_seq_len == 200 and r.total_blocks == c.total_blocks == 3
        assert torch.equal(r.partial_k, c.partial_k) and torch.equal(r.partial_v, c.partial_v)
        bk, bv, *_ = r.get_fused_attention_inputs()
        ck, cv, *_ = c.get_fused_attention_inputs()
        assert torch.equal(bk.radii, ck.radii) and torch.equal(bk.angle_codes_l1, ck.angle_codes_l1)
        assert torch.equal(bk.angle_codes_deep, ck.angle_codes_deep)
        assert torch.equal(bv.codes, cv.codes) and torch.equal(bv.scales, cv.scales)


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("tokens", [1, 300])
def test_append_stage_flag_modes(device, mode, tokens):
    """tp_append_stage's verdict through a device flag (check 1, read back with
    a copy) and through a pinned host flag (check 2, written by the kernel;
    one workgroup reports completion itself and the host polls, several are
    synchronised): both report a NaN, both pass finite input, and a stale
    value in the flag never reads as a new verdict."""
    from turbopolar_amd import _lib

    L = _lib.lib()
    flag = torch.zeros(1, dtype=torch.int32, device=device) if mode == 1 else torch.zeros(1, dtype=torch.int32, pin_memory=True)
    tail_k = torch.zeros((8, 64, 128), dtype=torch.float16, device=device)
    tail_v = torch.zeros_like(tail_k)
    k = torch.randn((8, tokens, 128), dtype=torch.float16, device=device)
    v = torch.randn_like(k)
    stream = torch.cuda.current_stream(device).cuda_stream

    def stage(kk, epoch):
        return L.tp_append_stage(kk.data_ptr(), v.data_ptr(), 0, 8, tokens, 0, 1, tail_k.data_ptr(), tail_v.data_ptr(),
                                 64, 0, mode, flag.data_ptr(), epoch, stream)

    assert stage(k, 2) == _lib.TP_OK
    bad = k.clone()
    bad[3, tokens - 1, 77] = float("nan")
    assert stage(bad, 4) == _lib.TP_ERR_NONFINITE
    assert stage(k, 6) == _lib.TP_OK  # the flag still holds the last verdict
    assert stage(bad, 8) == _lib.TP_ERR_NONFINITE
    assert stage(k, 10) == _lib.TP_OK
    assert torch.equal(tail_k[:, 0], k[:, 0])


@pytest.mark.parametrize("layout_name", ["default", "fast"])
def test_fetch_blocks_and_bytes_read(device, layout_name):
    """fetch_blocks (turbo_polar_cache.py:321-346): the selected pages decoded
    in the given order, equal within one fp16 ulp to the oracle's decode of
    the same stored pages, and bytes_read grown by the key bytes of each page
    fetched (radii + both angle rows, + the page scale for int8 radii)."""
    cfg = _cfg(layout_name, hq=8, hkv=2)
    rt = TurboPolarKVCacheRuntime(cfg)
    rng = np.random.default_rng(31)
    k = rng.standard_normal((2, 2, 3 * PAGE + 10, 128)).astype(np.float16)
    v = rng.standard_normal((2, 2, 3 * PAGE + 10, 128)).astype(np.float16)
    rt.append(torch.from_numpy(k).to(device), torch.from_numpy(v).to(device))
    blk, _, _, _, _ = _host_state(rt)
    rs = blk["radii_scales"]
    kref = oracle.decode_block(blk["radii"], None if rs is None else rs.reshape(rs.shape[:3] + (1, 1)),
                               blk["angle_codes_l1"], blk["angle_codes_deep"], blk["metadata"])
    kref = kref.reshape(2, 2, 3, PAGE, 128)
    int8, l1b, deepb, split = LAYOUTS[layout_name]
    l1_row, deep_row = oracle.layout_bytes(l1b, deepb, split)
    per_page = 2 * 2 * PAGE * (64 * (1 if int8 else 2) + l1_row + deep_row) + (2 * 2 * 2 if int8 else 0)
    assert rt.bytes_read == 0
    for indices, expect_pages in ((None, [0, 1, 2]), ([2, 0], [2, 0]), ([1], [1])):
        before = rt.bytes_read
        got = rt.fetch_blocks(indices)
        torch.cuda.synchronize()
        assert tuple(got.shape) == (2, 2, PAGE * len(expect_pages), 128) and got.dtype == torch.float16
        want = np.concatenate([kref[:, :, p] for p in expect_pages], axis=2)
        g = got.cpu().numpy().astype(np.float64)
        ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
        assert np.all(np.abs(g - want) <= ulp + 1e-12), indices
        assert rt.bytes_read - before == per_page * len(expect_pages)
    empty = TurboPolarKVCacheRuntime(cfg)
    assert empty.fetch_blocks().numel() == 0


def test_tail_views_follow_the_cache(device):
    """get_fused_attention_inputs returns the dense tail as views of the
    runtime's tail buffer (no copy per decode step): they hold the tail at the
    time of the call and are valid until the next append, which may rewrite
    them in place.  The partial_k / partial_v properties return copies that an
    append never changes, as the reference's immutable arrays do."""
    cfg = _cfg("default")
    rt = TurboPolarKVCacheRuntime(cfg)
    rng = np.random.default_rng(32)
    k = torch.from_numpy(rng.standard_normal((1, 2, 70, 128)).astype(np.float16)).to(device)
    v = torch.from_numpy(rng.standard_normal((1, 2, 70, 128)).astype(np.float16)).to(device)
    rt.append(k[:, :, :60], v[:, :, :60])
    pk = rt.partial_k
    snap = pk.clone()
    _, _, tk, _, _, seq = rt.get_fused_attention_inputs()
    assert seq == 60 and torch.equal(tk, k[:, :, :60])
    rt.append(k[:, :, 60:], v[:, :, 60:])  # completes page 0, 6 tokens stay in the tail
    torch.cuda.synchronize()
    assert torch.equal(pk, snap), "a partial_k copy changed under an append"
    assert torch.equal(rt.partial_k, k[:, :, 64:70])
    _, _, tk2, _, _, seq2 = rt.get_fused_attention_inputs()
    assert seq2 == 70 and torch.equal(tk2, k[:, :, 64:70])


@pytest.mark.parametrize("start", [10, 63, 127])
def test_deferred_check_rolls_back(device, start):
    """append(..., defer_check=True) does not wait for the non-finite verdict;
    resolve_deferred_check() reads it.  A non-finite token (here also one that
    completes a page: start 63, 127) is undone with every deferred append
    after it, the reference's ValueError is raised, and the cache then equals
    a twin that never saw the token: same counters, same pages, same decode
    output bit for bit."""
    cfg = _cfg("default", hq=8, hkv=2)
    g = torch.Generator(device=device).manual_seed(start)
    kv = torch.randn((1, 2, start + 8, 128), generator=g, device=device).half()
    a, b = TurboPolarFastCache(cfg), TurboPolarFastCache(cfg)
    a.runtime.append(kv[:, :, :start], kv[:, :, :start])
    b.runtime.append(kv[:, :, :start], kv[:, :, :start])
    bad = kv[:, :, start:start + 1].clone()
    bad[0, 1, 0, 5] = float("nan")
    a.runtime.append(bad, kv[:, :, start:start + 1], defer_check=True)  # returns without a verdict
    nxt = kv[:, :, start + 1:start + 2]
    if (start + 1) % PAGE:  # the bad token left a tail: a second deferred append stacks on it
        a.runtime.append(nxt, nxt, defer_check=True)
        assert a.runtime.deferred_verdict_pending() and a.offset == start + 2
        with pytest.raises(ValueError, match="finite"):
            a.runtime.resolve_deferred_check()
    else:  # it completed a page: the next deferred append would restart the tail, so it resolves first
        assert a.runtime.deferred_verdict_pending() and a.offset == start + 1
        with pytest.raises(ValueError, match="finite"):
            a.runtime.append(nxt, nxt, defer_check=True)
    assert not a.runtime.deferred_verdict_pending()
    for attr in ("actual_seq_len", "_tail_len", "total_blocks", "bytes_written"):
        assert getattr(a.runtime, attr) == getattr(b.runtime, attr), attr
    assert a.runtime.k_storage.block_count == b.runtime.k_storage.block_count
    # Both continue with the same finite tokens (deferred, then resolved) and agree exactly.
    q = torch.randn((1, 8, 1, 128), generator=g, device=device).half()
    for t in range(start + 1, start + 8):
        tok = kv[:, :, t:t + 1]
        oa = a.decode_attention(q, tok, tok, 0.088, defer_check=True)
        ob = b.decode_attention(q, tok, tok, 0.088)
        assert torch.equal(oa, ob), t
    a.runtime.resolve_deferred_check()
    assert a.offset == b.offset == start + 7


def test_deferred_check_resolved_by_next_plain_append(device):
    """A pending deferred verdict is resolved before any append that is not
    itself deferred, so a non-finite token cannot slip past the contract."""
    rt = TurboPolarKVCacheRuntime(_cfg("default", hq=4, hkv=2))
    x = torch.randn((1, 2, 5, 128), device=device).half()
    rt.append(x, x)
    bad = x[:, :, :1].clone()
    bad[0, 0, 0, 0] = float("inf")
    rt.append(bad, x[:, :, :1], defer_check=True)
    with pytest.raises(ValueError, match="finite"):
        rt.append(x[:, :, :2], x[:, :, :2])
    assert rt.actual_seq_len == 5 and rt._tail_len == 5
    rt.append(x[:, :, :2], x[:, :, :2])
    assert rt.actual_seq_len == 7
