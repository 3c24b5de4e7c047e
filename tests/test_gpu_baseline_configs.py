"""Every BASELINE configuration at its full size through the HIP path, checked
against the oracle on the same pages.

configs[0] (4096 tokens) and configs[2] at 32k run in test_gpu_attention.py;
this file holds the rest at their stated sizes:

* Llama-3.2-1B shape (32 q / 8 kv heads), 32768 tokens per layer,
  K ~ N(0,1) x per-channel scales log-uniform in [0.25, 4], several layers,
  each through its own ``TurboPolarKVCacheRuntime`` and the kernel bridge,
  all sharing the bridge's split-K workspace;
* Llama-3-8B shape (32 q / 8 kv heads) at 8192 and 131072 tokens,
  K with 4 outlier channels x20 per head, q ~ N(0,1)/sqrt(128);
* bulk encode of 32768 fp16 tokens x 8 kv heads into 512 pages
  (bit-exact against the oracle encoder) and 4096 single-token appends
  (storage bit-identical to the bulk encode);
* Llama-3-70B shape (64 q / 8 kv heads), 131072 tokens, K
  Student-t(3) x per-channel scales log-uniform in [0.1, 10]: the NaN and
  +-inf positions of the reference's CPU path exactly (at this length every
  query head is NaN there), and the same shape with K clipped to +-200, whose
  outputs are finite, within tolerance.

The oracle is evaluated one kv head at a time in float64 (the decoded fp16 K
and V of one head at 131072 tokens are 64 MiB each), which is the reference
CPU path's ``_cpu_online_attention_dense_tail`` (metal.py:293-332) per GQA
group.  Tolerances: max-abs 2e-3, relative L2 1e-3.
"""

import numpy as np
import pytest
import torch

import oracle
from common import LAYOUTS, PAGE, gen_kv, gen_q, oracle_pages
from test_gpu_attention import SCALE16, build_case, check, run_gpu
from test_gpu_encode import assert_bits_equal, encode_gpu

pytestmark = pytest.mark.gpu


def oracle_by_head(host, tk, tv, q, seq_len, hkv):
    """The oracle's dense-tail attention, one kv head (and its q heads) at a time."""
    hq = q.shape[1]
    g = hq // hkv
    out = np.empty((1, hq, 128), np.float64)
    rs = host["radii_scales"]
    for h in range(hkv):
        blk = {
            "radii": host["radii"][:, h:h + 1],
            "radii_scales": None if rs is None else rs[:, h:h + 1].reshape(1, 1, -1, 1, 1),
            "angle_codes_l1": host["angle_codes_l1"][:, h:h + 1],
            "angle_codes_deep": host["angle_codes_deep"][:, h:h + 1],
            "metadata": host["metadata"],
        }
        qv = (host["v_codes"][:, h:h + 1], host["v_scales"][:, h:h + 1])
        out[:, h * g:(h + 1) * g] = oracle.cpu_online_attention_dense_tail(
            q[:, h * g:(h + 1) * g], blk, qv, tk[:, h:h + 1], tv[:, h:h + 1], SCALE16, seq_len)
    return out


@pytest.mark.parametrize("context", [8192, 131072])
def test_config2_contexts(device, context):
    """configs[2] at 8k and 131072 tokens (default split, so 131072 runs the
    long split-K reduction: 32 splits of 64 pages per kv head), plus a dense
    tail and a masked suffix at 131072 + 37 tokens."""
    S = context // PAGE
    tail = 37 if context == 131072 else 0
    print(f"[config2] context={context} tail={tail}", flush=True)
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS["default"], 32, 8, S, tail, seed=5, kind="outlier",
                                            qscale=1.0 / np.sqrt(128.0))
    seq = S * PAGE + tail
    out = run_gpu(device, block, qv, tk, tv, q, seq)
    check(out, oracle_by_head(host, tk, tv, q, seq, 8), f"config2 {context}")
    if tail:
        seq = S * PAGE - 100  # masks the tail and the end of the last page
        out = run_gpu(device, block, qv, tk, tv, q, seq)
        check(out, oracle_by_head(host, tk, tv, q, seq, 8), f"config2 {context} masked")


@pytest.mark.parametrize("layout_name", ["default", "fast"])
def test_config4_full_length(device, layout_name):
    """64 q / 8 kv heads, 131072 tokens, Student-t K.  Over 131072
    tokens the fp16 x*x of some pair of every kv head overflows, so every kv
    head holds +inf radii (fast layout: +inf page scales) and the reference's
    CPU path returns NaN for every query head; the kernel must return exactly
    the reference's NaN / +-inf pattern."""
    S = 2048
    print(f"[config4] layout={layout_name} S={S}", flush=True)
    block, qv, host, tk, tv, q = build_case(device, LAYOUTS[layout_name], 64, 8, S, 0, seed=7, kind="studentt",
                                            qscale=1.0 / np.sqrt(128.0))
    seq = S * PAGE
    ref = oracle_by_head(host, tk, tv, q, seq, 8)
    out = run_gpu(device, block, qv, tk, tv, q, seq)
    nan_heads = sorted({int(h) for h in np.nonzero(np.isnan(ref))[1]})
    print(f"[config4] {layout_name}: {len(nan_heads)} of 64 query heads NaN in the reference", flush=True)
    assert np.array_equal(np.isnan(out), np.isnan(ref)), "NaN positions differ"
    assert np.array_equal(np.isposinf(out), np.isposinf(ref)), "+inf positions differ"
    assert np.array_equal(np.isneginf(out), np.isneginf(ref)), "-inf positions differ"
    fin = np.isfinite(ref)
    if fin.any():
        check(out[fin], ref[fin], f"config4 {layout_name} finite outputs")


@pytest.mark.parametrize("layout_name", ["default", "fast"])
def test_config4_shape_finite(device, layout_name):
    """configs[4]'s shape and split-K reduction (64 q / 8 kv heads, GQA 8,
    131072 tokens, 32 splits of 64 pages per kv head) with finite outputs:
    the same Student-t(3) x log-uniform [0.1, 10] K clipped to +-200, so no
    fp16 x*x overflows while the heavy tail (|K| up to 200) stays, against the
    oracle at the north_star tolerance."""
    S = 2048
    k, v = gen_kv(8, 1, 8, S * PAGE, "studentt", np.float16)
    k = np.clip(k.astype(np.float32), -200.0, 200.0).astype(np.float16)
    q = gen_q(8, 1, 64, 1.0 / np.sqrt(128.0))
    layout = LAYOUTS[layout_name]
    print(f"[config4-finite] layout={layout_name}", flush=True)
    host = encode_gpu(k, v, layout, device)
    host["metadata"] = oracle.encode_block(k[:, :, :PAGE], l1_bits=layout[1], deep_bits=layout[2],
                                           split_dim=layout[3], use_int8_radii=layout[0])["metadata"]
    from test_gpu_attention import PolarKeyBlock, QuantizedVBlock
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    block = PolarKeyBlock(radii=t(host["radii"]), angle_codes_l1=t(host["angle_codes_l1"]),
                          angle_codes_deep=t(host["angle_codes_deep"]), shape=(1, 8, S * PAGE, 128), block_size=PAGE,
                          head_dim=128, metadata=host["metadata"],
                          radii_scales=t(host["radii_scales"]) if layout[0] else None)
    qvb = QuantizedVBlock(codes=t(host["v_codes"]), scales=t(host["v_scales"]), group_size=32)
    empty = np.zeros((1, 8, 0, 128), np.float16)
    out = run_gpu(device, block, qvb, empty, empty, q, S * PAGE)
    check(out, oracle_by_head(host, empty, empty, q, S * PAGE, 8), f"config4 finite {layout_name}")


def test_config1_layers_through_runtime(device):
    """the full 16-layer step.  32768 tokens of log-uniform K per
    layer, appended in bulk to one runtime per layer, then one decode query
    per layer through the kernel bridge with a dense tail of 5 tokens; the
    layers share the bridge's split-K workspace and run back to back before
    any result is read, and every layer's output is checked against the
    oracle."""
    from turbopolar_amd import HipKernelBridge, TurboPolarConfig, TurboPolarKVCacheRuntime

    n_layers, T = 16, 32768 + 5
    S = 512
    cfg = TurboPolarConfig(num_q_heads=32, num_kv_heads=8)
    bridge = HipKernelBridge()
    layers = []
    k0 = v0 = None
    for layer in range(n_layers):
        print(f"[config1] layer {layer}: append {T} tokens", flush=True)
        k, v = gen_kv(100 + layer, 1, 8, T, "loguniform", np.float16)
        rt = TurboPolarKVCacheRuntime(cfg)
        rt.append(torch.from_numpy(k).to(device), torch.from_numpy(v).to(device))
        q = gen_q(100 + layer, 1, 32, 1.0 / np.sqrt(128.0))
        if layer == 0:
            k0, v0 = k[:, :, :S * PAGE], v[:, :, :S * PAGE]
        # only the dense tail's tokens are needed on the host from here on
        layers.append((rt, np.ascontiguousarray(k[:, :, S * PAGE:]), np.ascontiguousarray(v[:, :, S * PAGE:]), q))
        del k, v
    outs = []
    for rt, k, v, q in layers:
        block, qv, tk, tv, _, seq = rt.get_fused_attention_inputs()
        out, trace = bridge.execute_online_attention_quant_v_dense_tail(
            torch.from_numpy(q).to(device), block, qv, tk, tv, None, None, cfg, seq)
        assert trace["hip_used"] and not trace["fallback_used"] and trace["tail_length"] == 5
        outs.append(out)
    torch.cuda.synchronize()
    for layer, ((rt, k_tail, v_tail, q), out) in enumerate(zip(layers, outs)):
        print(f"[config1] layer {layer}: oracle check", flush=True)
        block, qv, tk, tv, _, seq = rt.get_fused_attention_inputs()
        host = {
            "radii": block.radii.cpu().numpy(), "radii_scales": None,
            "angle_codes_l1": block.angle_codes_l1.cpu().numpy(),
            "angle_codes_deep": block.angle_codes_deep.cpu().numpy(),
            "v_codes": qv.codes.cpu().numpy(), "v_scales": qv.scales.cpu().numpy(), "metadata": block.metadata,
        }
        assert host["radii"].shape[2] == S and seq == T
        # the pages the runtime stored are the oracle encoder's pages of the same tokens
        if layer == 0:
            blk, (vc, vs) = oracle_pages(k0, v0, LAYOUTS["default"])
            assert_bits_equal(host["radii"], blk["radii"], "radii")
            assert_bits_equal(host["angle_codes_l1"], blk["angle_codes_l1"], "l1")
            assert_bits_equal(host["angle_codes_deep"], blk["angle_codes_deep"], "deep")
            assert_bits_equal(host["v_codes"], vc, "v_codes")
            assert_bits_equal(host["v_scales"], vs, "v_scales")
        ref = oracle_by_head(host, k_tail, v_tail, q, T, 8)
        check(out.float().cpu().numpy(), ref, f"config1 layer {layer}")
        del host, ref


def test_config3_bulk_encode_full_size(device):
    """configs[3] workload 1: 32768 fp16 tokens x 8 kv heads (seed 3) into 512
    pages per head in one launch, bit-exact against the oracle encoder in the
    default and the fast layout."""
    k, v = gen_kv(3, 1, 8, 32768, "normal", np.float16)
    for name in ("default", "fast"):
        print(f"[config3] bulk encode {name}", flush=True)
        layout = LAYOUTS[name]
        gpu = encode_gpu(k, v, layout, device)
        blk, (vc, vs) = oracle_pages(k, v, layout)
        assert_bits_equal(gpu["radii"], blk["radii"], "radii")
        if layout[0]:
            assert_bits_equal(gpu["radii_scales"], blk["radii_scales"].reshape(gpu["radii_scales"].shape),
                              "radii_scales")
        assert_bits_equal(gpu["angle_codes_l1"], blk["angle_codes_l1"], "l1")
        assert_bits_equal(gpu["angle_codes_deep"], blk["angle_codes_deep"], "deep")
        assert_bits_equal(gpu["v_codes"], vc, "v_codes")
        assert_bits_equal(gpu["v_scales"], vs, "v_scales")


def test_config3_sequential_appends(device):
    """configs[3] workload 2: 4096 single-token appends (8 kv heads, seed 3)
    complete 64 pages; the runtime's storage, tail and counters equal those of
    one bulk append of the same tokens, and the pages equal the oracle's."""
    from turbopolar_amd import TurboPolarConfig, TurboPolarKVCacheRuntime

    cfg = TurboPolarConfig(num_q_heads=32, num_kv_heads=8)
    k, v = gen_kv(3, 1, 8, 4096 + 3, "normal", np.float16)
    kd, vd = torch.from_numpy(k).to(device), torch.from_numpy(v).to(device)
    seq_rt = TurboPolarKVCacheRuntime(cfg)
    print("[config3] 4099 single-token appends", flush=True)
    for t in range(k.shape[2]):
        seq_rt.append(kd[:, :, t:t + 1].contiguous(), vd[:, :, t:t + 1].contiguous())
    bulk_rt = TurboPolarKVCacheRuntime(cfg)
    bulk_rt.append(kd, vd)
    a = seq_rt.get_fused_attention_inputs()
    b = bulk_rt.get_fused_attention_inputs()
    assert a[5] == b[5] == 4099
    for x, y, what in ((a[0].radii, b[0].radii, "radii"), (a[0].angle_codes_l1, b[0].angle_codes_l1, "l1"),
                       (a[0].angle_codes_deep, b[0].angle_codes_deep, "deep"), (a[1].codes, b[1].codes, "codes"),
                       (a[1].scales, b[1].scales, "scales"), (a[2], b[2], "tail_k"), (a[3], b[3], "tail_v")):
        assert torch.equal(x, y), what
    blk, (vc, vs) = oracle_pages(k[:, :, :4096], v[:, :, :4096], LAYOUTS["default"])
    assert_bits_equal(a[0].radii.cpu().numpy(), blk["radii"], "radii vs oracle")
    assert_bits_equal(a[1].codes.cpu().numpy(), vc, "v_codes vs oracle")
    assert_bits_equal(a[1].scales.cpu().numpy(), vs, "v_scales vs oracle")
    ta, tb = seq_rt.get_io_telemetry(), bulk_rt.get_io_telemetry()
    for key in ("total_blocks", "partial_tokens", "actual_cache_bytes", "compression_ratio"):
        assert ta[key] == tb[key], key
