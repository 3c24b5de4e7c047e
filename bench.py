"""Decode-attention benchmark on one MI355X (BASELINE.json metric).

One step = one fused decode-attention launch (tp_decode_attention) over a
Llama-3-8B-shape cache: 32 query heads, 8 kv heads, head_dim 128, 32768 tokens
(512 pages of 64 per kv head), TurboPolarConfig() default layout, batch 1
(BASELINE configs[2] at 32k).  Inputs are synthetic:
K fp16 N(0,1) with 4 outlier channels x20 per head, V fp16 N(0,1),
q fp16 N(0,1)/sqrt(128).  The caches are encoded on the GPU by the same
library before timing and stay resident in HBM.  Steps rotate over enough
independent caches (> 256 MB in total) that the MI355X Infinity Cache cannot
hold them, so the timed reads come from HBM.

Prints one JSON line.  ``value`` is microseconds per decode step (lower is
better); ``roofline.achieved`` is the algorithmic compressed bytes per step
(get_io_telemetry()["actual_cache_bytes"] + q + out) over the measured
average step time.  The CPU baseline is the oracle's NumPy restatement of the
reference CPU fallback (_cpu_online_attention_dense_tail), timed on a bounded
sample on this host.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBPS = 8000.0
# Decode-kernel variants of the measurement library (tp_measure_set_decode_variant).
VARIANTS = {"mfma": 0, "release": 1, "valu": 2, "valu+release": 3, "no-acquire": 4}
METRIC = "decode-attn µs/step + achieved HBM GB/s (% peak), Llama-3-8B shape, 32k ctx"
LAYOUTS = {"default": (False, 4, 4, 64), "fast": (True, 4, 8, 0)}


def algorithmic_bytes(hq, hkv, n_pages, layout, tail=0):
    int8 = layout[0]
    kb = 128 if layout == LAYOUTS["fast"] else None
    if kb is None:
        split_half = layout[3] // 2
        l1 = {4: (split_half + 1) // 2, 8: split_half}[layout[1]]
        deep = {8: 64 - split_half, 4: (64 - split_half + 1) // 2, 2: (64 - split_half + 3) // 4}[layout[2]]
        kb = (64 if int8 else 128) + l1 + deep
    rs = 2 if int8 else 0
    return hkv * n_pages * 64 * (kb + 136) + hkv * n_pages * rs + hkv * tail * 512 + hq * 128 * 2 * 2


def workload_name(args):
    shape = {(32, 8): ("llama3-8b-shape", "configs[2]"), (64, 8): ("llama3-70b-shape", "configs[4]")}
    name, cfg = shape.get((args.hq, args.hkv), (f"{args.hq}q/{args.hkv}kv", "not a BASELINE config"))
    if (args.hq, args.hkv, args.context) == (32, 8, 4096):
        name, cfg = "llama3.2-1b-shape", "configs[0]"
    tail = getattr(args, "tail", 0)
    ctx = f"{args.context} ctx" + (f" + {tail} dense tail tokens" if tail else "")
    return f"{name} single-layer decode attention, {ctx}, K {args.kind} (BASELINE {cfg})"


def synthetic_k(kind, hkv, tokens, g, dev):
    """K of the BASELINE configs, fp32 ``[1, hkv, tokens, 128]``: ``outlier``
    N(0,1) with 4 channels x20 per head; ``loguniform`` N(0,1) x
    per-channel scales log-uniform in [0.25, 4]; ``studentt``
    t(3) x per-channel scales log-uniform in [0.1, 10];
    ``normal`` N(0,1) (configs[0], [3])."""
    import torch

    k = torch.randn((1, hkv, tokens, 128), generator=g, device=dev, dtype=torch.float32)
    if kind == "outlier":
        for h in range(hkv):
            ch = torch.randperm(128, generator=g, device=dev)[:4]
            k[:, h, :, ch] *= 20.0
    elif kind in ("loguniform", "studentt"):
        lo, hi = (0.25, 4.0) if kind == "loguniform" else (0.1, 10.0)
        u = torch.rand((1, hkv, 1, 128), generator=g, device=dev)
        c = torch.exp(np.log(lo) + u * (np.log(hi) - np.log(lo)))
        if kind == "studentt":
            # t(3) = N(0,1) / sqrt(chi2(3) / 3), chi2(3) a sum of three squared normals
            chi2 = sum(torch.randn(k.shape, generator=g, device=dev) ** 2 for _ in range(3))
            k = k / torch.sqrt(chi2 / 3.0)
        k = k * c
    elif kind != "normal":
        raise ValueError(kind)
    return k


def build_caches(args, dev, layout):
    import torch

    from turbopolar_amd import TurboPolarConfig, TurboPolarKVCacheRuntime
    from turbopolar_amd.kernels import PageSet

    int8, l1b, deepb, split = layout
    cfg = TurboPolarConfig(num_q_heads=args.hq, num_kv_heads=args.hkv, use_int8_radii=int8,
                           k_angle_bits_level1=l1b, k_angle_bits_deep=deepb, split_dim=split)
    caches = []
    kind = getattr(args, "kind", "outlier")
    tail = getattr(args, "tail", 0)
    for r in range(args.rotate):
        g = torch.Generator(device=dev).manual_seed(1000 + r)
        k = synthetic_k(kind, args.hkv, args.context + tail, g, dev)
        v = torch.randn((1, args.hkv, args.context + tail, 128), generator=g, device=dev, dtype=torch.float32)
        rt = TurboPolarKVCacheRuntime(cfg)
        rt.append(k.half(), v.half())
        v_dense = None
        if getattr(args, "dense_v", False):
            # The same V rows, dense fp16 [1, hkv, pages, 64, 128]: the dense-V
            # attention reads these in place of the runtime's quantised pages.
            v_dense = v.half().reshape(1, args.hkv, args.context // 64, 64, 128).contiguous()
        del k, v
        block, qv, tk, tv, _, seq = rt.get_fused_attention_inputs()
        q = (torch.randn((1, args.hq, 128), generator=g, device=dev) / np.sqrt(128.0)).half()
        c = {"rt": rt, "pages": PageSet(block, qv), "q": q, "seq": seq,
             "out": torch.empty((1, args.hq, 128), dtype=torch.float16, device=dev),
             "tail": (None, None, 0, 0), "v_dense": v_dense}
        if tail:
            from turbopolar_amd.kernels import _tail_view

            (tkv, stride), (tvv, stride_v) = _tail_view(tk), _tail_view(tv)
            if stride != stride_v or tkv.shape[2] != tail:
                raise RuntimeError("the runtime's tail views do not share one layout")
            c["tail"] = (tkv, tvv, tail, stride)
        caches.append(c)
    torch.cuda.synchronize()
    return cfg, caches


def run_gpu(args, layout):
    import torch

    from turbopolar_amd import _lib
    from turbopolar_amd.kernels import fp16_scale

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg, caches = build_caches(args, dev, layout)
    L = _lib.lib()
    n_pages = caches[0]["pages"].S
    pps = args.pps or int(L.tp_default_pages_per_split(1, args.hq, args.hkv, n_pages))
    need = int(L.tp_decode_workspace_bytes(1, args.hq, args.hkv, n_pages, getattr(args, "tail", 0), pps))
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    scale = fp16_scale(cfg.attention_scale)
    stream = torch.cuda.current_stream(dev).cuda_stream
    fn = L.tp_decode_attention
    calls = []
    for i, c in enumerate(caches):
        ps = c["pages"]
        if getattr(args, "qjl", False):
            # Synthetic sketches of the pages' residuals (random bits and norms:
            # the kernel's work does not depend on their values) and of q.
            from turbopolar_amd.qjl import QJLPages, QJLPayload

            g = torch.Generator(device=dev).manual_seed(77 + i)
            signs = torch.randint(0, 256, (1, args.hkv, n_pages, 64, 8), generator=g, device=dev, dtype=torch.uint8)
            norms = (torch.rand((1, args.hkv, n_pages, 64), generator=g, device=dev) * 0.1).half()
            qsig = torch.randint(0, 256, (1, args.hq, 8), generator=g, device=dev, dtype=torch.uint8)
            c["qjl"] = QJLPages(QJLPayload(signs, norms, 64, 42, (1, args.hkv, n_pages, 64, 128)), qsig)
            fn = L.tp_decode_attention_qjl
            calls.append((c["q"].data_ptr(), 1, args.hq, args.hkv, ctypes.byref(ps.layout), ctypes.byref(ps.pages),
                          n_pages, ctypes.byref(c["qjl"].desc), None, None, 0, 0, c["seq"], scale, pps,
                          ws.data_ptr(), need, c["out"].data_ptr(), stream))
            continue
        if getattr(args, "dense_v", False):
            fn = L.tp_decode_attention_dense_v
            calls.append((c["q"].data_ptr(), 1, args.hq, args.hkv, ctypes.byref(ps.layout), ctypes.byref(ps.pages),
                          n_pages, None, c["v_dense"].data_ptr(), n_pages, c["seq"], scale, pps, ws.data_ptr(), need,
                          c["out"].data_ptr(), stream))
            continue
        tkv, tvv, tlen, tstride = c["tail"]
        calls.append((c["q"].data_ptr(), 1, args.hq, args.hkv, ctypes.byref(ps.layout), ctypes.byref(ps.pages),
                      n_pages, tkv.data_ptr() if tlen else None, tvv.data_ptr() if tlen else None, tlen, tstride,
                      c["seq"], scale, pps, ws.data_ptr(), need, c["out"].data_ptr(), stream))

    def step(i):
        st = fn(*calls[i % len(calls)])
        if st:
            _lib.check(st, "tp_decode_attention")

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    graph_equal = None
    if getattr(args, "graph", False):
        # The timed launches captured once into a HIP graph (the same calls on
        # the capture stream) and timed as one replay: the GPU runs them back
        # to back without waiting for the host's launch path.
        eager = [c["out"].clone() for c in caches]
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            cap = torch.cuda.current_stream(dev).cuda_stream
            for i in range(args.steps):
                st = fn(*calls[i % len(calls)][:-1], cap)
                if st:
                    _lib.check(st, "tp_decode_attention")
        graph_equal = True
        for _ in range(3):  # replays between eager launches and syncs must match the eager outputs
            for c in caches:
                c["out"].zero_()
            graph.replay()
            torch.cuda.synchronize()
            covered = range(min(args.steps, len(caches)))  # the caches the captured launches write
            graph_equal &= all(torch.equal(caches[k]["out"], eager[k]) for k in covered)
            step(0)
            torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    if graph_equal is not None:
        graph.replay()
    else:
        for i in range(args.steps):
            step(i)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps

    # Determinism guard on the timed configuration: the first cache's output
    # from the timed launches against one more launch of the same call.
    ref_out = caches[0]["out"].clone()
    step(0)
    torch.cuda.synchronize()
    ok = bool(torch.isfinite(caches[0]["out"]).all())
    return {"ms": ms, "pps": pps, "n_pages": n_pages, "finite": ok, "cfg": cfg, "caches": caches,
            "ws_bytes": need, "rerun_equal": bool(torch.equal(ref_out, caches[0]["out"])), "graph_equal": graph_equal}


def host_cores() -> int:
    """Host threads the CPU baselines use: every core this process may run on
    (its CPU affinity), or ``TP_BENCH_CPU_THREADS`` when set."""
    env = os.environ.get("TP_BENCH_CPU_THREADS")
    if env:
        return max(1, int(env))
    return affinity_cores()


def affinity_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


def cgroup_cpu_quota():
    """CPUs' worth of time the process's cgroup grants (cgroup v2 cpu.max), or
    None when unlimited or unknown."""
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()
        return None if quota == "max" else round(int(quota) / int(period), 2)
    except (OSError, ValueError):
        return None


class _OneBlasThread:
    """BLAS and OpenMP pools at one thread inside (the baselines' own thread
    pools carry the parallelism)."""

    def __enter__(self):
        try:
            from threadpoolctl import threadpool_limits
            self._ctx = threadpool_limits(1)
        except ImportError:  # pragma: no cover
            self._ctx = None
        return self

    def __exit__(self, *exc):
        if self._ctx is not None:
            self._ctx.__exit__(*exc)


def _chunks(n: int, parts: int):
    """[0, n) cut into at most ``parts`` contiguous ranges."""
    parts = max(1, min(parts, n))
    edges = [n * i // parts for i in range(parts + 1)]
    return [(edges[i], edges[i + 1]) for i in range(parts) if edges[i] < edges[i + 1]]


def _sample(fn, budget_s: float, min_runs: int = 2):
    """Median wall time of repeated ``fn()`` calls for about ``budget_s``
    seconds (at least ``min_runs`` calls) and the last result."""
    times, out = [], None
    start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        out = fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - start > budget_s and len(times) >= min_runs:
            break
    return float(np.median(times)), len(times), out


def cpu_attention_all_cores(oracle, pool, cores, q, blk, qv, scale, seq, tail_k, tail_v):
    """The oracle's _cpu_online_attention_dense_tail (metal.py:293-332) spread
    over ``pool``: K decode and V dequantisation per (kv head, page range),
    the dense tail after the pages, then the float32 masked softmax attention
    per kv head.  Every element takes the oracle's own arithmetic; only the
    work is divided."""
    codes, scales = qv
    B, H, S, L, D = codes.shape
    T = tail_k.shape[2]
    k = np.empty((B, H, S * L + T, D), np.float16)
    v = np.empty((B, H, S * L + T, D), np.float16)
    k[:, :, S * L:] = tail_k
    v[:, :, S * L:] = tail_v
    rs = blk["radii_scales"]

    def dec(h, p0, p1):
        hs, ps, ts = slice(h, h + 1), slice(p0, p1), slice(p0 * L, p1 * L)
        k[:, hs, ts] = oracle.decode_block(blk["radii"][:, hs, ps], None if rs is None else rs[:, hs, ps],
                                           blk["angle_codes_l1"][:, hs, ps], blk["angle_codes_deep"][:, hs, ps],
                                           blk["metadata"])
        v[:, hs, ts] = oracle.dequantize_block(codes[:, hs, ps], scales[:, hs, ps]).reshape(B, 1, (p1 - p0) * L, D)

    parts = max(1, -(-4 * cores // H))
    list(pool.map(lambda t: dec(*t), [(h, p0, p1) for h in range(H) for p0, p1 in _chunks(S, parts)]))
    g = q.shape[1] // H
    out = np.empty(q.shape, np.float32)

    def att(h):
        out[:, h * g:(h + 1) * g] = oracle.softmax_attention(q[:, h * g:(h + 1) * g], k[:, h:h + 1], v[:, h:h + 1],
                                                             scale, seq, dtype=np.float32)

    list(pool.map(att, range(H)))
    return out


def cpu_baseline(args, layout, caches, budget_s):
    """The oracle's restatement of the reference CPU fallback
    (_cpu_online_attention_dense_tail, metal.py:293-332) on one cache, float32:
    on every host core the process may use (``host_cores``), and once more on
    one thread for comparison with single-core figures."""
    from concurrent.futures import ThreadPoolExecutor

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import oracle
    from turbopolar_amd.kernels import fp16_scale

    c = caches[0]
    ps = c["pages"]
    t = ps.tensors
    blk = {
        "radii": t["radii"].cpu().numpy(),
        "radii_scales": t["radii_scales"].cpu().numpy() if "radii_scales" in t else None,
        "angle_codes_l1": t["angle_l1"].cpu().numpy(),
        "angle_codes_deep": t["angle_deep"].cpu().numpy(),
        "metadata": c["rt"].k_storage.metadata,
    }
    qv = (t["v_codes"].cpu().numpy(), t["v_scales"].cpu().numpy())
    q = c["q"].cpu().numpy()
    tkv, tvv, tlen, _ = c["tail"]
    tail_k = tkv.cpu().numpy() if tlen else np.zeros((1, args.hkv, 0, 128), np.float16)
    tail_v = tvv.cpu().numpy() if tlen else np.zeros((1, args.hkv, 0, 128), np.float16)
    scale = fp16_scale(1.0 / np.sqrt(128.0))
    cores = host_cores()
    with _OneBlasThread(), ThreadPoolExecutor(cores) as pool:
        t_all, n_all, out = _sample(lambda: cpu_attention_all_cores(oracle, pool, cores, q, blk, qv, scale, c["seq"],
                                                                    tail_k, tail_v), budget_s)
    t16 = n16 = None
    if cores != 16:
        # The 16-thread figure of earlier runs (one GPU's share of a GPU box's
        # host), beside the all-core one.
        with _OneBlasThread(), ThreadPoolExecutor(16) as pool:
            t16, n16, _ = _sample(lambda: cpu_attention_all_cores(oracle, pool, 16, q, blk, qv, scale, c["seq"],
                                                                  tail_k, tail_v), budget_s / 4)
    with _OneBlasThread():
        t_one, n_one, out1 = _sample(lambda: oracle.cpu_online_attention_dense_tail(
            q, blk, qv, tail_k, tail_v, scale, c["seq"], dtype=np.float32), budget_s / 4)
    gpu = c["out"].float().cpu().numpy()
    return {"us": t_all * 1e6, "runs": n_all, "cores": cores, "err": float(np.max(np.abs(gpu - out))),
            "one_thread_us": t_one * 1e6, "one_thread_runs": n_one,
            "same_as_one_thread": bool(np.array_equal(out, out1)),
            "sixteen_us": None if t16 is None else t16 * 1e6, "sixteen_runs": n16}


def run_layers(args, layout) -> dict:
    """one decode query per layer over ``args.layers``
    layer caches of ``args.context`` tokens each (K log-uniform per channel);
    a step launches every layer once, in order, on one stream.  With
    ``args.graph`` the step's launches are captured once into a HIP graph and a
    step is one replay."""
    import torch

    from turbopolar_amd import _lib
    from turbopolar_amd.kernels import fp16_scale

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    args.rotate = args.layers
    cfg, caches = build_caches(args, dev, layout)
    L = _lib.lib()
    n_pages = caches[0]["pages"].S
    pps = args.pps or int(L.tp_default_pages_per_split(1, args.hq, args.hkv, n_pages))
    need = int(L.tp_decode_workspace_bytes(1, args.hq, args.hkv, n_pages, 0, pps))
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    scale = fp16_scale(cfg.attention_scale)
    fn = L.tp_decode_attention

    def step():
        stream = torch.cuda.current_stream(dev).cuda_stream
        for c in caches:
            ps = c["pages"]
            st = fn(c["q"].data_ptr(), 1, args.hq, args.hkv, ctypes.byref(ps.layout), ctypes.byref(ps.pages),
                    n_pages, None, None, 0, 0, c["seq"], scale, pps, ws.data_ptr(), need, c["out"].data_ptr(), stream)
            if st:
                _lib.check(st, "tp_decode_attention")

    step()
    torch.cuda.synchronize()
    eager = [c["out"].clone() for c in caches]
    run = step
    graph_equal = None
    if args.graph:
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph):
            step()
        run = graph.replay
        graph_equal = True
        for _ in range(3):  # replays interleaved with eager work and syncs must all match eager
            for c in caches:
                c["out"].zero_()
            graph.replay()
            torch.cuda.synchronize()
            graph_equal &= all(torch.equal(c["out"], e) for c, e in zip(caches, eager))
            step()
            torch.cuda.synchronize()
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(args.steps):
        run()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    ok = all(bool(torch.isfinite(c["out"]).all()) and torch.equal(c["out"], e) for c, e in zip(caches, eager))
    return {"ms": ms, "pps": pps, "n_pages": n_pages, "outputs_match_first_step": ok, "graph_equal": graph_equal}


def _gpu_busy_ms(step, n: int):
    """Sum of the device kernel durations of one ``step()`` (median over ``n``
    profiled steps, torch.profiler's device activity), in ms; None if the
    profiler gives no device events here."""
    import torch

    try:
        from torch.profiler import ProfilerActivity, profile
        per = []
        for _ in range(n):
            with profile(activities=[ProfilerActivity.CPU, ProfilerActivity.CUDA]) as prof:
                with torch.no_grad():
                    step()
                torch.cuda.synchronize()
            us = sum(e.time_range.elapsed_us() for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA)
            per.append(us / 1e3)
        busy = float(np.median(per))
        return round(busy, 3) if busy > 0 else None
    except Exception:  # pragma: no cover - profiler unavailable
        return None


def run_model(args) -> dict:
    """§8 f2: decode through a randomly initialised Llama of the configs[1]
    shape (``args.layers`` layers, ``args.hq`` / ``args.hkv`` heads, head_dim
    128, float32 weights) with the transformers hook, its caches pre-filled
    with ``args.context`` synthetic tokens per layer; the same tokens run
    through the model's own DynamicCache as the dense baseline
    (run_fast_attention_bench.py:104-121: tokens/s of greedy decode; here the
    tokens are teacher-forced so both runs see the same inputs)."""
    import torch
    from transformers import DynamicCache, LlamaConfig, LlamaForCausalLM

    from turbopolar_amd import llama as tl

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.model_path:
        # A local checkpoint (run_fast_attention_bench.py:155 loads its --model
        # the same way, by path), in the dtype it was saved in; its shape
        # replaces --layers / --hq / --hkv.
        model = tl.load_local_llama(args.model_path, device=dev, dtype="auto", patch=False)
        cfg = model.config
        head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        if head_dim != 128:
            raise SystemExit(f"--model-path: the decode kernel takes head_dim 128, the checkpoint has {head_dim}")
        args.layers, args.hq = cfg.num_hidden_layers, cfg.num_attention_heads
        args.hkv = getattr(cfg, "num_key_value_heads", None) or args.hq
    else:
        cfg = LlamaConfig(vocab_size=128256, hidden_size=args.hq * 128, intermediate_size=8192,
                          num_hidden_layers=args.layers, num_attention_heads=args.hq, num_key_value_heads=args.hkv,
                          head_dim=128, max_position_embeddings=args.context + 4096, attn_implementation="eager")
        torch.manual_seed(0)
        with torch.device(dev):
            model = LlamaForCausalLM(cfg).eval()
    turbo = tl.make_turbo_cache(model)
    dense = DynamicCache(config=model.config)
    g = torch.Generator(device=dev).manual_seed(7)
    with torch.no_grad():
        for layer in range(args.layers):
            k = synthetic_k("loguniform", args.hkv, args.context, g, dev).half()
            v = torch.randn(k.shape, generator=g, device=dev).half()
            turbo.fast(layer).runtime.append(k, v)
            dense.update(k.to(model.dtype), v.to(model.dtype), layer)
            del k, v
    tokens = torch.randint(0, cfg.vocab_size, (1, args.warmup + args.steps), generator=g, device=dev)
    res = {}
    logits = {}
    busy = {}
    for name, cache in (("dense", dense), ("turbo", turbo)):
        if name == "turbo":
            tl.patch_llama_attention(model)
        try:
            with torch.no_grad():
                outs = []
                for i in range(args.warmup):
                    model(tokens[:, i:i + 1], past_key_values=cache, use_cache=True)
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for i in range(args.warmup, args.warmup + args.steps):
                    outs.append(model(tokens[:, i:i + 1], past_key_values=cache, use_cache=True).logits[0, -1])
                torch.cuda.synchronize()
                res[name] = (time.perf_counter() - t0) / args.steps
                logits[name] = torch.stack(outs).double()
                # three more steps (after the timed ones) under the profiler
                busy[name] = _gpu_busy_ms(lambda: model(tokens[:, -1:], past_key_values=cache, use_cache=True), 3)
        finally:
            tl.unpatch_llama_attention(model)
    a, b = logits["turbo"], logits["dense"]
    cos = torch.nn.functional.cosine_similarity(a, b, dim=-1)
    top1 = (a.argmax(-1) == b.argmax(-1)).double().mean()
    return {"weights": str(model.dtype).replace("torch.", ""),
            "turbo_s": res["turbo"], "dense_s": res["dense"], "cos_min": float(cos.min()), "top1": float(top1),
            "turbo_busy_ms": busy.get("turbo"), "dense_busy_ms": busy.get("dense"),
            "turbo_bytes": int(turbo.nbytes), "dense_bytes": int(sum(x.numel() * x.element_size() for x in (
                *[layer.keys for layer in dense.layers], *[layer.values for layer in dense.layers])))}


def run_decompress(args, layout) -> dict:
    """§8 f1 decompress-on-read: one tp_decode_pages launch per step turns
    every page of a 32k cache (8 kv heads, 512 pages) back into dense fp16 K
    and V [1, 8, 32768, 128], as update_and_fetch does before prefill
    attention.  Three rotating caches, so the reads come from HBM."""
    import torch

    from turbopolar_amd import _lib

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    args.rotate = 3
    _, caches = build_caches(args, dev, layout)
    L = _lib.lib()
    n_pages = caches[0]["pages"].S
    k_out = torch.empty((1, args.hkv, n_pages * 64, 128), dtype=torch.float16, device=dev)
    v_out = torch.empty_like(k_out)
    stream = torch.cuda.current_stream(dev).cuda_stream

    def step(i):
        ps = caches[i % len(caches)]["pages"]
        st = L.tp_decode_pages(ctypes.byref(ps.layout), ctypes.byref(ps.pages), args.hkv, 0, n_pages,
                               k_out.data_ptr(), v_out.data_ptr(), stream)
        if st:
            _lib.check(st, "tp_decode_pages")

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(args.steps):
        step(i)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    read = algorithmic_bytes(args.hq, args.hkv, n_pages, layout) - args.hq * 128 * 4
    write = 2 * k_out.numel() * 2
    step(0)  # the outputs of cache 0, for the CPU baseline's check
    torch.cuda.synchronize()
    return {"ms": ms, "read": read, "write": write, "n_pages": n_pages, "cache0": caches[0], "k_out": k_out,
            "v_out": v_out}


PREFILL_TAIL = 37  # tokens left in the dense tail before and after every prefill step


def run_prefill(args, layout) -> dict:
    """Prefill with a tail: TurboPolarFastCache.update_and_fetch
    (turbopolar_fast_attention.py:56-86) of a 64-token chunk over a cache of
    ``context`` + 37 tokens.  Each step appends the chunk (one page encoded,
    the 37-token tail kept), decodes every stored page and the zero-padded tail
    page in place into the dense fp16 K and V it returns.  The cache grows by
    64 tokens a step; the timed region is ``steps`` whole calls, host work
    included (wall clock, synchronised at both ends)."""
    import torch

    from turbopolar_amd import TurboPolarConfig
    from turbopolar_amd.fast_attention import TurboPolarFastCache

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    int8, l1b, deepb, split = layout
    cfg = TurboPolarConfig(num_q_heads=args.hq, num_kv_heads=args.hkv, use_int8_radii=int8,
                           k_angle_bits_level1=l1b, k_angle_bits_deep=deepb, split_dim=split)
    g = torch.Generator(device=dev).manual_seed(11)
    cache = TurboPolarFastCache(cfg)
    t0 = args.context + PREFILL_TAIL
    k0 = synthetic_k(args.kind, args.hkv, t0, g, dev).half()
    v0 = torch.randn((1, args.hkv, t0, 128), generator=g, device=dev).half()
    k, v = cache.update_and_fetch(k0, v0)
    if k.shape[2] != t0 or cache.runtime._tail_len != PREFILL_TAIL:
        raise RuntimeError("prefill returned the wrong length")
    del k0, v0, k, v
    n_chunks = args.warmup + args.steps
    ck = synthetic_k(args.kind, args.hkv, 64 * n_chunks, g, dev).half()
    cv = torch.randn((1, args.hkv, 64 * n_chunks, 128), generator=g, device=dev).half()
    for i in range(args.warmup):
        cache.update_and_fetch(ck[:, :, 64 * i:64 * (i + 1)], cv[:, :, 64 * i:64 * (i + 1)])
    torch.cuda.synchronize()
    first = cache.offset + 64
    start = time.perf_counter()
    for i in range(args.warmup, n_chunks):
        k, v = cache.update_and_fetch(ck[:, :, 64 * i:64 * (i + 1)], cv[:, :, 64 * i:64 * (i + 1)])
    torch.cuda.synchronize()
    ms = (time.perf_counter() - start) * 1e3 / args.steps
    last = cache.offset
    mid_pages = ((first + last) // 2) // 64
    read = algorithmic_bytes(0, args.hkv, mid_pages, layout) + args.hkv * PREFILL_TAIL * 512 + 2 * args.hkv * 64 * 256
    write = 2 * args.hkv * (mid_pages + 1) * 64 * 256
    tail_ok = cache.runtime._tail_len == PREFILL_TAIL and k.shape[2] == last and bool(torch.isfinite(k).all())
    return {"ms": ms, "first": first, "last": last, "read": read, "write": write, "tail_ok": tail_ok}


def _f16_ulp_gap(a, b) -> int:
    """Largest distance in fp16 ulps between finite elements of a and b."""
    def ordered(x):
        bits = x.view(np.int16).astype(np.int32)
        return np.where(bits < 0, -(bits & 0x7FFF), bits)
    fin = np.isfinite(a) & np.isfinite(b)
    return int(np.max(np.abs(ordered(a) - ordered(b))[fin], initial=0))


def cpu_decompress_baseline(args, r, budget_s):
    """Oracle restatement of decompress-on-read (decode_block +
    dequantize_block, decoder.py:7-67, v_quant/encoder.py:32-38) of the whole
    cache, page ranges spread over every host core (``host_cores``), repeated
    for about ``budget_s`` seconds; the result is compared with the GPU's dense
    K (ulps) and V (bitwise).  Also one page range on one thread, scaled to the
    cache, for comparison with single-core figures."""
    from concurrent.futures import ThreadPoolExecutor

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import oracle

    c = r["cache0"]
    t = c["pages"].tensors
    radii, l1, deep = (t[n].cpu().numpy() for n in ("radii", "angle_l1", "angle_deep"))
    rs = t["radii_scales"].cpu().numpy() if "radii_scales" in t else None
    codes, scales = t["v_codes"].cpu().numpy(), t["v_scales"].cpu().numpy()
    meta = c["rt"].k_storage.metadata
    kg, vg = r["k_out"].cpu().numpy(), r["v_out"].cpu().numpy()
    S = r["n_pages"]
    k = np.empty(kg.shape, np.float16)
    v = np.empty(vg.shape, np.float16)

    def dec(p0, p1):
        ps, ts = slice(p0, p1), slice(64 * p0, 64 * p1)
        k[:, :, ts] = oracle.decode_block(radii[:, :, ps], rs[:, :, ps] if rs is not None else None, l1[:, :, ps],
                                          deep[:, :, ps], meta)
        v[:, :, ts] = oracle.dequantize_block(codes[:, :, ps], scales[:, :, ps]).reshape(k[:, :, ts].shape)

    cores = host_cores()
    ranges = _chunks(S, 4 * cores)
    with _OneBlasThread(), ThreadPoolExecutor(cores) as pool:
        t_all, n_all, _ = _sample(lambda: list(pool.map(lambda pr: dec(*pr), ranges)), budget_s)
        p1 = max(1, S // 16)
        t_one, n_one, _ = _sample(lambda: dec(0, p1), budget_s / 4)
    v_exact = bool(np.array_equal(v.view(np.uint16), vg.view(np.uint16)))
    return {"us": t_all * 1e6, "runs": n_all, "cores": cores, "v_exact": v_exact, "k_ulps": _f16_ulp_gap(k, kg),
            "one_thread_us": t_one * S / p1 * 1e6, "one_thread_sample": f"{n_one} runs over {p1} of {S} pages"}


def k_page_bytes(layout) -> int:
    """Compressed K bytes of one page of one kv head (radii, angle codes, radius scale)."""
    return bench_page_bytes(layout) - 64 * 136


def run_fused_qk(args, layout) -> dict:
    """tp_fused_qk (execute_fused_qk, metal.py:494-530) over every page of the
    cache: fp16 scores of all query heads for all S*64 slots, one launch per
    step, rotating caches as the decode line does."""
    import torch

    from turbopolar_amd import _lib
    from turbopolar_amd.kernels import fp16_scale

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    k_bytes = args.hkv * (args.context // 64) * k_page_bytes(layout)
    args.rotate = max(4, int(np.ceil(320e6 / k_bytes)))  # more than the Infinity Cache holds
    cfg, caches = build_caches(args, dev, layout)
    L = _lib.lib()
    n_pages = caches[0]["pages"].S
    scores = torch.empty((1, args.hq, n_pages * 64), dtype=torch.float16, device=dev)
    scale = fp16_scale(cfg.attention_scale)
    stream = torch.cuda.current_stream(dev).cuda_stream

    def step(i):
        c = caches[i % len(caches)]
        ps = c["pages"]
        st = L.tp_fused_qk(c["q"].data_ptr(), 1, args.hq, args.hkv, ctypes.byref(ps.layout), ctypes.byref(ps.pages),
                           n_pages, scale, scores.data_ptr(), stream)
        if st:
            _lib.check(st, "tp_fused_qk")

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(args.steps):
        step(i)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    step(0)
    torch.cuda.synchronize()
    read = args.hkv * n_pages * k_page_bytes(layout) + args.hq * 128 * 2
    write = args.hq * n_pages * 64 * 2
    return {"ms": ms, "read": read, "write": write, "n_pages": n_pages, "cache0": caches[0], "scores": scores,
            "scale": scale, "n_caches": len(caches)}


def cpu_qk_baseline(args, r, budget_s):
    """Oracle restatement of _cpu_fused_qk (metal.py:254-260) over the whole
    cache in float32, per (kv head, page range) on every host core, repeated
    for about ``budget_s`` seconds, and once on one thread; compared with the
    GPU scores by the reference's own QK test bar (max-abs, cosine)."""
    from concurrent.futures import ThreadPoolExecutor

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import oracle

    c = r["cache0"]
    t = c["pages"].tensors
    blk = {"radii": t["radii"].cpu().numpy(),
           "radii_scales": t["radii_scales"].cpu().numpy() if "radii_scales" in t else None,
           "angle_codes_l1": t["angle_l1"].cpu().numpy(), "angle_codes_deep": t["angle_deep"].cpu().numpy(),
           "metadata": c["rt"].k_storage.metadata}
    S = r["n_pages"]
    for n in ("radii", "radii_scales", "angle_codes_l1", "angle_codes_deep"):
        if blk[n] is not None:
            blk[n] = blk[n][:, :, :S]
    q = c["q"].cpu().numpy()
    H = blk["radii"].shape[1]
    g = q.shape[1] // H
    ref = np.empty((q.shape[0], q.shape[1], S * 64), np.float32)

    def part(h, p0, p1):
        sub = {n: (None if blk[n] is None else blk[n][:, h:h + 1, p0:p1])
               for n in ("radii", "radii_scales", "angle_codes_l1", "angle_codes_deep")}
        sub["metadata"] = blk["metadata"]
        ref[:, h * g:(h + 1) * g, 64 * p0:64 * p1] = oracle.cpu_fused_qk(q[:, h * g:(h + 1) * g], sub, r["scale"],
                                                                         dtype=np.float32)

    cores = host_cores()
    tasks = [(h, p0, p1) for h in range(H) for p0, p1 in _chunks(S, max(1, -(-4 * cores // H)))]
    with _OneBlasThread(), ThreadPoolExecutor(cores) as pool:
        t_all, n_all, _ = _sample(lambda: list(pool.map(lambda a: part(*a), tasks)), budget_s)
        t_one, n_one, one = _sample(lambda: oracle.cpu_fused_qk(q, blk, r["scale"], dtype=np.float32), budget_s / 4)
    g_ = r["scores"].float().cpu().numpy().reshape(ref.shape)
    err = float(np.max(np.abs(g_ - ref)))
    cos = float(np.sum(g_ * ref) / (np.linalg.norm(g_) * np.linalg.norm(ref)))
    return {"us": t_all * 1e6, "runs": n_all, "cores": cores, "err": err, "cos": cos,
            "one_thread_us": t_one * 1e6, "one_thread_runs": n_one,
            "same_as_one_thread": bool(np.array_equal(one.reshape(ref.shape), ref))}


def run_encode(args, layout) -> dict:
    """Bulk prefill (workload 1): one tp_encode_pages launch
    encodes ``context`` fp16 tokens of ``hkv`` kv heads into pages.  Input and
    page sets rotate (> 256 MB in total) so reads and writes go to HBM."""
    import torch

    from turbopolar_amd import TurboPolarConfig, _lib
    from turbopolar_amd.codecs import PolarQuantEncoder

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    int8, l1b, deepb, split = layout
    cfg = TurboPolarConfig(num_q_heads=args.hq, num_kv_heads=args.hkv, use_int8_radii=int8,
                           k_angle_bits_level1=l1b, k_angle_bits_deep=deepb, split_dim=split)
    enc = PolarQuantEncoder(cfg)
    n_pages = args.context // 64
    g = torch.Generator(device=dev).manual_seed(3)
    sets = []
    for _ in range(3):
        k = torch.randn((1, args.hkv, args.context, 128), generator=g, device=dev).half()
        v = torch.randn((1, args.hkv, args.context, 128), generator=g, device=dev).half()
        bufs = enc.alloc_pages(1, args.hkv, n_pages, dev)
        codes = torch.empty((1, args.hkv, n_pages, 64, 128), dtype=torch.int8, device=dev)
        scales = torch.empty((1, args.hkv, n_pages, 64, 4), dtype=torch.float16, device=dev)
        pages = _lib.TPPages(_lib.ptr(bufs["radii"]), _lib.ptr(bufs["radii_scales"]), _lib.ptr(bufs["angle_codes_l1"]),
                             _lib.ptr(bufs["angle_codes_deep"]), _lib.ptr(codes), _lib.ptr(scales), n_pages)
        sets.append((k, v, bufs, codes, scales, pages))
    L = _lib.lib()
    stream = torch.cuda.current_stream(dev).cuda_stream
    lay = enc.layout

    def step(i):
        k, v, _, _, _, pages = sets[i % len(sets)]
        st = L.tp_encode_pages(k.data_ptr(), v.data_ptr(), 0, args.hkv, args.context, 0, args.context,
                               ctypes.byref(lay), ctypes.byref(pages), 0, stream)
        if st:
            _lib.check(st, "tp_encode_pages")

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(args.steps):
        step(i)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    kv_bytes = 2 * args.hkv * args.context * 128 * 2
    page_bytes = args.hkv * n_pages * (bench_page_bytes(layout))
    k, v, bufs, codes, scales, _ = sets[0]
    return {"ms": ms, "read": kv_bytes, "write": page_bytes, "n_pages": n_pages,
            "set0": (k, v, bufs, codes, scales)}


def cpu_encode_baseline(args, layout, set0, budget_s):
    """Oracle restatement of the reference's page flush (encode_block +
    quantize_block, encoder.py:24-98, v_quant/encoder.py:16-30) of every page
    of the first input set, page ranges spread over every host core
    (``host_cores``), repeated for about ``budget_s`` seconds; every page is
    compared bitwise with what the GPU wrote for it.  Also a sample of pages
    on one thread, scaled to the cache."""
    from concurrent.futures import ThreadPoolExecutor

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import oracle

    int8, l1b, deepb, split = layout
    k, v, bufs, codes, scales = set0
    kn = k.cpu().numpy()
    vn = v.cpu().numpy()
    gpu = {name: t.cpu().numpy() for name, t in bufs.items() if t is not None}
    codes_n, scales_n = codes.cpu().numpy(), scales.cpu().numpy()
    S = args.context // 64
    res = [None] * S

    def same(a, b):  # bitwise
        return bool(np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8)))

    def enc(p0, p1):
        for p in range(p0, p1):
            ks, vs = kn[:, :, 64 * p:64 * (p + 1)], vn[:, :, 64 * p:64 * (p + 1)]
            blk = oracle.encode_block(ks, l1_bits=l1b, deep_bits=deepb, split_dim=split, use_int8_radii=int8)
            res[p] = (blk, oracle.quantize_block(vs[:, :, None]))

    cores = host_cores()
    ranges = _chunks(S, 4 * cores)
    with _OneBlasThread(), ThreadPoolExecutor(cores) as pool:
        t_all, n_all, _ = _sample(lambda: list(pool.map(lambda pr: enc(*pr), ranges)), budget_s, min_runs=1)
        p1 = max(1, S // 32)
        t_one, n_one, _ = _sample(lambda: enc(0, p1), budget_s / 4, min_runs=1)
    exact = True
    for p, (blk, (vc, vsc)) in enumerate(res):
        exact &= same(blk["radii"], gpu["radii"][:, :, p])
        exact &= same(blk["angle_codes_l1"], gpu["angle_codes_l1"][:, :, p])
        exact &= same(blk["angle_codes_deep"], gpu["angle_codes_deep"][:, :, p])
        if blk["radii_scales"] is not None:
            exact &= same(blk["radii_scales"].reshape(-1), gpu["radii_scales"][:, :, p].reshape(-1))
        exact &= same(vc[:, :, 0], codes_n[:, :, p]) and same(vsc[:, :, 0], scales_n[:, :, p])
    return {"us": t_all * 1e6, "runs": n_all, "cores": cores, "exact": exact, "pages": S,
            "one_thread_us": t_one * S / p1 * 1e6, "one_thread_sample": f"{n_one} runs over {p1} of {S} pages"}


def bench_page_bytes(layout) -> int:
    """Compressed bytes of one page of one kv head (K codes + radii + V codes + V scales)."""
    return algorithmic_bytes(0, 1, 1, layout)


def run_append(args, layout, n_appends: int = 4096) -> dict:
    """Single-token appends (workload 2) through
    TurboPolarKVCacheRuntime.append: every 64th append encodes a page."""
    import torch

    from turbopolar_amd import TurboPolarConfig, TurboPolarKVCacheRuntime

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    int8, l1b, deepb, split = layout
    cfg = TurboPolarConfig(num_q_heads=args.hq, num_kv_heads=args.hkv, use_int8_radii=int8,
                           k_angle_bits_level1=l1b, k_angle_bits_deep=deepb, split_dim=split)
    g = torch.Generator(device=dev).manual_seed(3)
    k = torch.randn((1, args.hkv, n_appends + 128, 128), generator=g, device=dev).half()
    v = torch.randn((1, args.hkv, n_appends + 128, 128), generator=g, device=dev).half()
    # One contiguous [1, hkv, 1, 128] tensor per step, as a decode loop hands
    # over each step's projected K and V (a strided slice of one big tensor
    # would add a copy kernel to every append).
    ks = [k[:, :, t:t + 1].contiguous() for t in range(n_appends + 128)]
    vs = [v[:, :, t:t + 1].contiguous() for t in range(n_appends + 128)]
    warm = TurboPolarKVCacheRuntime(cfg)
    for t in range(128):
        warm.append(ks[t], vs[t])
    torch.cuda.synchronize()
    rt = TurboPolarKVCacheRuntime(cfg)
    t0 = time.perf_counter()
    for t in range(n_appends):
        rt.append(ks[128 + t], vs[128 + t])
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    return {"us_per_append": dt / n_appends * 1e6, "appends": n_appends, "pages": rt.total_blocks}


def run_snapshot(args, layout, reps: int = 3) -> dict:
    """Page snapshot (turbopolar_amd.wire) of a full cache: device-to-host
    state_dict, safetensors write and read back onto the device.  Not a
    reference workload (the reference has no on-disk format)."""
    import tempfile

    import torch

    from turbopolar_amd import TurboPolarConfig, TurboPolarKVCacheRuntime, wire

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    int8, l1b, deepb, split = layout
    cfg = TurboPolarConfig(num_q_heads=args.hq, num_kv_heads=args.hkv, use_int8_radii=int8,
                           k_angle_bits_level1=l1b, k_angle_bits_deep=deepb, split_dim=split)
    g = torch.Generator(device=dev).manual_seed(5)
    rt = TurboPolarKVCacheRuntime(cfg)
    n = args.context + 37  # full pages plus a dense tail
    rt.append(torch.randn((1, args.hkv, n, 128), generator=g, device=dev).half(),
              torch.randn((1, args.hkv, n, 128), generator=g, device=dev).half())
    torch.cuda.synchronize()
    t_state, t_save, t_load = [], [], []
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "cache.safetensors")
        for _ in range(reps):
            t0 = time.perf_counter()
            tensors, meta = wire.state_dict(rt)
            t_state.append(time.perf_counter() - t0)
            t0 = time.perf_counter()
            wire.save(rt, path)
            t_save.append(time.perf_counter() - t0)
            t0 = time.perf_counter()
            back = wire.load(path, dev)
            torch.cuda.synchronize()
            t_load.append(time.perf_counter() - t0)
        file_bytes = os.path.getsize(path)
    S = rt.k_storage.block_count
    same = all(torch.equal(x[:, :, :S], y[:, :, :S]) for x, y in (
        (rt.k_storage.radii, back.k_storage.radii), (rt.k_storage.angle_codes_deep, back.k_storage.angle_codes_deep),
        (rt.v_storage.codes, back.v_storage.codes), (rt.v_storage.scales, back.v_storage.scales)))
    same = same and torch.equal(rt.partial_k, back.partial_k)
    payload = sum(t.numel() * t.element_size() for t in tensors.values())
    return {"state_dict_ms": min(t_state) * 1e3, "save_ms": min(t_save) * 1e3, "load_ms": min(t_load) * 1e3,
            "payload_bytes": payload, "file_bytes": file_bytes, "pages": S, "tail": rt._tail_len,
            "identical": bool(same)}


def run_timeline(args, layout) -> dict:
    """Phase timeline of the decode kernel: the same workload as the headline
    line, run on libturbopolar_hip_timeline.so (the product's code with the
    kernel's s_memrealtime phase stamps compiled in, TP_TIMELINE).  Thread 0 of
    every workgroup stamps its start, the issue of its first loads, each of
    wave 0's pages (scored once its codes arrived, done), the end of wave 0's
    pages, the workgroup's record stores, their completion and its ticket; the
    last workgroup of each unit also stamps the end of its combine.  The stamps of the last of ``steps``
    back-to-back launches are read back; times are microseconds from the first
    workgroup's start (100 MHz clock), median and max over workgroups."""
    import torch

    from turbopolar_amd import _lib, build
    from turbopolar_amd.kernels import fp16_scale

    if _lib._lib is not None:
        raise RuntimeError("the timeline workload must load its library first")
    _lib.LIB_PATH = build.TIMELINE_LIB_PATH
    if args.variant is not None:
        fn = _lib.lib().tp_measure_set_decode_variant
        fn.restype, fn.argtypes = ctypes.c_int32, [ctypes.c_int32]
        if fn(VARIANTS[args.variant]) != 0:
            raise RuntimeError(f"variant {args.variant} rejected")
    if not args.rotate:
        args.rotate = max(4, int(np.ceil(320e6 / algorithmic_bytes(args.hq, args.hkv, args.context // 64, layout))))
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg, caches = build_caches(args, dev, layout)
    L = _lib.lib()
    n_pages = caches[0]["pages"].S
    pps = args.pps or int(L.tp_default_pages_per_split(1, args.hq, args.hkv, n_pages))
    need = int(L.tp_decode_workspace_bytes(1, args.hq, args.hkv, n_pages, 0, pps))
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    scale = fp16_scale(cfg.attention_scale)
    stream = torch.cuda.current_stream(dev).cuda_stream
    for i in range(args.warmup + args.steps):
        c = caches[i % len(caches)]
        ps = c["pages"]
        st = L.tp_decode_attention(c["q"].data_ptr(), 1, args.hq, args.hkv, ctypes.byref(ps.layout),
                                   ctypes.byref(ps.pages), n_pages, None, None, 0, 0, c["seq"], scale, pps,
                                   ws.data_ptr(), need, c["out"].data_ptr(), stream)
        _lib.check(st, "tp_decode_attention")
    torch.cuda.synchronize()
    L.tp_timeline_address.restype = ctypes.c_void_p
    addr = L.tp_timeline_address()
    stamps = np.zeros((2048, 80), np.uint64)
    hip = ctypes.CDLL("libamdhip64.so")
    rc = hip.hipMemcpy(stamps.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(addr), ctypes.c_size_t(stamps.nbytes), 2)
    if rc != 0:
        raise RuntimeError(f"hipMemcpy of the stamps failed: {rc}")
    units = args.hkv * ((args.hq // args.hkv + 15) // 16)
    groups = units * ((n_pages + pps - 1) // pps)
    t = stamps[:groups].astype(np.int64)
    start = t[:, 0]
    us = (t - start.min()) / 100.0
    valid = t >= start[:, None]  # stamps written by this launch
    names = {0: "start", 59: "wave 0: kernel arguments loaded", 60: "wave 0: q loads issued",
             1: "wave 0: first page loads issued", 3: "wave 0: code table entries built",
             2: "barrier passed (all waves' first loads issued, tables ready)"}
    for i in range(12):
        names[4 + 4 * i] = f"wave 0 page {i}: codes arrived, scored"
        names[5 + 4 * i] = f"wave 0 page {i}: done"
    names.update({52: "wave 0 pages done", 53: "workgroup record stored", 54: "stores complete",
                  55: "ticket drawn", 64: "last workgroup: combine entered",
                  65: "last workgroup: record addresses computed", 66: "last workgroup: one more stamp (its cost)",
                  61: "last workgroup: first record loads issued",
                  62: "last workgroup: their (m, l) pairs arrived", 57: "last workgroup: records folded",
                  63: "last workgroup: every wave's fold in LDS", 58: "last workgroup: groups merged",
                  56: "last workgroup: output stored"})
    phases = {}
    for k, name in names.items():
        col = us[valid[:, k], k]
        if col.size:
            phases[name] = {"median_us": round(float(np.median(col)), 2), "max_us": round(float(col.max()), 2),
                            "workgroups": int(col.size)}
    # The combining workgroups' own ticket (they draw the last ticket of their
    # unit), and the phases per XCD: workgroup i runs on XCD i mod 8.
    last = valid[:, 56]
    if last.any():
        col = us[last & valid[:, 55], 55]
        phases["last workgroup: ticket drawn"] = {"median_us": round(float(np.median(col)), 2),
                                                  "max_us": round(float(col.max()), 2), "workgroups": int(col.size)}
    xcd = np.arange(groups) % 8
    per_xcd = {}
    for k in (0, 1, 2, 52, 53, 55):
        row = []
        for x in range(8):
            col = us[(xcd == x) & valid[:, k], k]
            row.append([round(float(np.median(col)), 2), round(float(col.max()), 2)] if col.size else None)
        per_xcd[names[k]] = row
    return {"phases": phases, "per_xcd_median_max_us": per_xcd, "pps": pps, "groups": groups}


# Bytes per page and kv head of each page field the decode kernel reads, in
# its order (default: radii, level-1 codes, deep codes, V codes, V scales;
# fast: int8 log radii, radius scale, deep codes, V codes, V scales).
PAGE_FIELDS = {"default": (8192, 1024, 1024, 8192, 512), "fast": (4096, 2, 4096, 8192, 512)}
# Launch shapes of the streaming-read sweep (grid, threads, unroll); the
# decode kernel's own grid is added in front.
STREAM_SHAPES = ((256, 512, 16), (512, 256, 16), (256, 1024, 8), (2048, 512, 8), (4096, 512, 8), (8192, 512, 8),
                 (8192, 256, 8), (4096, 1024, 4))
# Launch shapes of the dynamic sweep (tp_measure_stream_read_dynamic: every
# wave claims U-KiB chunks from a counter); the decode grid is added in front.
STREAM_DYNAMIC_SHAPES = ((256, 512, 4), (256, 512, 16), (512, 512, 8), (512, 256, 8), (1024, 256, 8), (1024, 512, 8),
                         (2048, 256, 8))


def run_stream(args, layout) -> dict:
    """The streaming-read ceiling: tp_measure_stream_read (measurement
    library) reads buffers of exactly the page fields one decode step reads
    (same sizes, same 16-byte non-temporal loads), with nothing computed, at
    the decode kernel's grid and at the launch shapes of STREAM_SHAPES, then
    with the chunks claimed dynamically by every wave
    (tp_measure_stream_read_dynamic) at the decode grid and at
    STREAM_DYNAMIC_SHAPES.  Buffers rotate over > 320 MB as in the headline
    line, so reads come from HBM; each shape is timed over ``steps``
    back-to-back launches with HIP events on the launch stream."""
    import torch

    from turbopolar_amd import _lib, build

    if _lib._lib is not None:
        raise RuntimeError("the stream workload must load its library first")
    _lib.LIB_PATH = build.TIMELINE_LIB_PATH
    L = _lib.lib()
    fn = L.tp_measure_stream_read
    fn.restype = ctypes.c_int32
    fn.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_int64), ctypes.c_int32, ctypes.c_int32,
                   ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p]
    fn_dyn = L.tp_measure_stream_read_dynamic
    fn_dyn.restype = ctypes.c_int32
    fn_dyn.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_int64), ctypes.c_int32,
                       ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_uint64,
                       ctypes.POINTER(ctypes.c_uint64), ctypes.c_void_p, ctypes.c_void_p]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    n_pages = args.context // 64
    fields = [args.hkv * n_pages * f for f in PAGE_FIELDS[args.layout]]
    fields = [(f + 15) // 16 * 16 for f in fields]
    total = sum(fields)
    rotate = args.rotate or max(4, int(np.ceil(320e6 / total)))
    g = torch.Generator(device=dev).manual_seed(7)
    sets = []
    for _ in range(rotate):
        bufs = [torch.randint(0, 256, (f,), dtype=torch.uint8, device=dev, generator=g) for f in fields]
        ptrs = (ctypes.c_void_p * len(bufs))(*[b.data_ptr() for b in bufs])
        sizes = (ctypes.c_int64 * len(bufs))(*fields)
        sets.append((bufs, ptrs, sizes))
    pps = int(L.tp_default_pages_per_split(1, args.hq, args.hkv, n_pages))
    units = args.hkv * ((args.hq // args.hkv + 15) // 16)
    decode_grid = units * ((n_pages + pps - 1) // pps)
    shapes = [(decode_grid, 512, 8)] + [s for s in STREAM_SHAPES if s != (decode_grid, 512, 8)]
    dyn_shapes = [(decode_grid, 512, 8)] + [s for s in STREAM_DYNAMIC_SHAPES if s != (decode_grid, 512, 8)]
    sink = torch.zeros(max(s[0] for s in shapes + dyn_shapes), dtype=torch.int32, device=dev)
    counter = torch.zeros(1, dtype=torch.int64, device=dev)
    base = ctypes.c_uint64(0)
    stream = torch.cuda.current_stream(dev).cuda_stream
    results = []
    for dynamic, grid, threads, unroll in [(False, *x) for x in shapes] + [(True, *x) for x in dyn_shapes]:
        def launch(i):
            _, ptrs, sizes = sets[i % rotate]
            if dynamic:
                nxt = ctypes.c_uint64(0)
                rc = fn_dyn(ptrs, sizes, len(fields), grid, threads, unroll, ctypes.c_void_p(counter.data_ptr()),
                            base, ctypes.byref(nxt), ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(stream))
                base.value = nxt.value
            else:
                rc = fn(ptrs, sizes, len(fields), grid, threads, unroll, ctypes.c_void_p(sink.data_ptr()),
                        ctypes.c_void_p(stream))
            if rc != 0:
                raise RuntimeError("tp_measure_stream_read rejected its arguments")

        for i in range(args.warmup):
            launch(i)
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        for i in range(args.steps):
            launch(i)
        t1.record()
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) / args.steps * 1e3
        results.append({"grid": grid, "threads": threads, "unroll": unroll,
                        "claim": "dynamic" if dynamic else "static", "us": round(us, 3),
                        "GBps": round(total / (us * 1e-6) / 1e9, 1)})
    return {"bytes": total, "fields": fields, "rotate": rotate, "sweep": results, "decode_grid": decode_grid}


def profiled_traffic(name: str, args):
    """HBM bytes per launch that the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary profiles/<name>_8b_32k_traffic.json records, when this run is that
    workload (32k tokens, 32 q / 8 kv heads); else None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"{name}_8b_32k_traffic.json")
    if not (os.path.exists(path) and args.context == 32768 and args.hq == 32 and args.hkv == 8):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def cpu_append_baseline(args, layout, n_appends: int = 4096):
    """Host restatement of the reference's append (turbo_polar_cache.py:106-126):
    per single-token append a finiteness check of K and V, the tail
    concatenation, and at 64 tokens the oracle's page flush (encode_block +
    quantize_block); 1 thread, the same number of appends as the GPU line."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import oracle

    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    int8, l1b, deepb, split = layout
    rng = np.random.default_rng(3)
    ks = rng.standard_normal((n_appends, 1, args.hkv, 1, 128)).astype(np.float16)
    vs = rng.standard_normal((n_appends, 1, args.hkv, 1, 128)).astype(np.float16)
    pages = 0
    ctx = threadpool_limits(1) if threadpool_limits else None
    try:
        if ctx:
            ctx.__enter__()
        t0 = time.perf_counter()
        tk = tv = None
        for t in range(n_appends):
            k, v = ks[t], vs[t]
            if not (np.isfinite(k).all() and np.isfinite(v).all()):
                raise ValueError("non-finite synthetic input")
            tk = k if tk is None else np.concatenate([tk, k], axis=2)
            tv = v if tv is None else np.concatenate([tv, v], axis=2)
            if tk.shape[2] == 64:
                oracle.encode_block(tk, l1_bits=l1b, deep_bits=deepb, split_dim=split, use_int8_radii=int8)
                oracle.quantize_block(tv[:, :, None])
                tk = tv = None
                pages += 1
        dt = time.perf_counter() - t0
    finally:
        if ctx:
            ctx.__exit__(None, None, None)
    return dt / n_appends * 1e6, n_appends, pages


def copy_calibration(nbytes: int, reps: int = 10) -> None:
    """Plain device-to-device copy of a known size: the reference for scaling
    rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes."""
    import torch

    dev = torch.device("cuda:0")
    src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    # Push the source out of the caches' reach before each copy.
    flush = torch.empty(512 * 1024 * 1024 // 4, dtype=torch.float32, device=dev)
    for _ in range(reps):
        flush.zero_()
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "reps": reps}))


# Untimed warm-up steps per workload when --warmup is not given.  A kernel
# launched from a fresh process runs before the GPU's clocks have settled: the
# 32k decode step timed after 20 warm-up launches read 19.8 us and after 2000
# (about 40 ms of GPU work) 18.5-18.6 us on the same box, so the kernel
# workloads warm up for tens of milliseconds.  prefill and model consume their
# warm-up steps as real tokens (longer context), so they keep short warm-ups.
WARMUP_DEFAULTS = {"decode": 2000, "qk": 2000, "decompress": 1000, "encode": 1000, "stream": 1000,
                   "layers": 200, "timeline": 200, "prefill": 3, "model": 4}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run a plain copy of BYTES bytes (counter calibration)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps before the timed ones (default: per workload, WARMUP_DEFAULTS)")
    ap.add_argument("--layout", choices=sorted(LAYOUTS), default="default")
    ap.add_argument("--context", type=int, default=32768)
    ap.add_argument("--hq", type=int, default=32)
    ap.add_argument("--hkv", type=int, default=8)
    ap.add_argument("--pps", type=int, default=0, help="pages per workgroup (0 = library default)")
    ap.add_argument("--tail", type=int, default=0,
                    help="decode: dense fp16 tail tokens after the context's pages (0-63)")
    ap.add_argument("--rotate", type=int, default=0, help="independent caches to rotate (0 = auto, >256 MB)")
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU baseline sampling")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--workload", choices=["decode", "encode", "append", "layers", "model", "decompress", "snapshot", "qk",
                                           "timeline", "stream", "prefill"],
                    default="decode",
                    help="decode (the BASELINE metric, default); encode / append: configs[3] workloads; "
                         "layers: configs[1] (--layers decode launches per step); "
                         "model: a configs[1]-shape Llama decoding through the transformers hook; "
                         "decompress: tp_decode_pages of a whole cache (prefill decompress-on-read); "
                         "prefill: TurboPolarFastCache.update_and_fetch of a chunk over a cache with a tail; "
                         "timeline: the decode kernel's phase stamps; "
                         "stream: the streaming-read ceiling of the decode step's page bytes")
    ap.add_argument("--kind", choices=["outlier", "loguniform", "studentt", "normal"], default=None,
                    help="K distribution (default: outlier for decode, loguniform for layers)")
    ap.add_argument("--layers", type=int, default=16)
    ap.add_argument("--model-path", default=None,
                    help="model: a local Llama checkpoint directory (config.json + safetensors) instead of the "
                         "randomly initialised configs[1] shape; never downloads")
    ap.add_argument("--graph", action="store_true",
                    help="layers: replay the step as one HIP graph; decode: time the steps as one graph replay")
    ap.add_argument("--dense-v", action="store_true",
                    help="decode: tp_decode_attention_dense_v (compressed K pages, dense fp16 V pages)")
    ap.add_argument("--qjl", action="store_true",
                    help="decode: tp_decode_attention_qjl (QJL correction on every page token; synthetic sketches)")
    ap.add_argument("--variant", choices=sorted(VARIANTS), default=None,
                    help="decode: run a decode-kernel variant of the measurement library (release: agent-scope "
                         "release fence before the split ticket; valu: QK and PV on the VALU; no-acquire: without "
                         "the combining workgroup's acquire fence; mfma: the product kernel as built there)")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the decode-attention path shards by kv head "
              "across GPUs with no exchange; multi-GPU runs are out of scope here). Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    if args.context % 64:
        sys.exit("--context must be a multiple of 64")
    if not 0 <= args.tail < 64 or (args.tail and (args.workload != "decode" or args.qjl or args.variant)):
        sys.exit("--tail takes 0-63 tokens and only the plain decode workload")
    if args.dense_v and (args.workload != "decode" or args.qjl or args.variant or args.tail):
        sys.exit("--dense-v takes only the plain decode workload")
    if args.warmup is None:
        args.warmup = WARMUP_DEFAULTS.get(args.workload, 20)
    layout = LAYOUTS[args.layout]
    if args.kind is None:
        args.kind = "loguniform" if args.workload == "layers" else "outlier"
    if args.workload == "decompress":
        r = run_decompress(args, layout)
        cpu = None
        if not args.no_cpu:
            cb = cpu_decompress_baseline(args, r, args.cpu_budget)
            cpu = {"value": round(cb["us"], 1), "unit": "us/step", "cores": cb["cores"], "kind": "port",
                   "sample": f"{cb['runs']} decompressions of all {r['n_pages']} pages of {args.hkv} kv heads (oracle "
                             f"NumPy restatement of decode_block + dequantize_block, page ranges on {cb['cores']} "
                             f"threads; V bit-exact {cb['v_exact']}, K within {cb['k_ulps']} fp16 ulp of the oracle)",
                   "one_thread": {"value": round(cb["one_thread_us"], 1), "unit": "us/step", "cores": 1,
                                  "sample": cb["one_thread_sample"] + ", scaled to the cache"}}
        nbytes = r["read"] + r["write"]
        gbps = nbytes / (r["ms"] * 1e-3) / 1e9
        print(json.dumps({
            "metric": "page decompress us/step (decompress-on-read of a whole cache), Llama-3-8B kv shape",
            "value": round(r["ms"] * 1e3, 3), "unit": "us/step", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(r["ms"], 6), "higher_is_better": False,
            "dtype": "f16", "data": "synthetic",
            "config": {"workload": f"tp_decode_pages: {r['n_pages']} pages x {args.hkv} kv heads -> dense fp16 K "
                                   f"and V ({args.context} tokens)", "layout": args.layout},
            "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": profiled_traffic(f"decompress_{args.layout}", args)},
            "algorithmic_bytes_per_step": {"read": r["read"], "write": r["write"]},
            "cpu_baseline": cpu,
        }))
        return
    if args.workload == "qk":
        r = run_fused_qk(args, layout)
        cpu = None
        if not args.no_cpu:
            cb = cpu_qk_baseline(args, r, args.cpu_budget)
            cpu = {"value": round(cb["us"], 1), "unit": "us/step", "cores": cb["cores"], "kind": "port",
                   "sample": f"{cb['runs']} full steps over the {args.context}-token cache (oracle NumPy float32 "
                             f"restatement of _cpu_fused_qk per kv head and page range on {cb['cores']} threads; GPU "
                             f"scores max-abs {cb['err']:.2e}, cosine {cb['cos']:.6f})",
                   "one_thread": {"value": round(cb["one_thread_us"], 1), "unit": "us/step", "cores": 1,
                                  "sample": f"{cb['one_thread_runs']} steps of the unsplit oracle call",
                                  "outputs_identical": cb["same_as_one_thread"]}}
        nbytes = r["read"] + r["write"]
        gbps = nbytes / (r["ms"] * 1e-3) / 1e9
        print(json.dumps({
            "metric": "fused QK us/step (scores of every query head over every cached token), Llama-3-8B shape",
            "value": round(r["ms"] * 1e3, 3), "unit": "us/step", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(r["ms"], 6), "higher_is_better": False,
            "dtype": "f16", "data": "synthetic",
            "config": {"workload": f"tp_fused_qk: {args.hq} q / {args.hkv} kv heads, {r['n_pages']} pages "
                                   f"({args.context} tokens), {r['n_caches']} rotating caches", "layout": args.layout},
            "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": profiled_traffic(f"qk_{args.layout}", args)},
            "algorithmic_bytes_per_step": {"read": r["read"], "write": r["write"]},
            "cpu_baseline": cpu,
        }))
        return
    if args.workload == "prefill":
        r = run_prefill(args, layout)
        nbytes = r["read"] + r["write"]
        gbps = nbytes / (r["ms"] * 1e-3) / 1e9
        print(json.dumps({
            "metric": "prefill chunk ms/step (append 64 tokens + decompress-on-read of the whole history with a "
                      "37-token tail), Llama-3-8B kv shape",
            "value": round(r["ms"], 4), "unit": "ms/step", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(r["ms"], 4), "higher_is_better": False,
            "dtype": "f16", "data": "synthetic",
            "config": {"workload": f"TurboPolarFastCache.update_and_fetch of 64-token chunks, {args.hkv} kv heads, "
                                   f"history {r['first']} -> {r['last']} tokens (37 in the dense tail)",
                       "layout": args.layout, "k_distribution": args.kind},
            "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                         "note": "wall clock of whole calls (host work included) over the mid-run history's bytes"},
            "algorithmic_bytes_per_step": {"read": r["read"], "write": r["write"]},
            "checks": {"tail_kept_and_output_finite": r["tail_ok"]},
        }))
        return
    if args.workload == "stream":
        r = run_stream(args, layout)
        best = min(r["sweep"], key=lambda e: e["us"])
        gbps = r["bytes"] / (best["us"] * 1e-6) / 1e9
        print(json.dumps({
            "metric": "streaming-read ceiling: µs to read one decode step's page bytes (no compute)",
            "value": best["us"], "unit": "us/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "higher_is_better": False, "dtype": "u8", "data": "synthetic",
            "config": {"workload": f"tp_measure_stream_read over the page fields of {args.hkv} kv heads x "
                                   f"{args.context // 64} pages ({args.context} tokens), {r['rotate']} rotating sets",
                       "layout": args.layout, "field_bytes": r["fields"], "best_shape": best},
            "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None},
            "decode_grid": next(e for e in r["sweep"] if e["grid"] == r["decode_grid"] and e["threads"] == 512
                                and e["unroll"] == 8 and e["claim"] == "static"),
            "decode_grid_dynamic": next(e for e in r["sweep"] if e["grid"] == r["decode_grid"] and e["threads"] == 512
                                        and e["unroll"] == 8 and e["claim"] == "dynamic"),
            "sweep": r["sweep"],
        }))
        return
    if args.workload == "timeline":
        r = run_timeline(args, layout)
        print(json.dumps({"workload": workload_name(args) + " -- kernel phase timeline", "layout": args.layout,
                          "pages_per_split": r["pps"], "workgroups": r["groups"], "phases": r["phases"],
                          "per_xcd_median_max_us": r["per_xcd_median_max_us"]}))
        return
    if args.workload == "model":
        r = run_model(args)
        print(json.dumps({
            "metric": "Llama decode tokens/s through the transformers hook (fused decode attention)",
            "value": round(1.0 / r["turbo_s"], 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(r["turbo_s"] * 1e3, 3), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": f"{r['weights']} weights, f16 cache",
            "data": "synthetic tokens and cache" if args.model_path else "synthetic",
            "config": {"workload": (f"Llama checkpoint {args.model_path}" if args.model_path else "random-init Llama")
                                   + f", {args.layers} layers, {args.hq} q / {args.hkv} kv heads, "
                                   f"head_dim 128, {args.context} cached tokens per layer"
                                   + ("" if args.model_path else " (BASELINE configs[1] shape)")
                                   + ", teacher-forced single-token decode", "layout": "fast (make_turbo_caches)"},
            "dense_baseline": {"tokens_per_s": round(1.0 / r["dense_s"], 2), "ms_per_token": round(r["dense_s"] * 1e3, 3),
                               "kv_bytes": r["dense_bytes"], "note": "the model's own DynamicCache (the same fp16 "
                                                                      f"K/V values held as {r['weights']}), eager "
                                                                      "attention"},
            "turbo_kv_bytes": r["turbo_bytes"],
            "gpu_busy_ms_per_token": {"turbo": r["turbo_busy_ms"], "dense": r["dense_busy_ms"],
                                      "note": "sum of device kernel durations of one forward (torch.profiler), "
                                              "against ms_per_step of wall clock"},
            "checks": {"logit_cosine_min_vs_dense": round(r["cos_min"], 6), "top1_agreement_vs_dense": r["top1"]},
        }))
        return
    if args.workload == "layers":
        r = run_layers(args, layout)
        n_pages = args.context // 64
        step_bytes = args.layers * algorithmic_bytes(args.hq, args.hkv, n_pages, layout)
        us = r["ms"] * 1e3
        gbps = step_bytes / (r["ms"] * 1e-3) / 1e9
        print(json.dumps({
            "metric": f"{args.layers}-layer decode-attention µs/step (sum over layers) + achieved HBM GB/s",
            "value": round(us, 3), "unit": "us/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(r["ms"], 6), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
            "dtype": "f16", "data": "synthetic",
            "config": {"workload": f"{args.layers} layers x {args.context} ctx decode, one query per layer "
                                   f"(BASELINE configs[1])", "layout": args.layout, "q_heads": args.hq,
                       "kv_heads": args.hkv, "head_dim": 128, "batch": 1, "k_distribution": args.kind,
                       "pages_per_split": r["pps"], "hip_graph": bool(args.graph),
                       "algorithmic_bytes_per_step": step_bytes},
            "tokens_per_s": round(1e6 / us, 1), "us_per_layer": round(us / args.layers, 3),
            "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None},
            "checks": {"outputs_match_first_step": r["outputs_match_first_step"],
                       "graph_replays_match_eager": r["graph_equal"]},
        }))
        return
    if args.workload == "encode":
        r = run_encode(args, layout)
        cpu = None
        if not args.no_cpu:
            cb = cpu_encode_baseline(args, layout, r["set0"], args.cpu_budget)
            cpu = {"value": round(cb["us"], 1), "unit": "us/step", "cores": cb["cores"], "kind": "port",
                   "sample": f"{cb['runs']} encodes of all {cb['pages']} pages of {args.hkv} kv heads (oracle NumPy "
                             f"restatement of encode_block + quantize_block, page ranges on {cb['cores']} threads; "
                             f"every page bit-exact vs GPU: {cb['exact']})",
                   "one_thread": {"value": round(cb["one_thread_us"], 1), "unit": "us/step", "cores": 1,
                                  "sample": cb["one_thread_sample"] + ", scaled to the cache"}}
        nbytes = r["read"] + r["write"]
        gbps = nbytes / (r["ms"] * 1e-3) / 1e9
        print(json.dumps({
            "metric": "page encode us/step (bulk prefill), Llama-3-8B kv shape",
            "value": round(r["ms"] * 1e3, 3), "unit": "us/step", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(r["ms"], 6), "higher_is_better": False,
            "dtype": "f16", "data": "synthetic",
            "config": {"workload": f"encode {args.context} fp16 tokens x {args.hkv} kv heads into "
                                   f"{r['n_pages']} pages (BASELINE configs[3])", "layout": args.layout},
            "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": profiled_traffic(f"encode_{args.layout}", args)},
            "algorithmic_bytes_per_step": {"read": r["read"], "write": r["write"]},
            "cpu_baseline": cpu,
        }))
        return
    if args.workload == "append":
        r = run_append(args, layout)
        cpu = None
        if not args.no_cpu:
            cpu_us, n_cpu, cpu_pages = cpu_append_baseline(args, layout, r["appends"])
            cpu = {"value": round(cpu_us, 2), "unit": "us/append", "cores": 1, "kind": "port",
                   "sample": f"{n_cpu} single-token appends with {cpu_pages} page flushes (host restatement of "
                             f"append: finiteness check, tail concatenation, oracle encode_block + "
                             f"quantize_block per full page; 1 thread: each append depends on the one before)"}
        print(json.dumps({
            "metric": "single-token append latency, Llama-3-8B kv shape",
            "value": round(r["us_per_append"], 2), "unit": "us/append", "n_gpus": 1,
            "higher_is_better": False, "dtype": "f16", "data": "synthetic",
            "config": {"workload": f"{r['appends']} single-token appends of {args.hkv} kv heads "
                                   f"through TurboPolarKVCacheRuntime.append, {r['pages']} page encodes "
                                   f"(BASELINE configs[3])", "layout": args.layout},
            "cpu_baseline": cpu,
        }))
        return
    if args.workload == "snapshot":
        r = run_snapshot(args, layout)
        print(json.dumps({
            "metric": "page snapshot save + load, Llama-3-8B kv shape",
            "value": round(r["save_ms"] + r["load_ms"], 2), "unit": "ms", "n_gpus": 1,
            "higher_is_better": False, "dtype": "u8/i8/f16", "data": "synthetic",
            "breakdown": {k: round(r[k], 2) for k in ("state_dict_ms", "save_ms", "load_ms")},
            "payload_bytes": r["payload_bytes"], "file_bytes": r["file_bytes"], "identical": r["identical"],
            "config": {"workload": f"{r['pages']} pages + {r['tail']} tail tokens of {args.hkv} kv heads, "
                                   f"safetensors file in a temporary directory", "layout": args.layout},
        }))
        return
    n_pages = args.context // 64
    step_bytes = algorithmic_bytes(args.hq, args.hkv, n_pages, layout, args.tail)
    if args.qjl:
        step_bytes += args.hkv * n_pages * 64 * (8 + 2) + args.hq * 8  # sketches, residual norms, query sketches
    if args.dense_v:
        step_bytes += args.hkv * n_pages * 64 * (256 - 136)  # dense fp16 V rows in place of V codes and scales
    if not args.rotate:
        args.rotate = max(4, int(np.ceil(320e6 / step_bytes)))

    if args.variant is not None:
        from turbopolar_amd import _lib, build

        if _lib._lib is not None:
            raise RuntimeError("--variant must load the measurement library first")
        _lib.LIB_PATH = build.TIMELINE_LIB_PATH
        fn = _lib.lib().tp_measure_set_decode_variant
        fn.restype, fn.argtypes = ctypes.c_int32, [ctypes.c_int32]
        if fn(VARIANTS[args.variant]) != 0:
            raise RuntimeError(f"variant {args.variant} rejected")
    res = run_gpu(args, layout)
    ms = res["ms"]
    us = ms * 1e3
    gbps = step_bytes / (ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu and not args.qjl and not args.dense_v:
        cb = cpu_baseline(args, layout, res["caches"], args.cpu_budget)
        cpu = {"value": round(cb["us"], 1), "unit": "us/step", "cores": cb["cores"], "kind": "port",
               "sample": f"{cb['runs']} full decode steps of the {args.hq}-head/{args.hkv}-kv-head {args.context}-token "
                         f"cache (oracle NumPy float32 restatement of _cpu_online_attention_dense_tail, K decode and "
                         f"V dequantisation per kv head and page range, attention per kv head, on {cb['cores']} "
                         f"threads; max-abs vs GPU {cb['err']:.2e})",
               "one_thread": {"value": round(cb["one_thread_us"], 1), "unit": "us/step", "cores": 1,
                              "sample": f"{cb['one_thread_runs']} steps of the unsplit oracle call",
                              "outputs_identical": cb["same_as_one_thread"]},
               "host": {"affinity_cores": affinity_cores(), "os_cpu_count": os.cpu_count(),
                        "cgroup_cpu_quota": cgroup_cpu_quota()}}
        if cb["sixteen_us"] is not None:
            cpu["sixteen_threads"] = {"value": round(cb["sixteen_us"], 1), "unit": "us/step", "cores": 16,
                                      "sample": f"{cb['sixteen_runs']} full decode steps on 16 threads"}
    traffic = None
    tpath = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                         f"decode_attention_{'dense_v_' if args.dense_v else ''}{args.layout}_8b_32k_traffic.json")
    if os.path.exists(tpath) and args.context == 32768 and args.hq == 32 and args.hkv == 8 and not args.tail:
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    metric = METRIC
    if (args.context, args.hq, args.hkv, args.tail) != (32768, 32, 8, 0):
        metric = (f"decode-attn µs/step + achieved HBM GB/s (% peak), {args.hq} q / {args.hkv} kv heads, "
                  f"{args.context} ctx" + (f" + {args.tail} tail tokens" if args.tail else ""))
    line = {
        "metric": metric,
        "value": round(us, 3),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": workload_name(args),
            "layout": args.layout,
            "q_heads": args.hq,
            "kv_heads": args.hkv,
            "head_dim": 128,
            "context": args.context,
            "tail_tokens": args.tail,
            "batch": 1,
            "pages_per_split": res["pps"],
            "rotated_caches": args.rotate,
            "algorithmic_bytes_per_step": step_bytes,
        },
        "tokens_per_s": round(1e6 / us, 1),
        "achieved_GBps": round(gbps, 1),
        "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": traffic},
        "cpu_baseline": cpu,
        "checks": {"finite": res["finite"], "deterministic_rerun": res["rerun_equal"]},
    }
    if args.variant is not None:
        line["kernel_variant"] = f"{args.variant} (measurement library: phase stamps compiled in)"
    if res.get("graph_equal") is not None:
        line["config"]["hip_graph"] = f"the {args.steps} timed launches captured once and timed as one replay"
        line["checks"]["graph_replays_equal_eager"] = bool(res["graph_equal"])
    if args.dense_v:
        line["metric"] = "decode-attn with dense V µs/step + achieved HBM GB/s, Llama-3-8B shape"
        line["config"]["workload"] += " + dense fp16 V (tp_decode_attention_dense_v)"
        line["cpu_baseline"] = None
    if args.qjl:
        line["metric"] = "decode-attn with QJL correction µs/step + achieved HBM GB/s, Llama-3-8B shape"
        line["config"]["workload"] += " + QJL (tp_decode_attention_qjl, 64-bit sketches, synthetic)"
        line["cpu_baseline"] = None
        line["roofline"]["traffic"] = None
    print(json.dumps(line))


if __name__ == "__main__":
    main()
