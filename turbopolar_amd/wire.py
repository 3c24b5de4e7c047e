"""On-disk / wire format of a TurboPolar cache.

The reference keeps its compressed cache only in memory
(rfsn_v11/generation/turbo_polar_cache.py:18-395, storage.py:17-169); this is
an extension: a snapshot of one ``TurboPolarKVCacheRuntime`` as a safetensors
file (or the same tensors and string metadata in memory), so a cache can be
written out, moved and restored bit for bit.

A snapshot holds only the valid pages, in the page layout of the storage
(``[B, H, S, ...]`` per buffer, contiguous), plus the dense tail:

========================  =============================================  ==========
name                      shape                                          dtype
========================  =============================================  ==========
``k.radii``               ``[B, H, S, 64, head_dim/2]``                  fp16 / int8
``k.radii_scales``        ``[B, H, S, 1, 1]`` (int8 radii only)           fp16
``k.angle_l1``            ``[B, H, S, 64, l1_row]`` (if l1_row > 0)       uint8
``k.angle_deep``          ``[B, H, S, 64, deep_row]`` (if deep_row > 0)   uint8
``v.codes``               ``[B, H, S, 1, 64, head_dim]``                 int8
``v.scales``              ``[B, H, S, 1, 64, head_dim/32]``              fp16
``tail.k``, ``tail.v``    ``[B, H, T, head_dim]``, T = tail tokens < 64  input dtype
========================  =============================================  ==========

and string metadata: ``format`` (``turbopolar-pages``), ``version`` (1), the
``TurboPolarConfig`` as JSON, the runtime's invariants (batch, kv heads,
head_dim, input dtype), ``actual_seq_len``, ``total_blocks``, the byte and
time counters and the encoder metadata.  Loading checks the format, version,
shapes and dtypes against the config and raises ``ValueError`` on any
mismatch; it never executes anything from the file (safetensors holds raw
tensors and strings only).
"""

from __future__ import annotations

import dataclasses
import json
from typing import Dict, Tuple

import torch

from .config import TurboPolarConfig
from .kernels import PAGE
from .runtime import TurboPolarKVCacheRuntime

FORMAT = "turbopolar-pages"
VERSION = 1

_DTYPES = {"torch.float16": torch.float16, "torch.float32": torch.float32}


def _config_json(config: TurboPolarConfig) -> str:
    return json.dumps(dataclasses.asdict(config), sort_keys=True)


def _runtime_of(cache) -> TurboPolarKVCacheRuntime:
    rt = getattr(cache, "runtime", cache)  # a TurboPolarFastCache wraps its runtime
    if not isinstance(rt, TurboPolarKVCacheRuntime):
        raise TypeError(f"expected a TurboPolarKVCacheRuntime or TurboPolarFastCache, got {type(cache).__name__}")
    return rt


def _host_copy(t: torch.Tensor) -> torch.Tensor:
    """A host copy that shares no memory with ``t``: device tensors go to
    pinned memory asynchronously (the caller synchronises once)."""
    if t.is_cuda:
        out = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
        out.copy_(t, non_blocking=True)
        return out
    return t.clone(memory_format=torch.contiguous_format)


def state_dict(cache) -> Tuple[Dict[str, torch.Tensor], Dict[str, str]]:
    """(tensors on the host, string metadata) of a runtime or fast cache."""
    rt = _runtime_of(cache)
    if not rt._initialized:
        raise ValueError("cannot snapshot an empty cache (nothing was appended)")
    S = rt.k_storage.block_count
    tensors: Dict[str, torch.Tensor] = {}
    if S:
        ks, vs = rt.k_storage, rt.v_storage
        tensors["k.radii"] = _host_copy(ks.radii[:, :, :S])
        if ks.radii_scales is not None:
            tensors["k.radii_scales"] = _host_copy(ks.radii_scales[:, :, :S])
        if ks.angle_codes_l1.shape[-1]:
            tensors["k.angle_l1"] = _host_copy(ks.angle_codes_l1[:, :, :S])
        if ks.angle_codes_deep.shape[-1]:
            tensors["k.angle_deep"] = _host_copy(ks.angle_codes_deep[:, :, :S])
        tensors["v.codes"] = _host_copy(vs.codes[:, :, :S])
        tensors["v.scales"] = _host_copy(vs.scales[:, :, :S])
    if rt._tail_len:
        tail_k, tail_v = rt._tail_views()
        tensors["tail.k"] = _host_copy(tail_k)
        tensors["tail.v"] = _host_copy(tail_v)
    devices = {t.device for t in (rt.k_storage.radii, rt._tail_k) if t is not None and t.is_cuda}
    for d in devices:
        torch.cuda.synchronize(d)
    meta = {
        "format": FORMAT,
        "version": str(VERSION),
        "config": _config_json(rt.config),
        "batch": str(rt._batch_size),
        "kv_heads": str(rt._num_kv_heads),
        "head_dim": str(rt._head_dim),
        "input_dtype": str(rt._input_dtype),
        "actual_seq_len": str(rt.actual_seq_len),
        "pages": str(S),
        "tail_tokens": str(rt._tail_len),
        "total_blocks": str(rt.total_blocks),
        "bytes_written": str(rt.bytes_written),
        "bytes_read": str(rt.bytes_read),
        "compression_time_ns": str(rt.compression_time_ns),
        "encoder_metadata": json.dumps(rt.k_storage.metadata, sort_keys=True),
        # growth telemetry: restored as it was, so get_io_telemetry() agrees
        "k_capacity": str(rt.k_storage.capacity),
        "v_capacity": str(rt.v_storage.capacity),
        "k_reallocs": str(rt.k_storage.reallocation_count),
        "v_reallocs": str(rt.v_storage.reallocation_count),
        "k_growth_bytes": str(rt.k_storage.bytes_copied_during_growth),
        "v_growth_bytes": str(rt.v_storage.bytes_copied_during_growth),
    }
    return tensors, meta


def _expect(tensors: Dict[str, torch.Tensor], name: str, shape: tuple, dtype: torch.dtype) -> torch.Tensor:
    t = tensors.get(name)
    if t is None:
        raise ValueError(f"snapshot lacks {name}")
    if tuple(t.shape) != shape or t.dtype != dtype:
        raise ValueError(f"snapshot {name}: expected {shape} {dtype}, got {tuple(t.shape)} {t.dtype}")
    return t


def load_state_dict(tensors: Dict[str, torch.Tensor], meta: Dict[str, str], device) -> TurboPolarKVCacheRuntime:
    """A runtime restored from ``state_dict``'s output, its pages on ``device``."""
    if meta.get("format") != FORMAT:
        raise ValueError(f"not a TurboPolar page snapshot (format {meta.get('format')!r})")
    if meta.get("version") != str(VERSION):
        raise ValueError(f"unsupported snapshot version {meta.get('version')!r} (this build reads {VERSION})")
    try:
        config = TurboPolarConfig(**json.loads(meta["config"]))
        B, H, D = int(meta["batch"]), int(meta["kv_heads"]), int(meta["head_dim"])
        S, T = int(meta["pages"]), int(meta["tail_tokens"])
        seq = int(meta["actual_seq_len"])
        in_dtype = _DTYPES[meta["input_dtype"]]
        caps = int(meta["k_capacity"]), int(meta["v_capacity"])
        growth = [int(meta[k]) for k in ("k_reallocs", "v_reallocs", "k_growth_bytes", "v_growth_bytes")]
    except (KeyError, TypeError, ValueError, json.JSONDecodeError) as e:
        raise ValueError(f"malformed snapshot metadata: {e}") from None
    if not (0 <= T < PAGE) or S < 0 or seq != S * PAGE + T or (S and min(caps) < S):
        raise ValueError(f"inconsistent snapshot: {S} pages, {T} tail tokens, actual_seq_len {seq}")
    rt = TurboPolarKVCacheRuntime(config)
    enc = rt.polar_encoder
    if H != config.num_kv_heads or D != config.head_dim:
        raise ValueError(f"snapshot shape (kv heads {H}, head_dim {D}) does not match its config")
    l1_row, deep_row = enc.row_bytes()
    rdt = torch.int8 if enc.use_int8_radii else torch.float16
    dev = torch.device(device)
    if S:
        radii = _expect(tensors, "k.radii", (B, H, S, PAGE, D // 2), rdt)
        v_codes = _expect(tensors, "v.codes", (B, H, S, 1, PAGE, D), torch.int8)
        v_scales = _expect(tensors, "v.scales", (B, H, S, 1, PAGE, D // 32), torch.float16)
        l1 = _expect(tensors, "k.angle_l1", (B, H, S, PAGE, l1_row), torch.uint8) if l1_row else None
        deep = _expect(tensors, "k.angle_deep", (B, H, S, PAGE, deep_row), torch.uint8) if deep_row else None
        rs = _expect(tensors, "k.radii_scales", (B, H, S, 1, 1), torch.float16) if enc.use_int8_radii else None
        # Allocated at the saved capacity in one step (no doubling copies).
        rt.k_storage.reserve(S, enc, B, H, dev, initial_capacity=caps[0])
        rt.v_storage.reserve(S, B, H, dev, initial_capacity=caps[1])
        rt.k_storage.radii[:, :, :S].copy_(radii)
        if l1 is not None:
            rt.k_storage.angle_codes_l1[:, :, :S].copy_(l1)
        if deep is not None:
            rt.k_storage.angle_codes_deep[:, :, :S].copy_(deep)
        if rs is not None:
            rt.k_storage.radii_scales[:, :, :S].copy_(rs)
        rt.v_storage.codes[:, :, :S].copy_(v_codes)
        rt.v_storage.scales[:, :, :S].copy_(v_scales)
        rt.k_storage.block_count = rt.v_storage.block_count = S
        rt.k_storage.reallocation_count, rt.v_storage.reallocation_count = growth[0], growth[1]
        rt.k_storage.bytes_copied_during_growth, rt.v_storage.bytes_copied_during_growth = growth[2], growth[3]
    if T:
        tk = _expect(tensors, "tail.k", (B, H, T, D), in_dtype)
        tv = _expect(tensors, "tail.v", (B, H, T, D), in_dtype)
        rt._tail_k = torch.zeros((B, H, PAGE, D), dtype=in_dtype, device=dev)
        rt._tail_v = torch.zeros((B, H, PAGE, D), dtype=in_dtype, device=dev)
        rt._tail_k[:, :, :T].copy_(tk)
        rt._tail_v[:, :, :T].copy_(tv)
        rt._tail_len = T
    rt._batch_size, rt._num_kv_heads, rt._head_dim, rt._input_dtype = B, H, D, in_dtype
    rt._initialized = True
    rt.actual_seq_len = seq
    rt.total_blocks = int(meta["total_blocks"])
    rt.bytes_written = int(meta["bytes_written"])
    rt.bytes_read = int(meta["bytes_read"])
    rt.compression_time_ns = int(meta["compression_time_ns"])
    return rt


def save(cache, path: str) -> None:
    """Write a runtime or fast cache to ``path`` as a safetensors file."""
    from safetensors.torch import save_file

    tensors, meta = state_dict(cache)
    save_file(tensors, path, metadata=meta)


def load(path: str, device) -> TurboPolarKVCacheRuntime:
    """Read a snapshot written by ``save`` onto ``device``."""
    from safetensors import safe_open

    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        tensors = {name: f.get_tensor(name) for name in f.keys()}
    return load_state_dict(tensors, meta, device)


def load_fast_cache(path: str, device):
    """A ``TurboPolarFastCache`` around the runtime read from ``path``."""
    from .fast_attention import TurboPolarFastCache

    rt = load(path, device)
    cache = TurboPolarFastCache(rt.config)
    cache.runtime = rt
    return cache
