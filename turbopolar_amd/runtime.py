"""Incremental compressed KV cache: the reference's ``TurboPolarKVCacheRuntime``.

Same public methods, attributes, telemetry keys and error contract as
rfsn_v11/generation/turbo_polar_cache.py:18-395.  Differences of mechanism
(not of behaviour):

* the dense tail lives in a preallocated ``[B, H, 64, D]`` device buffer
  instead of being re-concatenated on every append.  ``partial_k`` /
  ``partial_v`` return copies of its valid part (an append never changes
  them, like the reference's immutable arrays); ``get_fused_attention_inputs``
  returns views of it, valid until the next append, so a decode step copies
  nothing;
* full pages are encoded by one ``tp_encode_pages`` launch per append, written
  straight into the storage slots (no per-page Python loop, no intermediate
  block copies);
* a bulk append reserves capacity once (the doubling telemetry is unchanged).
"""

from __future__ import annotations

from typing import Any, Dict, Optional, Tuple

import torch

from . import _lib
from .codecs import GroupedVQuantizer, PolarQuantDecoder, PolarQuantEncoder
from .config import TurboPolarConfig
from .kernels import PAGE, decode_pages_gather, encode_pages
from .payload import PolarKeyBlock, QuantizedVBlock
from .storage import PolarKBlockStorage, QuantVBlockStorage, pages_of


def _nbytes(x: torch.Tensor) -> int:
    return int(x.numel() * x.element_size())


class TurboPolarKVCacheRuntime:
    def __init__(self, config: TurboPolarConfig):
        self.config = config
        self.polar_encoder = PolarQuantEncoder(config)
        self.v_quantizer = GroupedVQuantizer(group_size=32)
        # QJL is rejected by the config (turbo_polar_config.py:46-47); the
        # reference still builds an unused encoder here.
        self.qjl_encoder = None
        self.decoder = PolarQuantDecoder()

        self.k_storage = PolarKBlockStorage()
        self.v_storage = QuantVBlockStorage()
        self.qjl_blocks: list = []
        self.actual_seq_len = 0
        self.total_blocks = 0
        self.bytes_written = 0
        self.bytes_read = 0
        self.compression_time_ns = 0

        self._tail_k: Optional[torch.Tensor] = None
        self._tail_v: Optional[torch.Tensor] = None
        self._tail_len = 0
        self._flag: Optional[torch.Tensor] = None  # tp_append_stage verdict (pinned host memory)
        self._fused_views = None  # (block_count, storage buffers, (PolarKeyBlock, QuantizedVBlock))
        self._scratch = None  # one-page store for the padded tail when the storage is full
        self._epoch = 0
        # Appends whose non-finite verdict is deferred (append(..., defer_check=True)):
        # (epoch, state before the append), oldest first.
        self._pending: list = []

        self._initialized = False
        self._batch_size: Optional[int] = None
        self._num_kv_heads: Optional[int] = None
        self._head_dim: Optional[int] = None
        self._input_dtype = None

    # ------------------------------------------------------------------
    @property
    def partial_k(self) -> Optional[torch.Tensor]:
        return self._tail_k[:, :, : self._tail_len].clone() if self._tail_len else None

    @property
    def partial_v(self) -> Optional[torch.Tensor]:
        return self._tail_v[:, :, : self._tail_len].clone() if self._tail_len else None

    def _tail_views(self):
        """Views of the valid dense tail (rewritten in place by the next append)."""
        if not self._tail_len:
            return None, None
        return self._tail_k[:, :, : self._tail_len], self._tail_v[:, :, : self._tail_len]

    def _validate_shapes(self, k_new, v_new) -> None:
        # turbo_polar_cache.py:55-68, same order and messages.
        if not isinstance(k_new, torch.Tensor) or not isinstance(v_new, torch.Tensor):
            raise TypeError("append() expects torch.Tensor inputs")
        if k_new.ndim != 4 or v_new.ndim != 4:
            raise ValueError(
                f"append() expects 4-D inputs (B, H_kv, T, D), got {tuple(k_new.shape)} and {tuple(v_new.shape)}"
            )
        if k_new.shape != v_new.shape:
            raise ValueError(f"k_new shape {tuple(k_new.shape)} must match v_new shape {tuple(v_new.shape)}")
        B, H_kv, T_new, D = k_new.shape
        if T_new < 1:
            raise ValueError(f"input must have at least one token, got T={T_new}")
        if k_new.dtype != v_new.dtype:
            raise ValueError(f"k_new dtype {k_new.dtype} must match v_new dtype {v_new.dtype}")
        if k_new.dtype not in (torch.float16, torch.float32):
            raise ValueError(f"only float16 and float32 inputs are supported, got {k_new.dtype}")

    def _invariant_error(self, k_new) -> Optional[ValueError]:
        """The error turbo_polar_cache.py:71-104 would raise, without raising it."""
        B, H_kv, _, D = k_new.shape
        if self._initialized:
            if B != self._batch_size:
                return ValueError(
                    f"batch size changed from {self._batch_size} to {B}; "
                    "TurboPolar cache does not support varying batch size."
                )
            if H_kv != self._num_kv_heads:
                return ValueError(
                    f"KV head count changed from {self._num_kv_heads} to {H_kv}; "
                    "TurboPolar cache does not support varying head counts."
                )
            if D != self._head_dim:
                return ValueError(
                    f"head_dim changed from {self._head_dim} to {D}; "
                    "TurboPolar cache does not support varying head dimension."
                )
            if k_new.dtype != self._input_dtype:
                return ValueError(
                    f"input dtype changed from {self._input_dtype} to {k_new.dtype}; "
                    "TurboPolar cache does not support varying dtype."
                )
        else:
            if H_kv != self.config.num_kv_heads:
                return ValueError(f"input has {H_kv} KV heads but config expects {self.config.num_kv_heads}")
            if D != self.config.head_dim:
                return ValueError(f"input head_dim {D} does not match config {self.config.head_dim}")
        return None

    def _commit_invariants(self, k_new) -> None:
        if not self._initialized:
            B, H_kv, _, D = k_new.shape
            self._batch_size = B
            self._num_kv_heads = H_kv
            self._head_dim = D
            self._input_dtype = k_new.dtype
            self._initialized = True

    def _validate_append_inputs(self, k_new, v_new):
        """turbo_polar_cache.py:55-104 in full (shape, finiteness, invariants)."""
        self._validate_shapes(k_new, v_new)
        if not bool(torch.isfinite(k_new).all()) or not bool(torch.isfinite(v_new).all()):
            raise ValueError("append() inputs must contain finite values")
        err = self._invariant_error(k_new)
        if err is not None:
            raise err
        self._commit_invariants(k_new)

    # ------------------------------------------------------------------
    def _page_bytes(self) -> int:
        """Bytes the reference's _flush_block adds per page (turbo_polar_cache.py:154-161)."""
        B, H = self._batch_size, self._num_kv_heads
        l1_row, deep_row = self.polar_encoder.row_bytes()
        r_item = 1 if self.polar_encoder.use_int8_radii else 2
        k = B * H * PAGE * (self._head_dim // 2) * r_item + B * H * PAGE * (l1_row + deep_row)
        if self.polar_encoder.use_int8_radii:
            k += B * H * 2
        v = B * H * PAGE * self._head_dim + B * H * PAGE * (self._head_dim // 32) * 2
        return k + v

    def _encode_into_storage(self, k: torch.Tensor, v: torch.Tensor, token_begin: int, n_pages: int) -> None:
        B, H = self._batch_size, self._num_kv_heads
        start = self.k_storage.block_count
        self.k_storage.reserve(start + n_pages, self.polar_encoder, B, H, k.device)
        self.v_storage.reserve(start + n_pages, B, H, k.device)
        encode_pages(
            k, v, token_begin, n_pages * PAGE, self.polar_encoder.layout,
            pages_of(self.k_storage, self.v_storage), start,
        )
        self.k_storage.block_count += n_pages
        self.v_storage.block_count += n_pages
        self.total_blocks += n_pages
        self.bytes_written += n_pages * self._page_bytes()

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor, defer_check: bool = False) -> None:
        """turbo_polar_cache.py:106-126: extend the tail, flush every full page.

        On a HIP device one tp_append_stage launch checks the whole input for
        non-finite values and copies the tokens bound for the dense tail, with
        a single 4-byte read back (the reference synchronises once per input
        in mx.isfinite(...).all()).  Errors come in the reference's order and
        leave the cache unchanged.

        ``defer_check`` (no counterpart in the reference; single-token appends
        to an initialised cache on a HIP device, otherwise ignored): the
        non-finite verdict is not waited for, so the call does not drain the
        stream.  ``resolve_deferred_check()`` reads it later; an append found
        non-finite then is undone, with every append after it, and raises the
        reference's ValueError.  Any other call that appends resolves pending
        verdicts first, and so does a deferred one that would restart the
        dense tail (its token would overwrite tail rows an undo restores)."""
        if self._pending and not (defer_check and k_new.ndim == 4 and k_new.shape[2] == 1 and self._tail_len > 0):
            self.resolve_deferred_check()
        self._validate_shapes(k_new, v_new)
        if not (k_new.is_cuda and v_new.is_cuda) or self._invariant_error(k_new) is not None:
            self._validate_append_inputs(k_new, v_new)
            self._append_host_path(k_new, v_new)
            return
        B, H, T, D = k_new.shape
        k_new = k_new.contiguous()
        v_new = v_new.contiguous()
        if self._tail_k is not None and self._tail_k.device != k_new.device:
            raise ValueError(f"append() inputs moved from {self._tail_k.device} to {k_new.device}")
        if self._tail_k is None:
            self._tail_k = torch.zeros((B, H, PAGE, D), dtype=k_new.dtype, device=k_new.device)
            self._tail_v = torch.zeros((B, H, PAGE, D), dtype=k_new.dtype, device=k_new.device)
        if self._flag is None:
            # Written by the staging kernel and read after one synchronisation,
            # with no device-to-host copy.
            self._flag = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        if self._tail_len:
            n_head, head_dst = min(PAGE - self._tail_len, T), self._tail_len
        elif T < PAGE:
            n_head, head_dst = T, 0
        else:
            n_head, head_dst = 0, 0
        # A deferred single token lands at tail position tail_len (< 64) and
        # overwrites nothing valid (a pending append never lets a later one
        # restart the tail at row 0), so restoring the counters undoes it.
        defer = defer_check and T == 1 and self._initialized
        before = self._state() if defer else None
        self._stage(k_new, v_new, 0, n_head, head_dst, check=3 if defer else 2)
        if defer:
            self._pending.append((self._epoch, before))
        self._commit_invariants(k_new)
        self.actual_seq_len += T
        self._tail_len += n_head
        pos = n_head
        if self._tail_len == PAGE:
            self._encode_into_storage(self._tail_k, self._tail_v, 0, 1)
            self._tail_len = 0
        n_full = (T - pos) // PAGE
        if n_full:
            self._encode_into_storage(k_new, v_new, pos, n_full)
            pos += n_full * PAGE
        rem = T - pos
        if rem:
            self._stage(k_new, v_new, pos, rem, 0, check=0)
            self._tail_len = rem

    def _state(self) -> tuple:
        return (self.actual_seq_len, self._tail_len, self.k_storage.block_count, self.v_storage.block_count,
                self.total_blocks, self.bytes_written)

    def deferred_verdict_pending(self) -> bool:
        return bool(self._pending)

    def resolve_deferred_check(self, synchronize: bool = True) -> None:
        """Reads the verdicts of the deferred appends (one stream
        synchronisation unless the caller already synchronised: pass
        ``synchronize=False`` then).  If one found a non-finite value, the cache
        returns to its state before that append (later appends are undone
        too) and the reference's ValueError is raised."""
        if not self._pending:
            return
        if synchronize:
            torch.cuda.current_stream(self._tail_k.device).synchronize()
        bad = self._bad_pending()
        if bad is None:
            self._pending.clear()
            return
        self.rollback_deferred()
        raise ValueError("append() inputs must contain finite values")

    def _bad_pending(self):
        """Index of the first pending append whose verdict is non-finite (the
        stream must have passed the launches), or None."""
        word = int(self._flag[0].item()) & 0xFFFFFFFF
        for i, (epoch, _) in enumerate(self._pending):
            if word == (epoch + 1) & 0xFFFFFFFF:
                return i
        return None

    def rollback_deferred(self) -> None:
        """Undoes every pending deferred append (the cache returns to its state
        before the oldest)."""
        if not self._pending:
            return
        (self.actual_seq_len, self._tail_len, self.k_storage.block_count, self.v_storage.block_count,
         self.total_blocks, self.bytes_written) = self._pending[0][1]
        self._fused_views = None
        self._pending.clear()

    def _stage(self, k, v, begin: int, n: int, dst: int, check: int) -> None:
        B, H, T, _ = k.shape
        # Even epochs: the staging kernel reports epoch (finite) or epoch + 1.
        self._epoch = ((self._epoch + 2) & 0xFFFFFFFE) or 2
        idx = k.device.index
        prev = torch.cuda.current_device()
        if prev != idx:
            torch.cuda.set_device(idx)
        try:
            st = _lib.lib().tp_append_stage(
                k.data_ptr(), v.data_ptr(), 1 if k.dtype == torch.float32 else 0, B * H, T, begin, n,
                self._tail_k.data_ptr(), self._tail_v.data_ptr(), PAGE, dst, check,
                self._flag.data_ptr(), self._epoch, _lib.raw_stream(idx),
            )
        finally:
            if prev != idx:
                torch.cuda.set_device(prev)
        if st == _lib.TP_ERR_NONFINITE:
            raise ValueError("append() inputs must contain finite values")
        _lib.check(st, "tp_append_stage")

    def _append_host_path(self, k_new: torch.Tensor, v_new: torch.Tensor) -> None:
        """Tail bookkeeping with tensor copies (CPU tensors; flushes need HIP)."""
        B, H, T, D = k_new.shape
        self.actual_seq_len += T
        if self._tail_k is None:
            self._tail_k = torch.zeros((B, H, PAGE, D), dtype=k_new.dtype, device=k_new.device)
            self._tail_v = torch.zeros((B, H, PAGE, D), dtype=k_new.dtype, device=k_new.device)
        k_new = k_new.contiguous()
        v_new = v_new.contiguous()
        pos = 0
        if self._tail_len:
            n = min(PAGE - self._tail_len, T)
            self._tail_k[:, :, self._tail_len : self._tail_len + n] = k_new[:, :, :n]
            self._tail_v[:, :, self._tail_len : self._tail_len + n] = v_new[:, :, :n]
            self._tail_len += n
            pos = n
            if self._tail_len == PAGE:
                self._encode_into_storage(self._tail_k, self._tail_v, 0, 1)
                self._tail_len = 0
        n_full = (T - pos) // PAGE
        if n_full:
            self._encode_into_storage(k_new, v_new, pos, n_full)
            pos += n_full * PAGE
        rem = T - pos
        if rem:
            self._tail_k[:, :, :rem] = k_new[:, :, pos:]
            self._tail_v[:, :, :rem] = v_new[:, :, pos:]
            self._tail_len = rem

    # ------------------------------------------------------------------
    def get_fused_attention_inputs(
        self,
    ) -> Tuple[Optional[PolarKeyBlock], Optional[QuantizedVBlock], Optional[torch.Tensor], Optional[torch.Tensor], None, int]:
        """turbo_polar_cache.py:163-198: page views, the dense tail, no QJL."""
        compressed_k = None
        quant_v = None
        if self.k_storage.block_count > 0:
            # The page views are rebuilt only when a page was added or the
            # storage reallocated, so a decode step reuses them (and the device
            # descriptors the bridge attaches to them).  The key holds the
            # buffers themselves, so a freed buffer can never alias a new one.
            bufs = (self.k_storage.radii, self.v_storage.codes)
            key = self.k_storage.block_count
            hit = self._fused_views
            if hit is not None and hit[0] == key and hit[1][0] is bufs[0] and hit[1][1] is bufs[1]:
                compressed_k, quant_v = hit[2]
            else:
                L = self.config.block_size
                compressed_k = self.k_storage.to_unified_block(
                    (self._batch_size, self._num_kv_heads, self.k_storage.block_count * L, self._head_dim)
                )
                quant_v = self.v_storage.to_quantized_block()
                self._fused_views = (key, bufs, (compressed_k, quant_v))
        tail_k, tail_v = self._tail_views()
        return compressed_k, quant_v, tail_k, tail_v, None, self.actual_seq_len

    def _partial_page_store(self) -> Tuple[_lib.TPPages, int, bool]:
        """Encode the zero-padded dense tail as one page (turbo_polar_cache.py:276-319)
        and return ``(tp_pages, slot, in_storage)`` of where it went: the
        storage's first free slot when the capacity has one (``in_storage``;
        the stored pages and the tail page then form one run of slots), else a
        one-page scratch store kept by the runtime.  Either is rewritten by the
        next append."""
        B, H = self._batch_size, self._num_kv_heads
        dev = self._tail_k.device
        ks, vs = self.k_storage, self.v_storage
        in_storage = ks.radii is not None and ks.block_count < ks.capacity
        if in_storage:
            pages, slot = pages_of(ks, vs), ks.block_count
        else:
            sc = self._scratch
            if sc is None or sc["radii"].shape[:2] != (B, H) or sc["radii"].device != dev:
                sc = self.polar_encoder.alloc_pages(B, H, 1, dev)
                sc["v_codes"] = torch.zeros((B, H, 1, PAGE, self._head_dim), dtype=torch.int8, device=dev)
                sc["v_scales"] = torch.zeros((B, H, 1, PAGE, self._head_dim // 32), dtype=torch.float16, device=dev)
                sc["pages"] = _lib.TPPages(
                    _lib.ptr(sc["radii"]), _lib.ptr(sc["radii_scales"]), _lib.ptr(sc["angle_codes_l1"]),
                    _lib.ptr(sc["angle_codes_deep"]), _lib.ptr(sc["v_codes"]), _lib.ptr(sc["v_scales"]), 1,
                )
                self._scratch = sc
            pages, slot = sc["pages"], 0
        # The encoder reads tokens past n_tokens as zeros: the reference's
        # mx.pad zero padding of the tail (turbo_polar_cache.py:282-285).
        encode_pages(self._tail_k, self._tail_v, 0, self._tail_len, self.polar_encoder.layout, pages, slot)
        return pages, slot, in_storage

    def get_blocks_for_attention(self):
        """turbo_polar_cache.py:200-274: the stored pages plus the zero-padded
        tail page, as one key block and one value block of S (+1) pages.

        The tail page is encoded into the storage's first free slot when there
        is one, and the blocks are then views of the storage (no copy of the
        cache; valid until the next append).  Only when the storage is full is
        it encoded into a scratch page and the blocks concatenated."""
        L = self.config.block_size
        n = self.k_storage.block_count
        if n == 0 and not self._tail_len:
            return None, None, None, None, self.actual_seq_len
        shape_of = lambda r: (r.shape[0], r.shape[1], r.shape[2] * r.shape[3], self._head_dim)  # noqa: E731
        if not self._tail_len:
            k = self.k_storage.to_unified_block((self._batch_size, self._num_kv_heads, n * L, self._head_dim))
            return k, self.v_storage.to_quantized_block(), None, None, self.actual_seq_len
        _, _, in_storage = self._partial_page_store()
        ks, vs = self.k_storage, self.v_storage
        if in_storage:
            sl = slice(0, n + 1)
            radii, l1, deep = ks.radii[:, :, sl], ks.angle_codes_l1[:, :, sl], ks.angle_codes_deep[:, :, sl]
            rs = ks.radii_scales[:, :, sl] if ks.radii_scales is not None else None
            codes, scales = vs.codes[:, :, sl], vs.scales[:, :, sl]
        else:
            sc = self._scratch
            radii, l1, deep, rs = sc["radii"], sc["angle_codes_l1"], sc["angle_codes_deep"], sc["radii_scales"]
            codes, scales = sc["v_codes"], sc["v_scales"]
            if n:
                radii = torch.cat([ks.radii[:, :, :n], radii], dim=2)
                l1 = torch.cat([ks.angle_codes_l1[:, :, :n], l1], dim=2)
                deep = torch.cat([ks.angle_codes_deep[:, :, :n], deep], dim=2)
                if rs is not None:
                    rs = torch.cat([ks.radii_scales[:, :, :n], rs], dim=2)
                codes = torch.cat([vs.codes[:, :, :n], codes], dim=2)
                scales = torch.cat([vs.scales[:, :, :n], scales], dim=2)
        key = PolarKeyBlock(radii=radii, angle_codes_l1=l1, angle_codes_deep=deep, radii_scales=rs,
                            shape=shape_of(radii), block_size=L, head_dim=self.config.head_dim,
                            metadata=self.polar_encoder.metadata)
        return key, QuantizedVBlock(codes=codes, scales=scales, group_size=32), None, None, self.actual_seq_len

    def fetch_blocks(self, indices: Optional[list] = None) -> torch.Tensor:
        """turbo_polar_cache.py:321-346: the selected stored pages (all of
        them by default), in the given order, decoded to dense fp16 keys
        ``[B, H, 64 * len(indices), D]`` by one gather launch
        (tp_decode_pages_gather) over the index list.  ``bytes_read`` grows by
        each fetched page's key bytes (radii, both angle rows and, for int8
        radii, the page scale), as the reference counts them per page.

        An index outside [0, block_count) raises IndexError (the reference's
        slice there is empty and its decode of it fails); an empty list
        returns an empty tensor."""
        ks = self.k_storage
        n = ks.block_count
        if n == 0:
            return torch.empty(0)
        idx = list(range(n)) if indices is None else [int(i) for i in indices]
        bad = [i for i in idx if not 0 <= i < n]
        if bad:
            raise IndexError(f"page indices {bad} outside the {n} stored pages")
        B, H, D = self._batch_size, self._num_kv_heads, self._head_dim
        dev = ks.radii.device
        if not idx:
            return torch.empty((B, H, 0, D), dtype=torch.float16, device=dev)
        # Per stored page of every (batch, head): the same per-slice byte counts
        # as _nbytes of the reference's one-page slices.
        per_page = (_nbytes(ks.radii) + _nbytes(ks.angle_codes_l1) + _nbytes(ks.angle_codes_deep)
                    + (_nbytes(ks.radii_scales) if ks.radii_scales is not None else 0)) // ks.capacity
        page_index = torch.tensor(idx, dtype=torch.int32).to(dev, non_blocking=True)
        k, _ = decode_pages_gather(self.polar_encoder.layout, pages_of(ks, self.v_storage), B, H, n, page_index)
        self.bytes_read += per_page * len(idx)
        return k

    def get_io_telemetry(self) -> Dict[str, Any]:
        """turbo_polar_cache.py:348-377 (same keys and closed forms)."""
        if self.k_storage.block_count == 0 and not self._tail_len:
            return {}
        D = self.config.head_dim
        B, H = self._batch_size, self._num_kv_heads
        dense_kv_bytes = B * H * self.actual_seq_len * D * 2 * 2
        compressed = self.bytes_written
        if self._tail_len:
            compressed += 2 * B * H * self._tail_len * D * self._tail_k.element_size()
        return {
            "dense_kv_bytes": dense_kv_bytes,
            "actual_cache_bytes": compressed,
            "compression_ratio": float(dense_kv_bytes / compressed) if compressed > 0 else 0.0,
            "total_blocks": self.total_blocks,
            "partial_tokens": self._tail_len,
            "k_storage_capacity": self.k_storage.capacity,
            "v_storage_capacity": self.v_storage.capacity,
            "k_storage_reallocs": self.k_storage.reallocation_count,
            "v_storage_reallocs": self.v_storage.reallocation_count,
        }

    def reset(self) -> None:
        """turbo_polar_cache.py:379-395."""
        self.k_storage = PolarKBlockStorage()
        self.v_storage = QuantVBlockStorage()
        self.qjl_blocks = []
        self.actual_seq_len = 0
        self.total_blocks = 0
        self.bytes_written = 0
        self.bytes_read = 0
        self.compression_time_ns = 0
        self._tail_k = None
        self._tail_v = None
        self._tail_len = 0
        self._scratch = None
        self._fused_views = None
        self._pending = []
        self._initialized = False
        self._batch_size = None
        self._num_kv_heads = None
        self._head_dim = None
        self._input_dtype = None
