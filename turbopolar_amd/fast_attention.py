"""``TurboPolarFastCache`` -- one decoder layer's compressed KV cache as a
generation loop drives it -- and ``make_turbo_caches``.

Interface of the reference's mlx_lm cache object
(benchmarks/turbopolar_fast_attention.py:20-229): the class, its attributes and
method names, the meaning of every argument, the validation messages of
``_validate_decode_shape`` (:89-104) and the layout ``make_turbo_caches``
builds (:207-229).  The mechanism is this library's own:

* ``decode_attention`` appends the token through the runtime (one staging
  launch; a page encode when the token completes a page) and launches the
  split-K decode kernel straight over the runtime's page store, used in place
  with its capacity as the page stride, and over the runtime's dense-tail
  buffer.  The store's ``tp_pages`` descriptor is kept until the store moves
  (growth or reset).  A cache with no completed page runs the same kernel over
  the tail alone (the reference switches to dense MLX attention there, :150-159).
* ``update_and_fetch`` (prefill) appends, encodes the zero-padded tail as one
  page (the reference's ``_maybe_encode_partial``) and decodes the stored
  pages and that page side by side into one fp16 K and one fp16 V buffer
  (``tp_decode_pages_into``), returning views of its first ``offset`` tokens.
  Nothing the size of the cache is copied besides that output.
"""

from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from .bridge import HipKernelBridge
from .codecs import GroupedVQuantizer, PolarQuantDecoder
from .config import TurboPolarConfig
from .kernels import HEAD_DIM, PAGE, decode_attention_store, decode_pages_into, fp16_scale
from .runtime import TurboPolarKVCacheRuntime
from .storage import pages_of


class TurboPolarFastCache:
    def __init__(self, config: TurboPolarConfig):
        self.config = config
        self.runtime = TurboPolarKVCacheRuntime(config)
        # The reference's attributes: the kernel bridge (the decode step here
        # launches the kernel without it), the codecs, and no QJL encoder
        # (the config rejects QJL).
        self.bridge = HipKernelBridge()
        self.decoder = PolarQuantDecoder()
        self.v_dequantizer = GroupedVQuantizer(group_size=32)
        self.qjl_encoder = None
        self._store = None  # (radii buffer, V codes buffer, their tp_pages)
        self._scale = (None, None)  # (scale given, the fp16 scale the kernel takes)

    @property
    def offset(self) -> int:
        """Tokens held (the position the next token's RoPE uses)."""
        return self.runtime.actual_seq_len

    def _store_pages(self):
        """tp_pages of the runtime's page store, rebuilt when its buffers move."""
        ks, vs = self.runtime.k_storage, self.runtime.v_storage
        hit = self._store
        if hit is None or hit[0] is not ks.radii or hit[1] is not vs.codes:
            hit = (ks.radii, vs.codes, pages_of(ks, vs))
            self._store = hit
        return hit[2]

    # ------------------------------------------------------------------ prefill
    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """Append ``[B, H_kv, T, D]`` keys/values and return the whole history
        decompressed (turbopolar_fast_attention.py:56-86): the stored pages and
        the zero-padded tail page decoded exactly as the reference's
        ``decode_block`` / ``dequantize_block`` do, cut to ``offset`` tokens,
        in the dtype of ``keys``."""
        want = keys.dtype
        rt = self.runtime
        rt.append(keys.to(torch.float16), values.to(torch.float16))
        n_pages, tail = rt.k_storage.block_count, rt._tail_len
        if n_pages == 0 and tail == 0:
            raise RuntimeError("TurboPolar cache returned no blocks after append")
        B, H = rt._batch_size, rt._num_kv_heads
        slots = n_pages + (1 if tail else 0)
        dev = rt._tail_k.device
        k_out = torch.empty((B, H, slots * PAGE, HEAD_DIM), dtype=torch.float16, device=dev)
        v_out = torch.empty_like(k_out)
        layout = rt.polar_encoder.layout
        run = n_pages
        if tail:
            pages, slot, in_storage = rt._partial_page_store()
            if in_storage:  # the tail page sits in the store's next free slot
                run = n_pages + 1
            else:
                decode_pages_into(layout, pages, B * H, slot, 1, k_out, v_out, n_pages * PAGE)
        if run:
            decode_pages_into(layout, self._store_pages(), B * H, 0, run, k_out, v_out, 0)
        k, v = k_out[:, :, : rt.actual_seq_len], v_out[:, :, : rt.actual_seq_len]
        if want != torch.float16:
            k, v = k.to(want), v.to(want)
        return k, v

    # ------------------------------------------------------------------ decode
    @staticmethod
    def _validate_decode_shape(q, k_new, v_new, config: TurboPolarConfig) -> None:
        """The reference's decode-shape contract (turbopolar_fast_attention.py:89-104):
        same checks, exception types and messages."""
        if any(t.ndim != 4 for t in (q, k_new, v_new)):
            raise ValueError("decode_attention inputs must be 4-D (B, H, T, D)")
        B, H_q, T, D = q.shape
        H_kv, T_k, T_v = k_new.shape[1], k_new.shape[2], v_new.shape[2]
        if B != 1:
            raise NotImplementedError("TurboPolar fused decode only supports batch size 1.")
        if (T, T_k, T_v) != (1, 1, 1):
            raise ValueError("decode_attention only supports a single query/key/value token")
        if D != 128:
            raise NotImplementedError("TurboPolar fused decode only supports head_dim == 128.")
        if D != config.head_dim:
            raise ValueError(f"decode_attention head_dim {D} does not match config {config.head_dim}")
        if H_q % H_kv != 0:
            raise ValueError(f"decode_attention requires GQA ratio to divide evenly, got {H_q} and {H_kv}")

    def decode_attention(self, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                         scale: float, defer_check: bool = False) -> torch.Tensor:
        """One decode step (turbopolar_fast_attention.py:106-188): append the
        token's K/V ``[1, H_kv, 1, 128]`` and attend ``q`` ``[1, H_q, 1, 128]``
        over every cached token with ``scale`` (taken as fp16, as the
        reference's kernels receive it).  Returns fp16 ``[1, H_q, 128]``.

        ``defer_check``: the append's non-finite verdict is read later by
        ``runtime.resolve_deferred_check()`` instead of now (no stream drain
        per step; the transformers hook resolves every layer once per forward)."""
        self._validate_decode_shape(q, k_new, v_new, self.config)
        rt = self.runtime
        rt.append(k_new.to(torch.float16), v_new.to(torch.float16), defer_check=defer_check)
        if self._scale[0] != scale:
            self._scale = (scale, fp16_scale(scale))
        n_pages = rt.k_storage.block_count
        tail_k, tail_v = rt._tail_views()
        pages = self._store_pages() if n_pages else None
        layout = rt.polar_encoder.layout
        return decode_attention_store(q[:, :, 0], layout, pages, n_pages, rt._num_kv_heads, tail_k, tail_v,
                                      rt.actual_seq_len, self._scale[1])

    # ------------------------------------------------------------------ mlx_lm cache protocol
    def size(self) -> int:
        return self.offset

    @property
    def nbytes(self) -> int:
        return int(self.runtime.get_io_telemetry().get("actual_cache_bytes", 0))

    def empty(self) -> bool:
        return self.offset == 0


def make_turbo_caches(num_layers: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                      use_qjl: bool = False) -> List[TurboPolarFastCache]:
    """One cache per layer in the benchmark layout of the reference
    (turbopolar_fast_attention.py:207-229): int8 log radii, split 0, 8-bit
    deep angles, quantised V, pages of 64."""
    if head_dim not in (64, 128):
        raise ValueError(f"TurboPolar only supports head_dim 64 or 128, got {head_dim}")
    config = TurboPolarConfig(
        num_q_heads=num_q_heads, num_kv_heads=num_kv_heads, head_dim=head_dim, block_size=64,
        qjl_proj_dim=32 if head_dim == 64 else 64, use_qjl=use_qjl, storage_mode="kv_quant",
        use_int8_radii=True, k_angle_bits_deep=8, split_dim=0,
    )
    return [TurboPolarFastCache(config) for _ in range(num_layers)]
