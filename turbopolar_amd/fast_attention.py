"""Decode-step caller of the fused path: ``TurboPolarFastCache``.

Mirrors benchmarks/turbopolar_fast_attention.py:20-229 of the reference
(the mlx_lm cache object): ``decode_attention`` appends one token and runs the
fused HIP attention over compressed pages plus the dense tail;
``update_and_fetch`` is the prefill path (append, then decompress-on-read);
``make_turbo_caches`` builds the benchmark-quality fast layout.

One deliberate difference: with no completed page yet the reference computes
dense MLX attention over the tail (turbopolar_fast_attention.py:150-159); here
the same HIP kernel handles a tail-only cache, so every decode step runs on the
GPU path.
"""

from __future__ import annotations

import dataclasses
from typing import List, Tuple

import torch

from .bridge import HipKernelBridge
from .codecs import GroupedVQuantizer, PolarQuantDecoder
from .config import TurboPolarConfig
from .runtime import TurboPolarKVCacheRuntime


class TurboPolarFastCache:
    def __init__(self, config: TurboPolarConfig):
        self.config = config
        self.runtime = TurboPolarKVCacheRuntime(config)
        self.bridge = HipKernelBridge()
        self.decoder = PolarQuantDecoder()
        self.v_dequantizer = GroupedVQuantizer(group_size=32)
        self.qjl_encoder = None

    @property
    def offset(self) -> int:
        return self.runtime.actual_seq_len

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """Prefill: append, then return the decompressed history (turbopolar_fast_attention.py:56-86)."""
        original_dtype = keys.dtype
        if keys.dtype != torch.float16:
            keys = keys.to(torch.float16)
        if values.dtype != torch.float16:
            values = values.to(torch.float16)
        self.runtime.append(keys, values)
        block, quant_v, dense_v, _qjl, actual_len = self.runtime.get_blocks_for_attention()
        if block is None:
            raise RuntimeError("TurboPolar cache returned no blocks after append")
        k_dense = self.decoder.decode_block(block)[:, :, :actual_len, :]
        B, H_kv, S, L, _ = block.radii.shape
        if quant_v is None:
            raise RuntimeError("TurboPolar cache has no V payload")
        v_full = self.v_dequantizer.dequantize_block(quant_v).reshape(B, H_kv, S * L, self.config.head_dim)
        v_dense = v_full[:, :, :actual_len, :]
        if original_dtype != k_dense.dtype:
            k_dense = k_dense.to(original_dtype)
            v_dense = v_dense.to(original_dtype)
        return k_dense, v_dense

    @staticmethod
    def _validate_decode_shape(q, k_new, v_new, config: TurboPolarConfig) -> None:
        # turbopolar_fast_attention.py:89-104, same messages.
        if q.ndim != 4 or k_new.ndim != 4 or v_new.ndim != 4:
            raise ValueError("decode_attention inputs must be 4-D (B, H, T, D)")
        B, H_q, T, D = q.shape
        _, H_kv, T_k, _ = k_new.shape
        _, _, T_v, _ = v_new.shape
        if B != 1:
            raise NotImplementedError("TurboPolar fused decode only supports batch size 1.")
        if T != 1 or T_k != 1 or T_v != 1:
            raise ValueError("decode_attention only supports a single query/key/value token")
        if D != 128:
            raise NotImplementedError("TurboPolar fused decode only supports head_dim == 128.")
        if D != config.head_dim:
            raise ValueError(f"decode_attention head_dim {D} does not match config {config.head_dim}")
        if H_q % H_kv != 0:
            raise ValueError(f"decode_attention requires GQA ratio to divide evenly, got {H_q} and {H_kv}")

    def decode_attention(self, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, scale: float) -> torch.Tensor:
        """Append one token and attend (turbopolar_fast_attention.py:106-188). Returns ``[B, H_q, D]``."""
        self._validate_decode_shape(q, k_new, v_new, self.config)
        if k_new.dtype != torch.float16:
            k_new = k_new.to(torch.float16)
        if v_new.dtype != torch.float16:
            v_new = v_new.to(torch.float16)
        self.runtime.append(k_new, v_new)
        block, quant_v, tail_k, tail_v, _qjl, actual_seq_len = self.runtime.get_fused_attention_inputs()
        if block is None and tail_k is None:
            raise RuntimeError("TurboPolar cache returned no blocks after append")
        q_squeezed = q.squeeze(2)
        cfg = self._config_for_scale(scale)
        if block is not None and quant_v is None:
            raise RuntimeError("Fused attention requires kv_quant storage mode")
        if tail_k is not None and tail_k.shape[2] > 0:
            out, _ = self.bridge.execute_online_attention_quant_v_dense_tail(
                q_squeezed, block, quant_v, tail_k, tail_v, None, None, cfg, actual_seq_len, False
            )
        else:
            out, _ = self.bridge.execute_online_attention_quant_v(
                q_squeezed, block, quant_v, None, None, cfg, actual_seq_len, False
            )
        return out

    def _config_for_scale(self, scale: float) -> TurboPolarConfig:
        """The config with attention_scale = scale (turbopolar_fast_attention.py:147),
        built once per scale value."""
        hit = self.__dict__.get("_scaled_config")
        if hit is None or hit[0] != scale or hit[1] is not self.config:
            hit = (scale, self.config, dataclasses.replace(self.config, attention_scale=scale))
            self.__dict__["_scaled_config"] = hit
        return hit[2]

    def size(self) -> int:
        return self.offset

    @property
    def nbytes(self) -> int:
        return int(self.runtime.get_io_telemetry().get("actual_cache_bytes", 0))

    def empty(self) -> bool:
        return self.offset == 0


def make_turbo_caches(
    num_layers: int,
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
    use_qjl: bool = False,
) -> List[TurboPolarFastCache]:
    """Fast layout caches (turbopolar_fast_attention.py:207-229)."""
    if head_dim not in (64, 128):
        raise ValueError(f"TurboPolar only supports head_dim 64 or 128, got {head_dim}")
    config = TurboPolarConfig(
        num_q_heads=num_q_heads,
        num_kv_heads=num_kv_heads,
        head_dim=head_dim,
        block_size=64,
        qjl_proj_dim=32 if head_dim == 64 else 64,
        use_qjl=use_qjl,
        storage_mode="kv_quant",
        use_int8_radii=True,
        k_angle_bits_deep=8,
        split_dim=0,
    )
    return [TurboPolarFastCache(config) for _ in range(num_layers)]
