"""TurboPolar configuration contract.

Same fields, defaults, validation order and error messages as
``TurboPolarConfig`` (rfsn_v11/candidates/turbo_polar_config.py:6-55).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any, Dict


@dataclass(frozen=True)
class TurboPolarConfig:
    k_angle_bits_level1: int = 4
    k_angle_bits_deep: int = 4
    use_int8_radii: bool = False
    v_bits: int = 8
    block_size: int = 64
    head_dim: int = 128
    qjl_proj_dim: int = 64
    use_qjl: bool = False
    storage_mode: str = "kv_quant"
    seed: int = 42
    split_dim: int = 64
    attention_scale: float = 0.0  # 0 = 1/sqrt(head_dim)
    num_q_heads: int = 32
    num_kv_heads: int = 8
    metadata: Dict[str, Any] = field(default_factory=dict)

    def __post_init__(self):
        # turbo_polar_config.py:27-55, in the same order.
        if self.block_size <= 0:
            raise ValueError("block_size must be positive")
        if self.head_dim <= 0:
            raise ValueError("head_dim must be positive")
        if self.head_dim % 2 != 0:
            raise ValueError("head_dim must be divisible by 2 for polar pair coordinate mapping")
        if self.qjl_proj_dim <= 0:
            raise ValueError("qjl_proj_dim must be positive")
        if self.qjl_proj_dim % 8 != 0:
            raise ValueError("qjl_proj_dim must be divisible by 8 for bit packing")
        if self.v_bits != 8:
            raise ValueError("v_bits must be 8 (4-bit V quantization is not yet implemented)")
        if self.storage_mode not in {"k_only_first", "kv_quant", "dense_v_debug"}:
            raise ValueError("unknown storage_mode")
        if self.block_size != 64:
            raise ValueError("TurboPolar only supports block_size == 64 in this release")
        if self.head_dim != 128:
            raise ValueError("TurboPolar only supports head_dim == 128 in this release")
        if self.use_qjl:
            raise ValueError("QJL is not supported in this release; set use_qjl=False")
        if self.storage_mode != "kv_quant":
            raise ValueError("TurboPolar only supports storage_mode='kv_quant' in this release")
        if self.split_dim < 0 or self.split_dim > self.head_dim or self.split_dim % 2 != 0:
            raise ValueError("split_dim must be even and within [0, head_dim]")
        if self.num_q_heads % self.num_kv_heads != 0:
            raise ValueError("num_q_heads must be divisible by num_kv_heads for GQA")
        if self.attention_scale == 0.0:
            object.__setattr__(self, "attention_scale", 1.0 / math.sqrt(self.head_dim))
