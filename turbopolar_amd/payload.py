"""Payload types of one or more encoded pages (torch tensors on a HIP device).

``PolarKeyBlock`` mirrors rfsn_v11/quant/polar/payload.py:6-15 and
``QuantizedVBlock`` mirrors rfsn_v11/quant/v_quant/encoder.py:5-9.  Tensors are
4-D ``[B, H, L, .]`` for a single block or 5-D ``[B, H, S, L, .]`` for a
unified run of pages; ``radii_scales`` is ``[B, H, 1, 1]`` / ``[B, H, S, 1, 1]``
fp16 for int8 log radii and None otherwise.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, Optional, Tuple

import torch


@dataclass
class PolarKeyBlock:
    radii: torch.Tensor
    angle_codes_l1: torch.Tensor
    angle_codes_deep: torch.Tensor
    shape: Tuple[int, ...]
    block_size: int
    head_dim: int
    metadata: Dict[str, Any]
    radii_scales: Optional[torch.Tensor] = field(default=None)


@dataclass(frozen=True)
class QuantizedVBlock:
    codes: torch.Tensor
    scales: torch.Tensor
    group_size: int


def packed_row_bytes(n: int, bits: int) -> int:
    """Packed length of n codes (encoder.py:101-130 padding rules)."""
    if bits == 8:
        return n
    if bits == 4:
        return (n + 1) // 2
    if bits == 2:
        return (n + 3) // 4
    raise ValueError(f"unsupported bit width: {bits}")


def layout_metadata(l1_bits: int, deep_bits: int, split_dim: int, int8_radii: bool, head_dim: int = 128):
    """The encoder's metadata dict (rfsn_v11/quant/polar/encoder.py:85-97)."""
    if l1_bits not in (4, 8):
        raise ValueError(f"unsupported k_angle_bits_level1: {l1_bits}")
    if deep_bits not in (2, 4, 8):
        raise ValueError(f"unsupported k_angle_bits_deep: {deep_bits}")
    split_half = split_dim // 2
    return {
        "l1_scale": float(2 ** l1_bits - 1),
        "deep_scale": float(2 ** deep_bits - 1),
        "split_dim": split_dim,
        "l1_packed": l1_bits == 4,
        "deep_packed": deep_bits != 8,
        "deep_bits": deep_bits,
        "l1_bits": l1_bits,
        "int8_radii": bool(int8_radii),
        "log_radii": bool(int8_radii),
        "l1_original_len": split_half,
        "deep_original_len": head_dim // 2 - split_half,
    }


def layout_from_metadata(meta: Dict[str, Any], head_dim: int = 128):
    """(int8_radii, l1_bits, deep_bits, split_dim, l1_row_bytes, deep_row_bytes)."""
    split_dim = int(meta.get("split_dim", head_dim // 2))
    l1_bits = int(meta.get("l1_bits", 4))
    deep_bits = int(meta.get("deep_bits", 2))
    int8 = bool(meta.get("int8_radii", False))
    if int8 and not meta.get("log_radii", int8):
        raise ValueError("int8 radii without log_radii are not produced by the encoder and are unsupported")
    split_half = split_dim // 2
    return (
        int8,
        l1_bits,
        deep_bits,
        split_dim,
        packed_row_bytes(split_half, l1_bits),
        packed_row_bytes(head_dim // 2 - split_half, deep_bits),
    )
