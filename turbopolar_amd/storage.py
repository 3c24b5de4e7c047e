"""Persistent, capacity-growing page storage on the HIP device.

Mirrors ``PolarKBlockStorage`` and ``QuantVBlockStorage``
(rfsn_v11/generation/storage.py:17-169): structure-of-arrays buffers
``[B, H, capacity, ...]``, lazy allocation at capacity 4, capacity doubling,
``[:block_count]`` views, and the same growth telemetry
(``reallocation_count``, ``bytes_copied_during_growth``).  The HIP encoder
writes pages straight into the slots; a bulk reservation performs the
reference's sequence of doublings as one reallocation and one copy while
reporting the counters the doubling sequence would produce.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional, Tuple

import torch

from . import _lib
from .payload import PolarKeyBlock, QuantizedVBlock


def _doublings(capacity: int, needed: int):
    """Capacities at which the reference would call ``_grow`` to reach ``needed``."""
    caps = []
    while needed > capacity:
        caps.append(capacity)
        capacity *= 2
    return caps, capacity


def _regrow(t: Optional[torch.Tensor], new_cap: int) -> Optional[torch.Tensor]:
    if t is None:
        return None
    shape = list(t.shape)
    shape[2] = new_cap
    out = torch.zeros(shape, dtype=t.dtype, device=t.device)
    out[:, :, : t.shape[2]] = t
    return out


@dataclass
class PolarKBlockStorage:
    radii: Optional[torch.Tensor] = None
    angle_codes_l1: Optional[torch.Tensor] = None
    angle_codes_deep: Optional[torch.Tensor] = None
    radii_scales: Optional[torch.Tensor] = None
    block_count: int = 0
    capacity: int = 0
    metadata: dict = field(default_factory=dict)
    reallocation_count: int = 0
    bytes_copied_during_growth: int = 0

    def _buffers(self):
        return [t for t in (self.radii, self.angle_codes_l1, self.angle_codes_deep, self.radii_scales) if t is not None]

    def reserve(self, needed: int, encoder, B: int, H: int, device, initial_capacity: int = 4) -> None:
        """Make room for ``needed`` pages (storage.py:34-73 growth rule)."""
        if self.radii is None:
            bufs = encoder.alloc_pages(B, H, initial_capacity, device)
            self.radii = bufs["radii"]
            self.angle_codes_l1 = bufs["angle_codes_l1"]
            self.angle_codes_deep = bufs["angle_codes_deep"]
            self.radii_scales = bufs["radii_scales"]
            self.metadata = encoder.metadata
            self.capacity = initial_capacity
        caps, new_cap = _doublings(self.capacity, needed)
        if not caps:
            return
        per_slot = sum(t.numel() * t.element_size() for t in self._buffers()) // self.capacity
        for c in caps:
            self.bytes_copied_during_growth += per_slot * c
        self.reallocation_count += len(caps)
        self.radii = _regrow(self.radii, new_cap)
        self.angle_codes_l1 = _regrow(self.angle_codes_l1, new_cap)
        self.angle_codes_deep = _regrow(self.angle_codes_deep, new_cap)
        self.radii_scales = _regrow(self.radii_scales, new_cap)
        self.capacity = new_cap

    def append(self, block: PolarKeyBlock, initial_capacity: int = 4) -> None:
        """Copy one 4-D page into the next slot (storage.py:75-87)."""
        B, H = block.radii.shape[:2]
        if self.radii is None:
            self.radii = torch.zeros((B, H, initial_capacity) + tuple(block.radii.shape[2:]), dtype=block.radii.dtype, device=block.radii.device)
            self.angle_codes_l1 = torch.zeros((B, H, initial_capacity) + tuple(block.angle_codes_l1.shape[2:]), dtype=torch.uint8, device=block.radii.device)
            self.angle_codes_deep = torch.zeros((B, H, initial_capacity) + tuple(block.angle_codes_deep.shape[2:]), dtype=torch.uint8, device=block.radii.device)
            self.radii_scales = (
                torch.zeros((B, H, initial_capacity, 1, 1), dtype=torch.float16, device=block.radii.device)
                if block.radii_scales is not None else None
            )
            self.metadata = block.metadata
            self.capacity = initial_capacity
        elif self.block_count >= self.capacity:
            self.bytes_copied_during_growth += sum(t.numel() * t.element_size() for t in self._buffers())
            self.reallocation_count += 1
            new_cap = self.capacity * 2
            self.radii = _regrow(self.radii, new_cap)
            self.angle_codes_l1 = _regrow(self.angle_codes_l1, new_cap)
            self.angle_codes_deep = _regrow(self.angle_codes_deep, new_cap)
            self.radii_scales = _regrow(self.radii_scales, new_cap)
            self.capacity = new_cap
        idx = self.block_count
        self.radii[:, :, idx] = block.radii
        self.angle_codes_l1[:, :, idx] = block.angle_codes_l1
        self.angle_codes_deep[:, :, idx] = block.angle_codes_deep
        if self.radii_scales is not None and block.radii_scales is not None:
            self.radii_scales[:, :, idx] = block.radii_scales.reshape(B, H, 1, 1)
        self.block_count += 1

    def to_unified_block(self, shape: Tuple[int, ...]) -> PolarKeyBlock:
        """5-D view of the valid pages (storage.py:89-102)."""
        if self.radii is None or self.block_count == 0:
            raise ValueError("No compressed blocks to materialize")
        n = self.block_count
        return PolarKeyBlock(
            radii=self.radii[:, :, :n],
            angle_codes_l1=self.angle_codes_l1[:, :, :n],
            angle_codes_deep=self.angle_codes_deep[:, :, :n],
            radii_scales=self.radii_scales[:, :, :n] if self.radii_scales is not None else None,
            shape=shape,
            block_size=self.metadata.get("block_size", shape[-1]),
            head_dim=shape[-1],
            metadata=self.metadata,
        )


@dataclass
class QuantVBlockStorage:
    codes: Optional[torch.Tensor] = None
    scales: Optional[torch.Tensor] = None
    group_size: int = 32
    block_count: int = 0
    capacity: int = 0
    reallocation_count: int = 0
    bytes_copied_during_growth: int = 0

    def reserve(self, needed: int, B: int, H: int, device, initial_capacity: int = 4) -> None:
        if self.codes is None:
            # Stored 6-D [B, H, cap, 1, 64, 128] like storage.py:121-131.
            self.codes = torch.zeros((B, H, initial_capacity, 1, 64, 128), dtype=torch.int8, device=device)
            self.scales = torch.zeros((B, H, initial_capacity, 1, 64, 4), dtype=torch.float16, device=device)
            self.capacity = initial_capacity
        caps, new_cap = _doublings(self.capacity, needed)
        if not caps:
            return
        per_slot = (self.codes.numel() + self.scales.numel() * 2) // self.capacity
        for c in caps:
            self.bytes_copied_during_growth += per_slot * c
        self.reallocation_count += len(caps)
        self.codes = _regrow(self.codes, new_cap)
        self.scales = _regrow(self.scales, new_cap)
        self.capacity = new_cap

    def append(self, block: QuantizedVBlock, initial_capacity: int = 4) -> None:
        """Copy one page ``codes [B,H,1,64,128]`` into the next slot (storage.py:149-158)."""
        B, H = block.codes.shape[:2]
        if self.codes is None:
            self.reserve(1, B, H, block.codes.device, initial_capacity)
        elif self.block_count >= self.capacity:
            self.bytes_copied_during_growth += self.codes.numel() + self.scales.numel() * 2
            self.reallocation_count += 1
            self.codes = _regrow(self.codes, self.capacity * 2)
            self.scales = _regrow(self.scales, self.capacity * 2)
            self.capacity *= 2
        idx = self.block_count
        self.codes[:, :, idx] = block.codes.reshape(B, H, 1, 64, 128)
        self.scales[:, :, idx] = block.scales.reshape(B, H, 1, 64, 4)
        self.group_size = block.group_size
        self.block_count += 1

    def to_quantized_block(self) -> QuantizedVBlock:
        """5-D view ``[B, H, S, 64, .]`` of the valid pages (storage.py:160-169)."""
        if self.codes is None or self.block_count == 0:
            raise ValueError("No quantized V blocks to materialize")
        n = self.block_count
        return QuantizedVBlock(
            codes=self.codes[:, :, :n].squeeze(3),
            scales=self.scales[:, :, :n].squeeze(3),
            group_size=self.group_size,
        )


def pages_of(k_storage: PolarKBlockStorage, v_storage: QuantVBlockStorage) -> _lib.TPPages:
    """``tp_pages`` over the whole capacity of a pair of storages."""
    return _lib.TPPages(
        _lib.ptr(k_storage.radii),
        _lib.ptr(k_storage.radii_scales),
        _lib.ptr(k_storage.angle_codes_l1),
        _lib.ptr(k_storage.angle_codes_deep),
        _lib.ptr(v_storage.codes),
        _lib.ptr(v_storage.scales),
        int(k_storage.capacity),
    )
