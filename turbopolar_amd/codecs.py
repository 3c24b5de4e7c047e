"""Key/value codecs backed by the HIP kernels.

Same class and method names as the reference codecs:
``PolarQuantEncoder.encode_block`` (rfsn_v11/quant/polar/encoder.py:24-98),
``PolarQuantDecoder.decode_block`` (rfsn_v11/quant/polar/decoder.py:7-67) and
``GroupedVQuantizer.quantize_block`` / ``dequantize_block``
(rfsn_v11/quant/v_quant/encoder.py:16-38).  Inputs are torch tensors on a HIP
device; there is no CPU path.
"""

from __future__ import annotations

import torch

from . import _lib
from .kernels import HEAD_DIM, PAGE, PageSet, decode_pages, encode_pages
from .payload import PolarKeyBlock, QuantizedVBlock, layout_metadata, packed_row_bytes


class PolarQuantEncoder:
    def __init__(self, config):
        self.config = config
        self.head_dim = config.head_dim
        self.block_size = config.block_size
        self.split_dim = getattr(config, "split_dim", config.head_dim // 2)
        self.k_angle_bits_level1 = config.k_angle_bits_level1
        self.k_angle_bits_deep = config.k_angle_bits_deep
        self.l1_levels = 2 ** self.k_angle_bits_level1
        self.deep_levels = 2 ** self.k_angle_bits_deep
        self.l1_scale = float(self.l1_levels - 1)
        self.deep_scale = float(self.deep_levels - 1)
        self.use_int8_radii = bool(getattr(config, "use_int8_radii", False))

    @property
    def metadata(self):
        return layout_metadata(
            self.k_angle_bits_level1, self.k_angle_bits_deep, self.split_dim, self.use_int8_radii, self.head_dim
        )

    @property
    def layout(self):
        return _lib.make_layout(self.use_int8_radii, self.k_angle_bits_level1, self.k_angle_bits_deep, self.split_dim)

    def row_bytes(self):
        split_half = self.split_dim // 2
        return (
            packed_row_bytes(split_half, self.k_angle_bits_level1),
            packed_row_bytes(self.head_dim // 2 - split_half, self.k_angle_bits_deep),
        )

    def alloc_pages(self, B: int, H: int, n_pages: int, device) -> dict:
        """Zeroed page buffers ``[B, H, n_pages, 64, .]`` for this layout."""
        l1_row, deep_row = self.row_bytes()
        rdt = torch.int8 if self.use_int8_radii else torch.float16
        return {
            "radii": torch.zeros((B, H, n_pages, PAGE, self.head_dim // 2), dtype=rdt, device=device),
            "angle_codes_l1": torch.zeros((B, H, n_pages, PAGE, l1_row), dtype=torch.uint8, device=device),
            "angle_codes_deep": torch.zeros((B, H, n_pages, PAGE, deep_row), dtype=torch.uint8, device=device),
            "radii_scales": (
                torch.zeros((B, H, n_pages, 1, 1), dtype=torch.float16, device=device) if self.use_int8_radii else None
            ),
        }

    def encode_block(self, k_block: torch.Tensor) -> PolarKeyBlock:
        """Encode ``[B, H, L, D]`` keys into a single (4-D) block."""
        B, H, L, D = k_block.shape
        assert D == self.head_dim
        assert D % 2 == 0
        meta = self.metadata  # raises ValueError for unsupported bit widths
        n_pages = (L + PAGE - 1) // PAGE
        # The page encoder takes one log scale per 64-token page; a block of
        # another length (one scale over all of it, encoder.py:34-42) is
        # encoded with fp16 radii, whose logs tp_log_radii_rows then codes.
        whole_row_log = self.use_int8_radii and L != PAGE
        bufs = self.alloc_pages(B, H, n_pages, k_block.device)
        layout = self.layout
        if whole_row_log:
            bufs["radii"] = torch.zeros((B, H, n_pages, PAGE, D // 2), dtype=torch.float16, device=k_block.device)
            layout = _lib.make_layout(False, self.k_angle_bits_level1, self.k_angle_bits_deep, self.split_dim)
        pages = _lib.TPPages(
            _lib.ptr(bufs["radii"]), None if whole_row_log else _lib.ptr(bufs["radii_scales"]),
            _lib.ptr(bufs["angle_codes_l1"]), _lib.ptr(bufs["angle_codes_deep"]), None, None, n_pages,
        )
        encode_pages(k_block.contiguous(), None, 0, L, layout, pages, 0)

        def tokens(t):
            return t.reshape(B, H, n_pages * PAGE, t.shape[-1])[:, :, :L]

        scales = bufs["radii_scales"]
        radii = tokens(bufs["radii"])
        if whole_row_log:
            r16 = radii.contiguous()
            radii = torch.empty(r16.shape, dtype=torch.int8, device=r16.device)
            scales = torch.empty((B, H), dtype=torch.float16, device=r16.device)
            with _lib.on_device(r16.device):
                st = _lib.lib().tp_log_radii_rows(r16.data_ptr(), B * H, L * (D // 2), radii.data_ptr(),
                                                  scales.data_ptr(), _lib.stream_handle(r16.device))
            _lib.check(st, "tp_log_radii_rows")

        return PolarKeyBlock(
            radii=radii,
            angle_codes_l1=tokens(bufs["angle_codes_l1"]),
            angle_codes_deep=tokens(bufs["angle_codes_deep"]),
            shape=(B, H, L, D),
            block_size=L,
            head_dim=D,
            radii_scales=scales.reshape(B, H, 1, 1) if scales is not None else None,
            metadata=meta,
        )


def _pad_tokens(t: torch.Tensor, L: int) -> torch.Tensor:
    """Zero-pad dim 3 (tokens per page) of a 5-D page tensor up to 64."""
    if L == PAGE:
        return t
    shape = list(t.shape)
    shape[3] = PAGE
    out = torch.zeros(shape, dtype=t.dtype, device=t.device)
    out[:, :, :, :L] = t
    return out


class PolarQuantDecoder:
    def decode_block(self, block: PolarKeyBlock) -> torch.Tensor:
        """Dense fp16 ``[B, H, S*L, D]`` keys of a 4-D or 5-D block."""
        radii, l1, deep, rs = block.radii, block.angle_codes_l1, block.angle_codes_deep, block.radii_scales
        if radii.dim() == 4:
            radii, l1, deep = radii.unsqueeze(2), l1.unsqueeze(2), deep.unsqueeze(2)
            rs = rs.unsqueeze(2) if rs is not None else None
        B, H, S, L, _ = radii.shape
        if L > PAGE:
            raise ValueError(f"pages hold at most {PAGE} tokens, got {L}")
        view = PolarKeyBlock(
            radii=_pad_tokens(radii, L),
            angle_codes_l1=_pad_tokens(l1, L),
            angle_codes_deep=_pad_tokens(deep, L),
            shape=block.shape,
            block_size=PAGE,
            head_dim=block.head_dim,
            metadata=block.metadata,
            radii_scales=rs,
        )
        k, _ = decode_pages(PageSet(view, None, block.head_dim), want_k=True, want_v=False)
        if L != PAGE:
            k = k.reshape(B, H, S, PAGE, block.head_dim)[:, :, :, :L].reshape(B, H, S * L, block.head_dim)
        return k


class GroupedVQuantizer:
    def __init__(self, group_size: int = 32):
        self.group_size = group_size

    def quantize_block(self, v_block: torch.Tensor) -> QuantizedVBlock:
        """Grouped int8 codes ``[B, H, S, L, D]`` and fp16 scales ``[B, H, S, L, D/32]``."""
        B, H, S, L, D = v_block.shape
        assert D % self.group_size == 0
        if self.group_size != 32 or D != HEAD_DIM:
            return self._quantize_groups(v_block)
        T = S * L
        n_pages = (T + PAGE - 1) // PAGE
        dev = v_block.device
        codes = torch.zeros((B, H, n_pages, PAGE, D), dtype=torch.int8, device=dev)
        scales = torch.zeros((B, H, n_pages, PAGE, D // 32), dtype=torch.float16, device=dev)
        pages = _lib.TPPages(None, None, None, None, _lib.ptr(codes), _lib.ptr(scales), n_pages)
        layout = _lib.make_layout(False, 4, 4, 64)
        encode_pages(None, v_block.reshape(B, H, T, D).contiguous(), 0, T, layout, pages, 0)
        codes = codes.reshape(B, H, n_pages * PAGE, D)[:, :, :T].reshape(B, H, S, L, D)
        scales = scales.reshape(B, H, n_pages * PAGE, D // 32)[:, :, :T].reshape(B, H, S, L, D // 32)
        return QuantizedVBlock(codes=codes, scales=scales, group_size=self.group_size)

    def _quantize_groups(self, v_block: torch.Tensor) -> QuantizedVBlock:
        """Any group size dividing D (tp_quantize_v_groups)."""
        B, H, S, L, D = v_block.shape
        _lib.require_hip(v_block, "v_block")
        if v_block.dtype not in (torch.float16, torch.float32):
            raise ValueError(f"quantize_block expects float16 or float32, got {v_block.dtype}")
        v = v_block.contiguous()
        codes = torch.empty(v.shape, dtype=torch.int8, device=v.device)
        scales = torch.empty((B, H, S, L, D // self.group_size), dtype=torch.float16, device=v.device)
        with _lib.on_device(v.device):
            st = _lib.lib().tp_quantize_v_groups(v.data_ptr(), 1 if v.dtype == torch.float32 else 0, B * H * S * L, D,
                                                 self.group_size, codes.data_ptr(), scales.data_ptr(),
                                                 _lib.stream_handle(v.device))
        _lib.check(st, "tp_quantize_v_groups")
        return QuantizedVBlock(codes=codes, scales=scales, group_size=self.group_size)

    def dequantize_block(self, block: QuantizedVBlock) -> torch.Tensor:
        """Dense fp16 ``[B, H, S, L, D]`` values."""
        B, H, S, L, D = block.codes.shape
        if block.group_size != 32 or D != HEAD_DIM:
            # f16(f32(code) * f32(scale)) on the device: the product of an int8
            # and an fp16 is exact in fp32, so this rounds once, as the page decoder.
            _lib.require_hip(block.codes, "codes")
            g = block.group_size
            prod = block.codes.reshape(B, H, S, L, D // g, g).float() * block.scales.float()[..., None]
            return prod.reshape(B, H, S, L, D).half()
        if L > PAGE:
            raise ValueError(f"pages hold at most {PAGE} tokens, got {L}")
        view = QuantizedVBlock(
            codes=_pad_tokens(block.codes, L), scales=_pad_tokens(block.scales, L), group_size=block.group_size
        )
        _, v = decode_pages(PageSet(None, view), want_k=False, want_v=True)
        return v.reshape(B, H, S, PAGE, D)[:, :, :, :L]
