"""Launch wrappers: torch tensors -> the C ABI of libturbopolar_hip.so.

All device memory is owned by torch; the library never allocates.  Each call is
enqueued on the current torch stream of the tensors' device.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import numpy as np
import torch

from . import _lib
from ._lib import TPPages, check, lib, on_device, ptr, require_hip, stream_handle
from .payload import PolarKeyBlock, QuantizedVBlock, layout_from_metadata

PAGE = 64
HEAD_DIM = 128
PAIRS = 64
V_GROUPS = 4


def fp16_scale(scale: float) -> float:
    """The attention scale as the reference kernels receive it: a 0-d fp16
    array (rfsn_v11/kernels/turbo_polar/metal.py:518,692,774)."""
    return float(np.float16(scale))


# --------------------------------------------------------------------------
# page stores
# --------------------------------------------------------------------------

def _head_stride_pages(t: torch.Tensor, page_elems: int) -> Optional[int]:
    """Page slots between consecutive (batch, head) rows of a page tensor
    ``[B, H, S, ...]``; None when only one (batch, head) exists."""
    B, H = t.shape[0], t.shape[1]
    if H > 1:
        if B > 1 and t.stride(0) != H * t.stride(1):
            return -1
        st = t.stride(1)
    elif B > 1:
        st = t.stride(0)
    else:
        return None
    if st % page_elems:
        return -1
    return st // page_elems


def _inner_ok(t: torch.Tensor, inner_shape: Tuple[int, ...]) -> bool:
    """Dims 2.. are a dense run of pages of ``inner_shape``."""
    expect = 1
    for d in range(t.dim() - 1, 2, -1):
        if t.shape[d] > 1 and t.stride(d) != expect:
            return False
        expect *= t.shape[d]
    if t.shape[2] > 1 and t.stride(2) != expect:
        return False
    return tuple(t.shape[3:]) == inner_shape


def _fresh(t: torch.Tensor) -> torch.Tensor:
    out = torch.empty(t.shape, dtype=t.dtype, device=t.device)
    out.copy_(t)
    return out


class PageSet:
    """Device pointers (``tp_pages``) of a run of S pages per (batch, kv head),
    taken from 5-D page views (``[B, H, S, 64, .]``).  Views into a larger
    capacity buffer are used in place; anything else is copied once into a
    dense buffer, as the reference's ``_ensure_contiguous`` does."""

    def __init__(self, block: Optional[PolarKeyBlock], quant_v: Optional[QuantizedVBlock], head_dim: int = HEAD_DIM):
        self.keep = []
        tensors = {}
        if block is not None:
            int8, l1b, deepb, split, l1_row, deep_row = layout_from_metadata(block.metadata, head_dim)
            self.layout = _lib.make_layout(int8, l1b, deepb, split)
            self.l1_row, self.deep_row = l1_row, deep_row
            radii = block.radii
            if radii.dim() == 4:
                radii = radii.unsqueeze(2)
            if int8 and radii.dtype != torch.int8:
                raise ValueError(f"unsupported radii dtype: {radii.dtype}")
            if not int8 and radii.dtype != torch.float16:
                raise ValueError(f"unsupported radii dtype: {radii.dtype}")
            if int8 and block.radii_scales is None:
                raise ValueError("int8 radii require radii_scales")
            self.B, self.H, self.S = radii.shape[0], radii.shape[1], radii.shape[2]
            if radii.shape[3] != PAGE:
                raise ValueError(f"pages must hold {PAGE} tokens, got {radii.shape[3]}")
            tensors["radii"] = (radii, (PAGE, PAIRS))
            l1 = block.angle_codes_l1
            deep = block.angle_codes_deep
            if l1.dim() == 4:
                l1 = l1.unsqueeze(2)
                deep = deep.unsqueeze(2)
            tensors["angle_l1"] = (l1, (PAGE, l1_row))
            tensors["angle_deep"] = (deep, (PAGE, deep_row))
            if int8:
                rs = block.radii_scales
                if rs.dim() == 4:
                    rs = rs.unsqueeze(2)
                tensors["radii_scales"] = (rs.reshape(rs.shape[0], rs.shape[1], rs.shape[2], 1, 1), (1, 1))
        if quant_v is not None:
            codes, scales = quant_v.codes, quant_v.scales
            if codes.dim() == 4:
                codes = codes.unsqueeze(2)
                scales = scales.unsqueeze(2)
            if quant_v.group_size != 32 or codes.shape[-1] != HEAD_DIM:
                raise ValueError("quantised V must use groups of 32 over head_dim 128")
            if block is None:
                self.B, self.H, self.S = codes.shape[0], codes.shape[1], codes.shape[2]
            elif tuple(codes.shape[:3]) != (self.B, self.H, self.S):
                raise ValueError(f"K pages {(self.B, self.H, self.S)} and V pages {tuple(codes.shape[:3])} differ")
            tensors["v_codes"] = (codes, (PAGE, HEAD_DIM))
            tensors["v_scales"] = (scales, (PAGE, V_GROUPS))
        caps = set()
        for name, (t, inner) in tensors.items():
            require_hip(t, name)
            elems = int(np.prod(inner))
            if elems == 0:
                continue
            cap = _head_stride_pages(t, elems)
            if cap == -1 or not _inner_ok(t, inner) or (cap is not None and cap < self.S):
                t = _fresh(t)
                tensors[name] = (t, inner)
                cap = _head_stride_pages(t, elems)
            caps.add(cap)
        caps.discard(None)
        if len(caps) > 1:
            # Buffers disagree on capacity: copy everything dense.
            for name, (t, inner) in list(tensors.items()):
                if int(np.prod(inner)):
                    tensors[name] = (_fresh(t), inner)
            caps = {self.S}
        self.capacity = caps.pop() if caps else self.S
        self.tensors = {k: v[0] for k, v in tensors.items()}
        self.keep = list(self.tensors.values())
        self.pages = TPPages(
            ptr(self.tensors.get("radii")),
            ptr(self.tensors.get("radii_scales")),
            ptr(self.tensors.get("angle_l1")),
            ptr(self.tensors.get("angle_deep")),
            ptr(self.tensors.get("v_codes")),
            ptr(self.tensors.get("v_scales")),
            int(self.capacity),
        )


# --------------------------------------------------------------------------
# kernel calls
# --------------------------------------------------------------------------

def encode_pages(
    k: Optional[torch.Tensor],
    v: Optional[torch.Tensor],
    token_begin: int,
    n_tokens: int,
    layout,
    pages: TPPages,
    page_begin: int,
) -> None:
    """tp_encode_pages over ``k``/``v`` of shape ``[B, H, T, 128]`` (contiguous,
    fp16 or fp32)."""
    ref = k if k is not None else v
    require_hip(ref, "k/v")
    if ref.dtype not in (torch.float16, torch.float32):
        raise ValueError(f"only float16 and float32 inputs are supported, got {ref.dtype}")
    for t in (k, v):
        if t is not None and (not t.is_contiguous() or t.dtype != ref.dtype or t.shape != ref.shape):
            raise ValueError("k and v must be contiguous tensors of one dtype and shape")
    B, H, T, D = ref.shape
    if D != HEAD_DIM:
        raise ValueError(f"head_dim must be {HEAD_DIM}, got {D}")
    in_dtype = 1 if ref.dtype == torch.float32 else 0
    with on_device(ref.device):
        st = lib().tp_encode_pages(
            ptr(k), ptr(v), in_dtype, B * H, T, int(token_begin), int(n_tokens),
            ctypes.byref(layout), ctypes.byref(pages), int(page_begin), stream_handle(ref.device),
        )
    check(st, "tp_encode_pages")


def decode_pages_into(layout, pages: TPPages, bh: int, page_begin: int, n_pages: int,
                      k_out: Optional[torch.Tensor], v_out: Optional[torch.Tensor], out_offset: int) -> None:
    """tp_decode_pages_into: pages [page_begin, page_begin + n_pages) of every
    (batch, head) row into tokens [out_offset, out_offset + 64 n_pages) of
    ``k_out`` / ``v_out`` (fp16 ``[B, H, T, 128]``, contiguous)."""
    ref = k_out if k_out is not None else v_out
    for t in (k_out, v_out):
        if t is not None and (t.dtype != torch.float16 or not t.is_contiguous() or t.shape != ref.shape):
            raise ValueError("k_out / v_out must be contiguous fp16 tensors of one shape")
    dev = ref.device
    with on_device(dev):
        st = lib().tp_decode_pages_into(
            ctypes.byref(layout), ctypes.byref(pages), int(bh), int(page_begin), int(n_pages), ptr(k_out), ptr(v_out),
            int(ref.shape[2]), int(out_offset), stream_handle(dev),
        )
    check(st, "tp_decode_pages_into")


def decode_pages_gather(layout, pages: TPPages, B: int, H: int, n_stored: int, page_index: torch.Tensor,
                        want_k: bool = True, want_v: bool = False):
    """tp_decode_pages_gather: the stored pages ``page_index`` (a device int32
    tensor, every entry in [0, n_stored)) of every (batch, head) row, in that
    order, as dense fp16 ``[B, H, len(page_index)*64, 128]`` K and/or V."""
    if page_index.dtype != torch.int32 or page_index.dim() != 1 or not page_index.is_contiguous():
        raise ValueError("page_index must be a contiguous 1-D int32 tensor")
    require_hip(page_index, "page_index")
    n = int(page_index.shape[0])
    dev = page_index.device
    shape = (B, H, n * PAGE, HEAD_DIM)
    k_out = torch.empty(shape, dtype=torch.float16, device=dev) if want_k else None
    v_out = torch.empty(shape, dtype=torch.float16, device=dev) if want_v else None
    with on_device(dev):
        st = lib().tp_decode_pages_gather(
            ctypes.byref(layout), ctypes.byref(pages), B * H, int(n_stored), ptr(page_index), n, ptr(k_out),
            ptr(v_out), stream_handle(dev),
        )
    check(st, "tp_decode_pages_gather")
    return k_out, v_out


def decode_pages(pageset: PageSet, want_k: bool = True, want_v: bool = True):
    """tp_decode_pages -> dense fp16 ``[B, H, S*64, 128]`` K and/or V."""
    B, H, S = pageset.B, pageset.H, pageset.S
    dev = next(iter(pageset.tensors.values())).device
    k_out = torch.empty((B, H, S * PAGE, HEAD_DIM), dtype=torch.float16, device=dev) if want_k else None
    v_out = torch.empty((B, H, S * PAGE, HEAD_DIM), dtype=torch.float16, device=dev) if want_v else None
    layout = getattr(pageset, "layout", _lib.make_layout(False, 4, 4, 64))
    with on_device(dev):
        st = lib().tp_decode_pages(
            ctypes.byref(layout), ctypes.byref(pageset.pages), B * H, 0, S, ptr(k_out), ptr(v_out), stream_handle(dev)
        )
    check(st, "tp_decode_pages")
    return k_out, v_out


def _q16(q: torch.Tensor) -> torch.Tensor:
    require_hip(q, "q")
    if q.dim() != 3 or q.shape[-1] != HEAD_DIM:
        raise ValueError(f"q must be [B, H_q, {HEAD_DIM}], got {tuple(q.shape)}")
    return q.to(torch.float16).contiguous()


def fused_qk(q: torch.Tensor, pageset: PageSet, scale: float, qjl=None) -> torch.Tensor:
    """tp_fused_qk -> fp16 scores ``[B, H_q, S*64]``; with ``qjl`` (a
    ``qjl.QJLPages``) tp_fused_qk_qjl, which adds the QJL correction."""
    q16 = _q16(q)
    B, Hq, _ = q16.shape
    if B != pageset.B or Hq % pageset.H:
        raise ValueError(f"q heads {Hq} / batch {B} do not match kv pages {pageset.B}x{pageset.H}")
    scores = torch.empty((B, Hq, pageset.S * PAGE), dtype=torch.float16, device=q16.device)
    with on_device(q16.device):
        if qjl is None:
            st = lib().tp_fused_qk(
                ptr(q16), B, Hq, pageset.H, ctypes.byref(pageset.layout), ctypes.byref(pageset.pages),
                pageset.S, float(scale), ptr(scores), stream_handle(q16.device),
            )
        else:
            qjl.check_against(pageset.B, pageset.H, pageset.S, Hq)
            st = lib().tp_fused_qk_qjl(
                ptr(q16), B, Hq, pageset.H, ctypes.byref(pageset.layout), ctypes.byref(pageset.pages),
                pageset.S, ctypes.byref(qjl.desc), float(scale), ptr(scores), stream_handle(q16.device),
            )
    check(st, "tp_fused_qk_qjl" if qjl is not None else "tp_fused_qk")
    return scores


class _Workspace:
    """Per-(device, stream) split-K workspace, grown on demand; its counter area
    starts zeroed and every kernel call leaves it zeroed."""

    _bufs: dict = {}

    @classmethod
    def get(cls, device: torch.device, nbytes: int) -> torch.Tensor:
        key = (device.index, stream_handle(device))
        buf = cls._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            cls._bufs[key] = buf
        return buf


def decode_attention(
    q: torch.Tensor,
    pageset: Optional[PageSet],
    tail_k: Optional[torch.Tensor],
    tail_v: Optional[torch.Tensor],
    actual_seq_len: int,
    scale: float,
    num_kv_heads: Optional[int] = None,
    pages_per_split: int = 0,
    out: Optional[torch.Tensor] = None,
    qjl=None,
) -> torch.Tensor:
    """tp_decode_attention -> fp16 ``[B, H_q, 128]``.

    ``tail_k``/``tail_v``: ``[B, H_kv, T_tail, 128]`` (T_tail < 64, any float
    dtype; converted to fp16 as metal.py:744 does).  ``qjl`` (a
    ``qjl.QJLPages`` of the pages): tp_decode_attention_qjl."""
    q16 = _q16(q)
    B, Hq, _ = q16.shape
    tail_len = 0 if tail_k is None else int(tail_k.shape[2])
    if pageset is not None:
        Hkv, n_pages = pageset.H, pageset.S
        if pageset.B != B:
            raise ValueError(f"batch of q ({B}) and pages ({pageset.B}) differ")
    else:
        if tail_len == 0:
            raise ValueError("nothing to attend: no pages and no tail")
        Hkv, n_pages = int(tail_k.shape[1]), 0
    if num_kv_heads is not None and num_kv_heads != Hkv:
        raise ValueError(f"expected {num_kv_heads} kv heads, got {Hkv}")
    if Hq % Hkv:
        raise ValueError(f"H_q={Hq} is not a multiple of H_kv={Hkv}")
    tk = tv = None
    tail_stride = 0
    if tail_len:
        require_hip(tail_k, "tail_k")
        if tail_k.shape != tail_v.shape or tuple(tail_k.shape[:2]) != (B, Hkv) or tail_k.shape[3] != HEAD_DIM:
            raise ValueError(f"tail shape {tuple(tail_k.shape)} does not match [B={B}, H_kv={Hkv}, T, {HEAD_DIM}]")
        tk, tail_stride = _tail_view(tail_k.to(torch.float16))
        tv, tail_stride_v = _tail_view(tail_v.to(torch.float16))
        if tail_stride_v != tail_stride:
            tk, tv = _fresh(tk), _fresh(tv)
            tail_stride = tail_len
    layout = pageset.layout if pageset is not None else _DEFAULT_LAYOUT
    pages = pageset.pages if pageset is not None else _NO_PAGES
    if qjl is not None:
        qjl.check_against(B, Hkv, n_pages, Hq)
    return _launch_decode(q16, Hkv, layout, pages, n_pages, tk, tv, tail_len, tail_stride, actual_seq_len, scale,
                          pages_per_split, out, qjl)


_DEFAULT_LAYOUT = _lib.make_layout(False, 4, 4, 64)
_NO_PAGES = TPPages()


def _launch_decode(q16, Hkv, layout, pages, n_pages, tk, tv, tail_len, tail_stride, seq_len, scale, pps, out,
                   qjl=None):
    B, Hq, _ = q16.shape
    dev = q16.device
    if out is None:
        out = torch.empty((B, Hq, HEAD_DIM), dtype=torch.float16, device=dev)
    L = lib()
    pps = int(pps) or int(L.tp_default_pages_per_split(B, Hq, Hkv, n_pages))
    need = int(L.tp_decode_workspace_bytes(B, Hq, Hkv, n_pages, tail_len, pps))
    ws = _Workspace.get(dev, need)
    with on_device(dev):
        if qjl is None:
            st = L.tp_decode_attention(
                ptr(q16), B, Hq, Hkv, ctypes.byref(layout), ctypes.byref(pages), n_pages,
                ptr(tk), ptr(tv), tail_len, tail_stride, int(seq_len), float(scale), pps,
                ws.data_ptr(), ws.numel(), ptr(out), stream_handle(dev),
            )
        else:
            st = L.tp_decode_attention_qjl(
                ptr(q16), B, Hq, Hkv, ctypes.byref(layout), ctypes.byref(pages), n_pages, ctypes.byref(qjl.desc),
                ptr(tk), ptr(tv), tail_len, tail_stride, int(seq_len), float(scale), pps,
                ws.data_ptr(), ws.numel(), ptr(out), stream_handle(dev),
            )
    check(st, "tp_decode_attention_qjl" if qjl is not None else "tp_decode_attention")
    return out


def decode_attention_dense_v(
    q: torch.Tensor,
    pageset: PageSet,
    v_dense: torch.Tensor,
    actual_seq_len: int,
    scale: float,
    pages_per_split: int = 0,
    out: Optional[torch.Tensor] = None,
    qjl=None,
) -> torch.Tensor:
    """tp_decode_attention_dense_v -> fp16 ``[B, H_q, 128]``: attention over
    the compressed K pages of ``pageset`` (its V fields are not read) and dense
    V ``v_dense`` ``[B, H_kv, S, 64, 128]`` or ``[B, H_kv, S * 64, 128]`` (any
    float dtype; converted to fp16), the reference's
    execute_online_attention_dense_v (metal.py:586-649).  ``qjl``: a
    ``qjl.QJLPages`` of the pages (use_qjl=True)."""
    q16 = _q16(q)
    B, Hq, _ = q16.shape
    Hkv, n_pages = pageset.H, pageset.S
    if pageset.B != B:
        raise ValueError(f"batch of q ({B}) and pages ({pageset.B}) differ")
    if Hq % Hkv:
        raise ValueError(f"H_q={Hq} is not a multiple of H_kv={Hkv}")
    require_hip(v_dense, "v_dense")
    if v_dense.ndim == 5:
        if tuple(v_dense.shape[:2]) != (B, Hkv) or v_dense.shape[3] != PAGE or v_dense.shape[4] != HEAD_DIM:
            raise ValueError(f"v_dense shape {tuple(v_dense.shape)} does not match [B={B}, H_kv={Hkv}, S, "
                             f"{PAGE}, {HEAD_DIM}]")
        v_cap = int(v_dense.shape[2])
    elif v_dense.ndim == 4:
        if tuple(v_dense.shape[:2]) != (B, Hkv) or v_dense.shape[3] != HEAD_DIM or v_dense.shape[2] % PAGE:
            raise ValueError(f"v_dense shape {tuple(v_dense.shape)} does not match [B={B}, H_kv={Hkv}, S * {PAGE}, "
                             f"{HEAD_DIM}]")
        v_cap = int(v_dense.shape[2]) // PAGE
    else:
        raise ValueError(f"v_dense must be 4-D or 5-D, got shape {tuple(v_dense.shape)}")
    if v_cap < n_pages:
        raise ValueError(f"v_dense holds {v_cap} pages, the key block {n_pages}")
    v16 = v_dense.to(torch.float16).contiguous()
    if qjl is not None:
        qjl.check_against(B, Hkv, n_pages, Hq)
    dev = q16.device
    if out is None:
        out = torch.empty((B, Hq, HEAD_DIM), dtype=torch.float16, device=dev)
    L = lib()
    pps = int(pages_per_split) or int(L.tp_default_pages_per_split(B, Hq, Hkv, n_pages))
    need = int(L.tp_decode_workspace_bytes(B, Hq, Hkv, n_pages, 0, pps))
    ws = _Workspace.get(dev, need)
    with on_device(dev):
        st = L.tp_decode_attention_dense_v(
            ptr(q16), B, Hq, Hkv, ctypes.byref(pageset.layout), ctypes.byref(pageset.pages), n_pages,
            ctypes.byref(qjl.desc) if qjl is not None else None, ptr(v16), v_cap, int(actual_seq_len),
            float(scale), pps, ws.data_ptr(), ws.numel(), ptr(out), stream_handle(dev),
        )
    check(st, "tp_decode_attention_dense_v")
    return out


def decode_attention_store(q: torch.Tensor, layout, pages: TPPages, n_pages: int, num_kv_heads: int,
                           tail_k: Optional[torch.Tensor], tail_v: Optional[torch.Tensor], seq_len: int,
                           scale: float) -> torch.Tensor:
    """A cache's decode step: ``tp_decode_attention`` over the first ``n_pages``
    slots of a page store used in place (``pages`` carries its capacity) and a
    dense tail given as ``[B, H_kv, T, 128]`` views of a token-major buffer
    (``T`` < 64).  ``q`` is ``[B, H_q, 128]``."""
    q16 = _q16(q)
    tail_len = 0 if tail_k is None else int(tail_k.shape[2])
    tk = tv = None
    tail_stride = 0
    if tail_len:
        tk, tail_stride = _tail_view(tail_k.to(torch.float16))
        tv, stride_v = _tail_view(tail_v.to(torch.float16))
        if stride_v != tail_stride:
            tk, tv, tail_stride = _fresh(tk), _fresh(tv), tail_len
    if pages is None:
        pages, n_pages = _NO_PAGES, 0
    return _launch_decode(q16, num_kv_heads, layout, pages, n_pages, tk, tv, tail_len, tail_stride, seq_len, scale,
                          0, None)


def _tail_view(t: torch.Tensor):
    """(tensor, token stride) such that rows are dense 128-element fp16 rows and
    (batch, head) planes are ``stride`` rows apart."""
    B, H, T, D = t.shape
    ok = t.stride(3) == 1 and (T == 1 or t.stride(2) == D)
    if ok:
        if H > 1:
            plane = t.stride(1)
            ok = plane % D == 0 and (B == 1 or t.stride(0) == H * plane)
        elif B > 1:
            plane = t.stride(0)
            ok = plane % D == 0
        else:
            plane = T * D
        if ok:
            stride = plane // D
            if stride >= T:
                return t, stride
    t = _fresh(t)
    return t, T
