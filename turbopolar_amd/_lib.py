"""ctypes binding of the C ABI declared in ``include/turbopolar.h``.

The library is loaded from the package directory (built in-tree by
``python -m turbopolar_amd.build``).  There is no CPU fallback: if the library
is missing or the tensors are not on a HIP device, calls raise.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import torch  # noqa: F401  (loads torch's HIP runtime before the library)

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libturbopolar_hip.so"
HEADER_PATH = PKG_DIR.parent / "include" / "turbopolar.h"

TP_OK = 0
TP_ERR_INVALID = 1
TP_ERR_UNSUPPORTED = 2
TP_ERR_HIP = 3
TP_ERR_WORKSPACE = 4
TP_ERR_NONFINITE = 5
TP_NOALLOC_SCRATCH_BYTES = 8 << 20  # include/turbopolar.h

c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_vp = ctypes.c_void_p
c_size = ctypes.c_size_t
c_float = ctypes.c_float


class TPPageLayout(ctypes.Structure):
    _fields_ = [
        ("int8_radii", c_i32),
        ("l1_bits", c_i32),
        ("deep_bits", c_i32),
        ("split_dim", c_i32),
    ]


class TPPages(ctypes.Structure):
    _fields_ = [
        ("radii", c_vp),
        ("radii_scales", c_vp),
        ("angle_l1", c_vp),
        ("angle_deep", c_vp),
        ("v_codes", c_vp),
        ("v_scales", c_vp),
        ("capacity", c_i64),
    ]


class TPQjl(ctypes.Structure):
    _fields_ = [
        ("signs", c_vp),
        ("norms", c_vp),
        ("q_signs", c_vp),
        ("proj_dim", c_i32),
        ("capacity", c_i64),
    ]


class TPBoundsCase(ctypes.Structure):
    """tp_bounds_case: one launch shape for tp_selftest_decode_bounds."""

    _fields_ = [
        ("batch", c_i64),
        ("hq", c_i32),
        ("hkv", c_i32),
        ("layout", TPPageLayout),
        ("n_pages", c_i32),
        ("capacity", c_i64),
        ("tail_len", c_i32),
        ("tail_stride", c_i64),
        ("seq_len", c_i64),
        ("pages_per_split", c_i32),
        ("qjl", c_i32),
        ("qjl_capacity", c_i64),
        ("dense_v", c_i32),
        ("v_capacity", c_i64),
        ("kernel", c_i32),
        ("mutate", c_i32),
        ("qjl_bits", c_i32),
    ]


class TurboPolarHipError(RuntimeError):
    """A HIP runtime or launch failure inside the TurboPolar library."""


_P_LAYOUT = ctypes.POINTER(TPPageLayout)
_P_PAGES = ctypes.POINTER(TPPages)
_P_QJL = ctypes.POINTER(TPQjl)

_SIGNATURES = {
    "tp_last_error": (ctypes.c_char_p, []),
    "tp_version": (c_i32, []),
    "tp_layout_row_bytes": (c_i32, [_P_LAYOUT, ctypes.POINTER(c_i32), ctypes.POINTER(c_i32)]),
    "tp_encode_pages": (
        c_i32,
        [c_vp, c_vp, c_i32, c_i64, c_i64, c_i64, c_i64, _P_LAYOUT, _P_PAGES, c_i64, c_vp],
    ),
    "tp_fused_qk": (c_i32, [c_vp, c_i64, c_i32, c_i32, _P_LAYOUT, _P_PAGES, c_i32, c_float, c_vp, c_vp]),
    "tp_decode_attention": (
        c_i32,
        [
            c_vp, c_i64, c_i32, c_i32, _P_LAYOUT, _P_PAGES, c_i32,
            c_vp, c_vp, c_i32, c_i64, c_i64, c_float, c_i32, c_vp, c_size, c_vp, c_vp,
        ],
    ),
    "tp_decode_attention_noalloc": (
        c_i32,
        [
            c_vp, c_i64, c_i32, c_i32, _P_LAYOUT, _P_PAGES, c_i32,
            c_vp, c_vp, c_i32, c_i64, c_i64, c_float, c_i32, c_vp, c_vp,
        ],
    ),
    "tp_decode_workspace_bytes": (c_size, [c_i64, c_i32, c_i32, c_i32, c_i32, c_i32]),
    "tp_decode_counter_bytes": (c_size, [c_i64, c_i32, c_i32]),
    "tp_default_pages_per_split": (c_i32, [c_i64, c_i32, c_i32, c_i32]),
    "tp_decode_pages": (c_i32, [_P_LAYOUT, _P_PAGES, c_i64, c_i64, c_i32, c_vp, c_vp, c_vp]),
    "tp_decode_pages_into": (c_i32, [_P_LAYOUT, _P_PAGES, c_i64, c_i64, c_i32, c_vp, c_vp, c_i64, c_i64, c_vp]),
    "tp_decode_pages_gather": (c_i32, [_P_LAYOUT, _P_PAGES, c_i64, c_i32, c_vp, c_i32, c_vp, c_vp, c_vp]),
    "tp_append_stage": (
        c_i32,
        [c_vp, c_vp, c_i32, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, c_i64, c_i64, c_i32, c_vp, ctypes.c_uint32, c_vp],
    ),
    "tp_fused_qk_qjl": (c_i32, [c_vp, c_i64, c_i32, c_i32, _P_LAYOUT, _P_PAGES, c_i32, _P_QJL, c_float, c_vp, c_vp]),
    "tp_decode_attention_qjl": (
        c_i32,
        [
            c_vp, c_i64, c_i32, c_i32, _P_LAYOUT, _P_PAGES, c_i32, _P_QJL,
            c_vp, c_vp, c_i32, c_i64, c_i64, c_float, c_i32, c_vp, c_size, c_vp, c_vp,
        ],
    ),
    "tp_decode_attention_dense_v": (
        c_i32,
        [
            c_vp, c_i64, c_i32, c_i32, _P_LAYOUT, _P_PAGES, c_i32, _P_QJL,
            c_vp, c_i64, c_i64, c_float, c_i32, c_vp, c_size, c_vp, c_vp,
        ],
    ),
    "tp_qjl_sketch": (c_i32, [c_vp, c_i32, c_i64, c_i32, c_vp, c_i32, c_vp, c_vp, c_vp]),
    "tp_qjl_dot_estimate": (c_i32, [c_vp, c_i64, c_i32, c_i32, c_i32, c_vp, c_vp, c_i64, c_vp, c_i32, c_vp, c_vp]),
    "tp_quantize_v_groups": (c_i32, [c_vp, c_i32, c_i64, c_i32, c_i32, c_vp, c_vp, c_vp]),
    "tp_log_radii_rows": (c_i32, [c_vp, c_i64, c_i64, c_vp, c_vp, c_vp]),
    "tp_selftest_f16_tables": (c_i32, [c_vp, c_vp, c_vp, c_vp]),
    "tp_selftest_fastdiv": (ctypes.c_ulonglong, [ctypes.c_uint32, c_vp]),
    "tp_selftest_decode_bounds": (ctypes.c_ulonglong, [ctypes.POINTER(TPBoundsCase), ctypes.c_char_p, c_i32]),
    "tp_selftest_atan2_exhaustive": (c_i32, [c_vp, c_i32, c_i32, c_vp]),
    "tp_selftest_div_f16_exhaustive": (c_i32, [c_vp, c_i32, c_i32, c_vp]),
    "tp_selftest_vcode_exhaustive": (c_i32, [c_vp, c_i32, c_i32, c_vp]),
    "tp_selftest_lcode_exhaustive": (c_i32, [c_vp, c_i32, c_i32, c_vp]),
}

_lib = None


def header_symbols() -> list[str]:
    """Function names declared in include/turbopolar.h."""
    text = HEADER_PATH.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(tp_\w+)\s*\(", text, re.M)))


def open_library(path) -> ctypes.CDLL:
    """Loads a build of the library at ``path`` with its symbols kept local
    and declares the C signatures (``lib()`` for the product library; the
    measurement build is opened the same way beside it)."""
    path = Path(path)
    if not path.exists():
        raise RuntimeError(
            f"{path.name} is not built; run `python -m turbopolar_amd.build` "
            "(the TurboPolar path has no CPU fallback)"
        )
    handle = ctypes.CDLL(str(path), mode=ctypes.RTLD_LOCAL)
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return handle


def lib() -> ctypes.CDLL:
    """Loads libturbopolar_hip.so (once) and declares the C signatures."""
    global _lib
    if _lib is None:
        _lib = open_library(LIB_PATH)
    return _lib


def check(status: int, what: str) -> None:
    """Maps a C status code to the reference's exception types."""
    if status == TP_OK:
        return
    msg = lib().tp_last_error().decode(errors="replace")
    if status in (TP_ERR_INVALID, TP_ERR_UNSUPPORTED, TP_ERR_NONFINITE):
        raise ValueError(f"{what}: {msg}")
    raise TurboPolarHipError(f"{what}: {msg}")


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None or an empty tensor)."""
    if t is None or t.numel() == 0:
        return None
    return t.data_ptr()


def raw_stream(device_index: int) -> int:
    """The current stream of a device as a raw handle, without building a
    torch Stream object (the hot paths call this once per launch)."""
    return torch._C._cuda_getCurrentRawStream(device_index)


def stream_handle(device: torch.device) -> int:
    """raw_stream of ``device`` (its index, or the current device's)."""
    return raw_stream(device.index if device.index is not None else torch.cuda.current_device())


class on_device:
    """Makes ``device`` current for a launch, switching only when another
    device is current (a cheaper torch.cuda.device for the per-token paths)."""

    __slots__ = ("idx", "prev")

    def __init__(self, device: torch.device):
        self.idx = device.index if device.index is not None else torch.cuda.current_device()
        self.prev = self.idx

    def __enter__(self):
        self.prev = torch.cuda.current_device()
        if self.prev != self.idx:
            torch.cuda.set_device(self.idx)
        return self

    def __exit__(self, *exc):
        if self.prev != self.idx:
            torch.cuda.set_device(self.prev)
        return False


def require_hip(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(
            f"{name} must be on a HIP device; the TurboPolar path has no CPU fallback "
            f"(got device {t.device})"
        )


def make_layout(int8_radii: bool, l1_bits: int, deep_bits: int, split_dim: int) -> TPPageLayout:
    return TPPageLayout(int(bool(int8_radii)), int(l1_bits), int(deep_bits), int(split_dim))


def row_bytes(layout: TPPageLayout) -> tuple[int, int]:
    l1 = c_i32(0)
    deep = c_i32(0)
    check(lib().tp_layout_row_bytes(ctypes.byref(layout), ctypes.byref(l1), ctypes.byref(deep)), "layout")
    return l1.value, deep.value
