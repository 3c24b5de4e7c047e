"""QJL residual sketches: ``QJLPayload``, ``QJLResidualEncoder`` and
``qjl_dot_estimate``, on the HIP kernels of tp_qjl.hip.

Interface of the reference's rfsn_v11/quant/qjl/encoder.py:10-44 and
score_estimate.py:6-54 (class, method and argument names, payload fields and
layout: packed signs ``[B, H, S, L, P/8]`` uint8, bit i of byte j the sign of
projection 8j + i; residual norms ``[B, H, S, L]`` fp16).  The projection W is
built exactly as the reference builds it (NumPy ``default_rng(seed)``
standard normals, unit columns) and kept on the device in fp32.

``TurboPolarConfig`` rejects ``use_qjl=True`` (turbo_polar_config.py:46-47),
as the reference's does, so the runtime never makes sketches; these serve the
bridge-level QJL calls (``HipKernelBridge.execute_fused_qk_qjl`` and
``use_qjl=True`` attention), which take a payload and query sketches directly,
as the reference's own QJL tests do.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib


@dataclass
class QJLPayload:
    packed_signs: torch.Tensor
    norms: torch.Tensor
    proj_dim: int
    seed: int
    shape: tuple


def qjl_projection(seed: int, head_dim: int, proj_dim: int) -> np.ndarray:
    """W of QJLResidualEncoder.__init__ (encoder.py:20-28): ``[head_dim,
    proj_dim]`` float32 standard normals from ``np.random.default_rng(seed)``,
    each column divided by (its norm + 1e-12)."""
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((head_dim, proj_dim), dtype=np.float32)
    return w / (np.linalg.norm(w, axis=0, keepdims=True) + 1e-12)


class QJLResidualEncoder:
    def __init__(self, config):
        self.config = config
        self.proj_dim = config.qjl_proj_dim
        self.seed = getattr(config, "seed", 42)
        self.head_dim = config.head_dim
        self.W_host = qjl_projection(self.seed, self.head_dim, self.proj_dim)
        self._w = {}  # device -> fp32 W

    def W(self, device) -> torch.Tensor:
        """W on ``device`` (fp32 ``[head_dim, proj_dim]``)."""
        key = torch.device(device)
        w = self._w.get(key)
        if w is None:
            w = torch.from_numpy(self.W_host).to(key)
            self._w[key] = w
        return w

    def _sketch(self, x: torch.Tensor, want_norms: bool):
        _lib.require_hip(x, "input")
        if x.dtype not in (torch.float16, torch.float32):
            raise ValueError(f"QJL sketches take float16 or float32, got {x.dtype}")
        if x.shape[-1] != self.head_dim:
            raise ValueError(f"last dim {x.shape[-1]} != head_dim {self.head_dim}")
        xc = x.contiguous()
        rows = xc.numel() // self.head_dim
        packed = torch.empty(xc.shape[:-1] + (self.proj_dim // 8,), dtype=torch.uint8, device=x.device)
        norms = torch.empty(xc.shape[:-1], dtype=torch.float16, device=x.device) if want_norms else None
        w = self.W(x.device)
        with _lib.on_device(x.device):
            st = _lib.lib().tp_qjl_sketch(xc.data_ptr(), 1 if xc.dtype == torch.float32 else 0, rows, self.head_dim,
                                          w.data_ptr(), self.proj_dim, packed.data_ptr(),
                                          norms.data_ptr() if want_norms else None, _lib.stream_handle(x.device))
        _lib.check(st, "tp_qjl_sketch")
        return packed, norms

    def compute_residual_sketch(self, residual_E: torch.Tensor) -> QJLPayload:
        """Sketch of ``[B, H, S, L, D]`` residuals (encoder.py:30-44)."""
        B, H, S, L, D = residual_E.shape
        assert D == self.head_dim
        packed, norms = self._sketch(residual_E, True)
        return QJLPayload(packed_signs=packed, norms=norms, proj_dim=self.proj_dim, seed=self.seed,
                          shape=(B, H, S, L, D))

    def query_signs(self, q: torch.Tensor) -> torch.Tensor:
        """Packed signs of ``q @ W`` for ``[B, H_q, D]`` queries: the
        ``q_proj_signs`` the QJL score paths take."""
        return self._sketch(q, False)[0]


class QJLPages:
    """Device descriptor (``tp_qjl``) of a payload's sketches and the queries'
    sketches, for the QJL kernels; S pages of 64 tokens per (b, kv head)."""

    # Sketch widths the QJL kernels take: P = 64 (the default) on their
    # 64-bit path, any other multiple of 8 up to 256 on the byte-aligned one.
    MAX_PROJ_DIM = 256

    def __init__(self, payload: QJLPayload, q_proj_signs: torch.Tensor):
        P = int(payload.proj_dim)
        if P < 8 or P > self.MAX_PROJ_DIM or P % 8:
            raise NotImplementedError(f"the HIP QJL kernels take qjl_proj_dim a multiple of 8 up to "
                                      f"{self.MAX_PROJ_DIM}, got {P}")
        signs, norms = payload.packed_signs, payload.norms
        for name, t in (("packed_signs", signs), ("norms", norms), ("q_proj_signs", q_proj_signs)):
            _lib.require_hip(t, name)
        if (signs.dim() != 5 or signs.shape[3] != 64 or signs.shape[4] != P // 8
                or tuple(norms.shape) != tuple(signs.shape[:4])):
            raise ValueError(f"QJL payload must be [B, H, S, 64, {P // 8}] signs and [B, H, S, 64] norms, got "
                             f"{tuple(signs.shape)} and {tuple(norms.shape)}")
        if signs.dtype != torch.uint8 or norms.dtype != torch.float16 or q_proj_signs.dtype != torch.uint8:
            raise ValueError("QJL payload dtypes must be uint8 signs, fp16 norms and uint8 query signs")
        self.keep = (signs.contiguous(), norms.contiguous(), q_proj_signs.contiguous())
        self.B, self.H, self.S = int(signs.shape[0]), int(signs.shape[1]), int(signs.shape[2])
        self.q_shape = tuple(q_proj_signs.shape)
        self.proj_dim = P
        self.desc = _lib.TPQjl(self.keep[0].data_ptr(), self.keep[1].data_ptr(), self.keep[2].data_ptr(), P, self.S)

    def check_against(self, B: int, H: int, S: int, Hq: int) -> None:
        if (self.B, self.H) != (B, H) or self.S < S or self.q_shape != (B, Hq, self.proj_dim // 8):
            raise ValueError(f"QJL payload [{self.B}, {self.H}, {self.S}] / query signs {self.q_shape} do not match "
                             f"pages [{B}, {H}, {S}] and {Hq} query heads")


def qjl_dot_estimate(q: torch.Tensor, qjl_payload: QJLPayload, q_proj_signs: torch.Tensor) -> torch.Tensor:
    """The unscaled QJL estimate of q . E (score_estimate.py:6-54): fp32
    ``[B, H_q, S*L]``, ``|E| |q| sin(pi/2 * (P - 2 hamming) / P)``, query head
    h against the sketches of kv head h // (H_q / H_kv)."""
    B, H_kv, S, L, D = qjl_payload.shape
    Hq = int(q_proj_signs.shape[1])
    P = qjl_payload.proj_dim
    q16 = q.reshape(B, Hq, D).to(torch.float16).contiguous()
    signs = qjl_payload.packed_signs.contiguous()
    norms = qjl_payload.norms.contiguous()
    qs = q_proj_signs.contiguous()
    out = torch.empty((B, Hq, S * L), dtype=torch.float32, device=q.device)
    with _lib.on_device(q.device):
        st = _lib.lib().tp_qjl_dot_estimate(q16.data_ptr(), B, Hq, H_kv, D, signs.data_ptr(), norms.data_ptr(),
                                            S * L, qs.data_ptr(), P, out.data_ptr(), _lib.stream_handle(q.device))
    _lib.check(st, "tp_qjl_dot_estimate")
    return out
