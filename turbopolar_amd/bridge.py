"""HIP kernel bridge: the drop-in for ``MetalKernelBridge``.

Same method names, arguments and return values as
rfsn_v11/kernels/turbo_polar/metal.py:57-792 for the supported path:

* ``execute_fused_qk(q, block, config) -> scores``            (metal.py:494-530)
* ``execute_online_attention_quant_v(...) -> (out, trace)``    (metal.py:651-715)
* ``execute_online_attention_quant_v_dense_tail(...)``         (metal.py:717-792)
* ``execute_online_attention_dense_v(...) -> (out, trace)``    (metal.py:586-649)

* ``execute_fused_qk_qjl(q, block, qjl_payload, q_proj_signs, config)`` (metal.py:532-571)

Differences: there is no silent CPU fallback (unsupported inputs raise), and
the trace reports ``hip_used`` where the reference reports ``metal_used``.
``use_qjl=True`` adds the QJL correction to the page tokens' scores
(tp_decode_attention_qjl; the config still rejects QJL for the runtime,
turbo_polar_config.py:46-47, as in the reference).  ``attention_scale``
reaches the kernels as fp16, as the reference passes it (metal.py:518,692,774).
"""

from __future__ import annotations

from typing import Any, Dict, Optional, Tuple

import torch

from . import _lib
from .kernels import PageSet, decode_attention, decode_attention_dense_v, fp16_scale, fused_qk
from .payload import PolarKeyBlock, QuantizedVBlock
from .qjl import QJLPages


def _pages_of(block: PolarKeyBlock, quant_v: Optional[QuantizedVBlock], head_dim: int) -> PageSet:
    """PageSet of a key block and its values, kept on the block object: the
    runtime hands the same block objects to every decode step until a page is
    added, so the descriptors are built once per page, not once per step."""
    hit = block.__dict__.get("_tp_pages")
    if hit is not None and hit[0] is quant_v and hit[1] == head_dim:
        return hit[2]
    pages = PageSet(block, quant_v, head_dim)
    block.__dict__["_tp_pages"] = (quant_v, head_dim, pages)
    return pages


class HipKernelBridge:
    """Process-wide singleton, like the reference bridge (metal.py:72-86)."""

    _instance: "HipKernelBridge | None" = None

    def __new__(cls, *args, **kwargs):
        if cls._instance is None:
            inst = super().__new__(cls)
            _lib.lib()  # fail loudly if the HIP library is missing
            inst.threadgroup_supported = True
            cls._instance = inst
        return cls._instance

    @staticmethod
    def _supports_block(block: PolarKeyBlock) -> None:
        """Raises for formats the kernels cannot decode (metal.py:454-492)."""
        if block.radii.dtype == torch.int8:
            if block.radii_scales is None:
                raise ValueError("int8 radii require radii_scales")
        elif block.radii.dtype != torch.float16:
            raise ValueError(f"unsupported radii dtype: {block.radii.dtype}")

    @staticmethod
    def _qjl(use_qjl: bool, qjl_payload, q_proj_signs) -> Optional[QJLPages]:
        """The QJL descriptor when use_qjl (metal.py:573-580's check), else None."""
        if not use_qjl:
            return None
        if qjl_payload is None or q_proj_signs is None:
            raise ValueError("qjl_payload and q_proj_signs are required when use_qjl=True")
        return QJLPages(qjl_payload, q_proj_signs)

    def execute_fused_qk(self, q: torch.Tensor, block: PolarKeyBlock, config) -> torch.Tensor:
        self._supports_block(block)
        return fused_qk(q, PageSet(block, None, config.head_dim), fp16_scale(config.attention_scale))

    def execute_fused_qk_qjl(self, q: torch.Tensor, block: PolarKeyBlock, qjl_payload, q_proj_signs: torch.Tensor,
                             config) -> torch.Tensor:
        """Scores plus the QJL correction times attention_scale (metal.py:532-571)."""
        self._supports_block(block)
        qjl = self._qjl(True, qjl_payload, q_proj_signs)
        return fused_qk(q, PageSet(block, None, config.head_dim), fp16_scale(config.attention_scale), qjl=qjl)

    def execute_online_attention_quant_v(
        self,
        q: torch.Tensor,
        block: PolarKeyBlock,
        quant_v: QuantizedVBlock,
        qjl_payload: Optional[Any],
        q_proj_signs: Optional[torch.Tensor],
        config,
        actual_seq_len: int,
        use_qjl: bool = False,
    ) -> Tuple[torch.Tensor, Dict[str, Any]]:
        qjl = self._qjl(use_qjl, qjl_payload, q_proj_signs)
        self._supports_block(block)
        pages = _pages_of(block, quant_v, config.head_dim)
        out = decode_attention(q, pages, None, None, actual_seq_len, fp16_scale(config.attention_scale), qjl=qjl)
        trace = {
            "kernel_name": "tqpolar_online_attention_quant_v",
            "hip_kernel": "tp_decode_attention_qjl" if use_qjl else "tp_decode_attention",
            "hip_used": True,
            "fallback_used": False,
            "qjl_used": bool(use_qjl),
            "quant_v_used": True,
            "actual_seq_len": actual_seq_len,
            "num_queries_per_kv": q.shape[1] // pages.H,
        }
        return out, trace

    def execute_online_attention_dense_v(
        self,
        q: torch.Tensor,
        block: PolarKeyBlock,
        v_dense: torch.Tensor,
        qjl_payload: Optional[Any],
        q_proj_signs: Optional[torch.Tensor],
        config,
        actual_seq_len: int,
        use_qjl: bool = False,
    ) -> Tuple[torch.Tensor, Dict[str, Any]]:
        """Compressed K with dense V (metal.py:586-649, the dense_v_debug
        storage): ``v_dense`` ``[B, H_kv, S, 64, 128]`` (or ``[B, H_kv, S * 64,
        128]``), tp_decode_attention_dense_v."""
        qjl = self._qjl(use_qjl, qjl_payload, q_proj_signs)
        self._supports_block(block)
        pages = _pages_of(block, None, config.head_dim)
        out = decode_attention_dense_v(q, pages, v_dense, actual_seq_len, fp16_scale(config.attention_scale), qjl=qjl)
        trace = {
            "kernel_name": "tqpolar_online_attention_dense_v",
            "hip_kernel": "tp_decode_attention_dense_v",
            "hip_used": True,
            "fallback_used": False,
            "qjl_used": bool(use_qjl),
            "quant_v_used": False,
            "actual_seq_len": actual_seq_len,
            "num_queries_per_kv": q.shape[1] // pages.H,
        }
        return out, trace

    def execute_online_attention_quant_v_dense_tail(
        self,
        q: torch.Tensor,
        block: Optional[PolarKeyBlock],
        quant_v: Optional[QuantizedVBlock],
        tail_k: torch.Tensor,
        tail_v: torch.Tensor,
        qjl_payload: Optional[Any],
        q_proj_signs: Optional[torch.Tensor],
        config,
        actual_seq_len: int,
        use_qjl: bool = False,
    ) -> Tuple[torch.Tensor, Dict[str, Any]]:
        qjl = self._qjl(use_qjl, qjl_payload, q_proj_signs)
        pages = None
        if block is not None:
            self._supports_block(block)
            pages = _pages_of(block, quant_v, config.head_dim)
        tail_len = int(tail_k.shape[2]) if tail_k is not None else 0
        out = decode_attention(
            q, pages, tail_k if tail_len else None, tail_v if tail_len else None,
            actual_seq_len, fp16_scale(config.attention_scale), qjl=qjl if pages is not None else None,
        )
        hkv = pages.H if pages is not None else int(tail_k.shape[1])
        trace = {
            "kernel_name": "tqpolar_online_attention_quant_v_dense_tail",
            "hip_kernel": "tp_decode_attention_qjl" if (use_qjl and pages is not None) else "tp_decode_attention",
            "hip_used": True,
            "fallback_used": False,
            "qjl_used": bool(use_qjl),
            "quant_v_used": True,
            "tail_length": tail_len,
            "actual_seq_len": actual_seq_len,
            "num_queries_per_kv": q.shape[1] // hkv,
        }
        return out, trace
