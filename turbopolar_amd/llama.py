"""PyTorch Llama integration of the fused decode path.

Mirrors the reference's mlx_lm hook (benchmarks/turbopolar_fast_attention.py:
232-298: ``_is_standard_causal_mask``, ``_turbo_attention_call``,
``patch_llama_attention``, ``unpatch_llama_attention``) for Hugging Face
``transformers`` Llama models:

* ``TurboPolarCache`` is a ``transformers`` ``Cache`` whose layers are
  ``TurboPolarFastCache`` objects (one per decoder layer), so the model sees the
  cached length (positions, masks) as with its own caches.  Its ``update`` is
  the prefill path: append, then decompress on read
  (``TurboPolarFastCache.update_and_fetch``), followed by the model's own
  attention over the decompressed history, as mlx_lm does with the
  reference's cache.
* ``patch_llama_attention`` swaps ``LlamaAttention.forward`` for one that sends
  single-token decode steps with a standard causal mask through
  ``TurboPolarFastCache.decode_attention`` (the fused HIP kernel over the
  compressed pages) and everything else through the original forward.

The model's weights are untouched; any Llama checkpoint loaded from a local
path works, and tests use randomly initialised models.
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch

from .config import TurboPolarConfig
from .fast_attention import TurboPolarFastCache, make_turbo_caches

try:  # transformers is an optional dependency of this module only
    from transformers.cache_utils import Cache, CacheLayerMixin
    from transformers.models.llama import modeling_llama as _llama
except ImportError as exc:  # pragma: no cover - exercised only without transformers
    raise ImportError("turbopolar_amd.llama needs the transformers package") from exc

__all__ = [
    "TurboPolarCache",
    "TurboPolarLayer",
    "make_turbo_cache",
    "load_local_llama",
    "patch_llama_attention",
    "unpatch_llama_attention",
    "is_patched",
]


class TurboPolarLayer(CacheLayerMixin):
    """One decoder layer's cache: a ``TurboPolarFastCache``."""

    is_compileable = False
    is_sliding = False

    def __init__(self, fast: TurboPolarFastCache):
        super().__init__()
        self.fast = fast

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        self.is_initialized = True

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        """Prefill path: append and return the decompressed history (K, V)."""
        self.is_initialized = True
        return self.fast.update_and_fetch(key_states, value_states)

    def get_mask_sizes(self, query_length: int) -> tuple:
        # Called before the new tokens are appended: the keys the queries see are
        # the cached ones plus themselves, starting at position 0.
        return self.fast.offset + query_length, 0

    def get_seq_length(self) -> int:
        return self.fast.offset

    def get_max_length(self) -> int:
        return -1

    def reset(self) -> None:
        self.fast = TurboPolarFastCache(self.fast.config)
        self.is_initialized = False


class TurboPolarCache(Cache):
    """``transformers`` cache over one ``TurboPolarFastCache`` per decoder layer."""

    def __init__(self, fast_caches: Sequence[TurboPolarFastCache]):
        super().__init__(layers=[TurboPolarLayer(c) for c in fast_caches])

    def fast(self, layer_idx: int) -> TurboPolarFastCache:
        return self.layers[layer_idx].fast

    @property
    def nbytes(self) -> int:
        return sum(layer.fast.nbytes for layer in self.layers)

    def resolve_deferred_checks(self) -> None:
        """The non-finite verdicts of every layer's deferred appends, after one
        stream synchronisation.  If any layer's input was non-finite, every
        layer's pending appends are undone (the cache keeps one length across
        layers) and the reference's ValueError is raised."""
        runtimes = [layer.fast.runtime for layer in self.layers if layer.fast.runtime.deferred_verdict_pending()]
        if not runtimes:
            return
        torch.cuda.current_stream(runtimes[0]._tail_k.device).synchronize()
        if any(rt._bad_pending() is not None for rt in runtimes):
            for rt in runtimes:
                rt.rollback_deferred()
            raise ValueError("append() inputs must contain finite values")
        for rt in runtimes:
            rt.resolve_deferred_check(synchronize=False)


def make_turbo_cache(model, config: Optional[TurboPolarConfig] = None) -> TurboPolarCache:
    """A ``TurboPolarCache`` sized for ``model``: the reference's fast layout
    (``make_turbo_caches``, turbopolar_fast_attention.py:207-229) unless a
    ``TurboPolarConfig`` is given."""
    cfg = model.config
    n_layers = cfg.num_hidden_layers
    n_heads = cfg.num_attention_heads
    n_kv = getattr(cfg, "num_key_value_heads", None) or n_heads
    head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // n_heads
    if config is None:
        return TurboPolarCache(make_turbo_caches(n_layers, n_heads, n_kv, head_dim))
    return TurboPolarCache([TurboPolarFastCache(config) for _ in range(n_layers)])


_mask_verdict = None  # (mask, its version, seq_len, cache_len, verdict) of the last check


def _is_standard_causal_mask(mask: Optional[torch.Tensor], seq_len: int, cache_len: int) -> bool:
    """True for no mask or the full-history causal mask ``[1, 1, seq_len, cache_len]``
    (turbopolar_fast_attention.py:235-244), boolean (True = attend) or additive
    (0 = attend).  Query i (at position cache_len - seq_len + i) sees keys
    0 .. cache_len - seq_len + i.

    A forward pass hands the same mask tensor to every layer; the verdict is
    kept for that tensor (held, so its memory cannot be reused, and keyed on
    its version counter, so an in-place change is seen), which makes the
    comparison, a device-to-host read, once per forward instead of once per
    layer."""
    global _mask_verdict
    if mask is None:
        return True
    if tuple(mask.shape) != (1, 1, seq_len, cache_len):
        return False
    hit = _mask_verdict
    if hit is not None and hit[0] is mask and hit[1] == mask._version and hit[2] == seq_len and hit[3] == cache_len:
        return hit[4]
    allowed = mask[0, 0] if mask.dtype == torch.bool else mask[0, 0] == 0
    expected = torch.ones((seq_len, cache_len), dtype=torch.bool, device=mask.device).tril(cache_len - seq_len)
    ok = bool(torch.equal(allowed, expected))
    _mask_verdict = (mask, mask._version, seq_len, cache_len, ok)
    return ok


_orig_llama_attention_forward = None


def _turbo_llama_attention_forward(
    self,
    hidden_states: torch.Tensor,
    position_embeddings=None,
    attention_mask: Optional[torch.Tensor] = None,
    past_key_values=None,
    **kwargs,
):
    """``_turbo_attention_call`` (turbopolar_fast_attention.py:247-280) for
    ``transformers``' ``LlamaAttention``: a single-token step on a
    ``TurboPolarCache`` runs the fused decode kernel; anything else runs the
    original forward (prefill appends and decompresses through the cache)."""
    if isinstance(past_key_values, TurboPolarCache) and hidden_states.shape[1] == 1:
        fast = past_key_values.fast(self.layer_idx)
        B, L, _ = hidden_states.shape
        q = self.q_proj(hidden_states).view(B, L, -1, self.head_dim).transpose(1, 2)
        k = self.k_proj(hidden_states).view(B, L, -1, self.head_dim).transpose(1, 2)
        v = self.v_proj(hidden_states).view(B, L, -1, self.head_dim).transpose(1, 2)
        if q.shape[1] % k.shape[1] != 0:
            raise ValueError("TurboPolar fused decode requires GQA ratio to divide evenly.")
        if not _is_standard_causal_mask(attention_mask, L, fast.offset + L):
            raise NotImplementedError("TurboPolar fused decode only supports standard causal full-history masks.")
        cos, sin = position_embeddings
        q, k = _llama.apply_rotary_pos_emb(q, k, cos, sin)
        # The append's non-finite verdict is read once per forward, for every
        # layer together, by the model-forward wrapper (no stream drain per layer).
        out = fast.decode_attention(q, k, v, self.scaling, defer_check=_model_wrapped())  # [B, H_q, D] fp16
        out = out.to(hidden_states.dtype).reshape(B, L, -1)
        return self.o_proj(out), None
    return _orig_llama_attention_forward(
        self, hidden_states, position_embeddings, attention_mask, past_key_values, **kwargs
    )


_orig_llama_model_forward = None


def _model_wrapped() -> bool:
    return _llama.LlamaModel.forward is _turbo_llama_model_forward


def _turbo_llama_model_forward(self, *args, **kwargs):
    """LlamaModel.forward, then the deferred non-finite verdicts of the decode
    steps it ran on a ``TurboPolarCache``: one synchronisation per forward
    instead of one per layer.  A non-finite K/V in any layer undoes the
    token's append in every layer and raises the reference's ValueError
    (turbo_polar_cache.py:69) from the forward."""
    out = _orig_llama_model_forward(self, *args, **kwargs)
    pkv = kwargs.get("past_key_values", args[3] if len(args) > 3 else None)
    if isinstance(pkv, TurboPolarCache):
        pkv.resolve_deferred_checks()
    return out


def patch_llama_attention(model=None) -> None:
    """Route Llama decode steps on a ``TurboPolarCache`` through the fused kernel
    (turbopolar_fast_attention.py:283-290).  Patches the class, like the
    reference; ``model`` is accepted for the same signature.  LlamaModel.forward
    is wrapped too, to read the steps' non-finite verdicts once per forward."""
    global _orig_llama_attention_forward, _orig_llama_model_forward
    if _orig_llama_attention_forward is None:
        _orig_llama_attention_forward = _llama.LlamaAttention.forward
    _llama.LlamaAttention.forward = _turbo_llama_attention_forward
    if _orig_llama_model_forward is None:
        _orig_llama_model_forward = _llama.LlamaModel.forward
    _llama.LlamaModel.forward = _turbo_llama_model_forward


def unpatch_llama_attention(model=None) -> None:
    """Restore the original forward (turbopolar_fast_attention.py:293-298)."""
    global _orig_llama_attention_forward, _orig_llama_model_forward
    if _orig_llama_attention_forward is not None:
        _llama.LlamaAttention.forward = _orig_llama_attention_forward
        _orig_llama_attention_forward = None
    if _orig_llama_model_forward is not None:
        _llama.LlamaModel.forward = _orig_llama_model_forward
        _orig_llama_model_forward = None


def load_local_llama(path, device="cuda", dtype=torch.float16, patch: bool = True):
    """A Llama checkpoint from a local directory (``save_pretrained`` layout:
    ``config.json`` plus safetensors weights), ready for TurboPolar decode: the
    model in eval mode on ``device`` in ``dtype`` with eager attention, and the
    decode hook patched in (``patch``).  The counterpart of the reference
    benchmark's ``mlx_lm.load(path)`` (run_fast_attention_bench.py:155) for a
    local path only: ``local_files_only`` makes a missing file an error instead
    of a download.  Returns the model; ``make_turbo_cache(model)`` gives its
    cache."""
    from transformers import LlamaForCausalLM

    model = LlamaForCausalLM.from_pretrained(str(path), local_files_only=True, dtype=dtype,
                                             attn_implementation="eager", use_safetensors=True)
    model = model.to(device).eval()
    if patch:
        patch_llama_attention(model)
    return model


def is_patched() -> bool:
    return _llama.LlamaAttention.forward is _turbo_llama_attention_forward
