"""Host-side parts of the transformers Llama integration (no GPU): the causal
mask check (turbopolar_fast_attention.py:235-244), patch / unpatch
(:283-298) and the cache's view of lengths and mask sizes."""

import pytest
import torch

transformers = pytest.importorskip("transformers")

from turbopolar_amd import llama as tl  # noqa: E402
from turbopolar_amd.fast_attention import TurboPolarFastCache  # noqa: E402


def _tiny_model():
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=64, hidden_size=256, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=2, num_key_value_heads=1, head_dim=128, max_position_embeddings=512)
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).eval()


def test_standard_causal_mask():
    assert tl._is_standard_causal_mask(None, 1, 10)
    full = torch.ones((1, 1, 1, 10), dtype=torch.bool)
    assert tl._is_standard_causal_mask(full, 1, 10)
    assert not tl._is_standard_causal_mask(full, 1, 11)  # wrong shape
    holed = full.clone()
    holed[..., 3] = False
    assert not tl._is_standard_causal_mask(holed, 1, 10)
    # Additive form, three queries at positions 5..7 over 8 keys.
    add = torch.full((1, 1, 3, 8), float("-inf"))
    for i in range(3):
        add[0, 0, i, : 5 + i + 1] = 0.0
    assert tl._is_standard_causal_mask(add, 3, 8)
    add[0, 0, 0, 7] = 0.0  # a query that sees the future
    assert not tl._is_standard_causal_mask(add, 3, 8)


def test_patch_and_unpatch_restore_forward():
    from transformers.models.llama import modeling_llama as m

    orig = m.LlamaAttention.forward
    tl.patch_llama_attention()
    tl.patch_llama_attention()  # idempotent: the original is kept once
    assert tl.is_patched() and m.LlamaAttention.forward is not orig
    tl.unpatch_llama_attention()
    assert m.LlamaAttention.forward is orig and not tl.is_patched()
    tl.unpatch_llama_attention()
    assert m.LlamaAttention.forward is orig


def test_turbo_cache_shape_and_lengths():
    model = _tiny_model()
    cache = tl.make_turbo_cache(model)
    assert len(cache.layers) == 2
    fast = cache.fast(0)
    assert isinstance(fast, TurboPolarFastCache)
    # The reference's benchmark layout (make_turbo_caches): int8 log radii, 8-bit deep angles.
    assert fast.config.use_int8_radii and fast.config.k_angle_bits_deep == 8 and fast.config.split_dim == 0
    assert fast.config.num_q_heads == 2 and fast.config.num_kv_heads == 1
    assert cache.get_seq_length() == 0
    assert cache.get_mask_sizes(5, 0) == (5, 0)
    assert cache.nbytes == 0


def test_unpatched_model_ignores_turbo_forward():
    """Without the patch the model runs its own attention with its own cache."""
    model = _tiny_model()
    ids = torch.arange(6)[None]
    with torch.no_grad():
        a = model(ids).logits
        tl.patch_llama_attention()
        try:
            b = model(ids).logits  # no TurboPolarCache: the original forward runs
        finally:
            tl.unpatch_llama_attention()
    assert torch.equal(a, b)


def test_load_local_llama(tmp_path):
    """A checkpoint saved to a local directory loads with its weights intact,
    eager attention and the requested dtype (the counterpart of
    run_fast_attention_bench.py:155's mlx_lm.load(path)); patch=True installs
    the decode hook; a missing directory is an error, never a download."""
    model = _tiny_model()
    model.save_pretrained(tmp_path)
    loaded = tl.load_local_llama(tmp_path, device="cpu", dtype=torch.float32, patch=False)
    assert not tl.is_patched()
    assert loaded.dtype == torch.float32 and loaded.config._attn_implementation == "eager"
    ref = model.state_dict()
    got = loaded.state_dict()
    assert ref.keys() == got.keys() and all(torch.equal(ref[k], got[k]) for k in ref)
    half = tl.load_local_llama(tmp_path, device="cpu", dtype=torch.float16, patch=True)
    try:
        assert tl.is_patched() and half.dtype == torch.float16
    finally:
        tl.unpatch_llama_attention()
    assert not tl.is_patched()
    with pytest.raises(OSError):
        tl.load_local_llama(tmp_path / "missing", device="cpu", patch=False)
