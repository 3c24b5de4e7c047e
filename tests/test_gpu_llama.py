"""The transformers Llama hook end to end on the GPU (turbopolar_fast_attention.py:
232-298 of the reference, with run_fast_attention_bench.py's checks).

A randomly initialised float32 Llama (2 layers, 8 q / 2 kv heads, head_dim 128)
runs the same teacher-forced tokens three ways:

* dense: the model's own DynamicCache;
* fused: a TurboPolarCache with the patch, so every single-token step runs
  tp_decode_attention over the compressed pages plus the dense tail;
* decompress-on-read: a twin TurboPolarCache without the patch, so every step
  appends, decodes the pages (tp_decode_pages) and runs the model's attention.

Fused and decompress-on-read see the same compressed cache, so their logits
agree closely (a wrong RoPE position, GQA mapping or output layout would not);
against dense, the logits keep the reference benchmark's quality measures
(cosine, top-1 agreement) high.
"""

import numpy as np
import pytest
import torch

transformers = pytest.importorskip("transformers")

from turbopolar_amd import llama as tl  # noqa: E402
from turbopolar_amd.fast_attention import TurboPolarFastCache  # noqa: E402

pytestmark = pytest.mark.gpu


def _model(device):
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=512, hidden_size=1024, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=128, max_position_embeddings=4096,
                      attn_implementation="eager")
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).to(device=device, dtype=torch.float32).eval()


def _cos(a, b):
    a, b = a.double().flatten(), b.double().flatten()
    return float((a @ b) / (a.norm() * b.norm()))


def test_fused_decode_matches_decompress_on_read(device):
    model = _model(device)
    g = torch.Generator().manual_seed(1)
    tokens = torch.randint(0, 512, (1, 170), generator=g).to(device)
    prompt, steps = 100, 70  # the decode steps cross the page boundary at 128
    calls = {"n": 0}
    orig = TurboPolarFastCache.decode_attention

    def counted(self, *a, **k):
        calls["n"] += 1
        return orig(self, *a, **k)

    from transformers import DynamicCache

    dense = DynamicCache(config=model.config)
    fused = tl.make_turbo_cache(model)
    twin = tl.make_turbo_cache(model)
    with torch.no_grad():
        ld = [model(tokens[:, :prompt], past_key_values=dense, use_cache=True).logits[0, -1]]
        lt = [model(tokens[:, :prompt], past_key_values=twin, use_cache=True).logits[0, -1]]
        TurboPolarFastCache.decode_attention = counted
        tl.patch_llama_attention(model)
        try:
            lf = [model(tokens[:, :prompt], past_key_values=fused, use_cache=True).logits[0, -1]]
            for t in range(prompt, prompt + steps):
                step = tokens[:, t:t + 1]
                lf.append(model(step, past_key_values=fused, use_cache=True).logits[0, -1])
                tl.unpatch_llama_attention(model)
                lt.append(model(step, past_key_values=twin, use_cache=True).logits[0, -1])
                ld.append(model(step, past_key_values=dense, use_cache=True).logits[0, -1])
                tl.patch_llama_attention(model)
        finally:
            tl.unpatch_llama_attention(model)
            TurboPolarFastCache.decode_attention = orig
    torch.cuda.synchronize()
    assert calls["n"] == steps * 2  # every decode step of both layers ran the fused kernel
    assert fused.get_seq_length() == prompt + steps == twin.get_seq_length()
    cos_ft = [_cos(a, b) for a, b in zip(lf, lt)]
    cos_fd = [_cos(a, b) for a, b in zip(lf, ld)]
    top1 = np.mean([int(a.argmax() == b.argmax()) for a, b in zip(lf, ld)])
    print(f"[llama] fused vs decompress-on-read cosine min {min(cos_ft):.6f}; "
          f"fused vs dense cosine min {min(cos_fd):.5f}, top-1 agreement {top1:.3f}", flush=True)
    assert min(cos_ft) >= 0.9999
    assert min(cos_fd) >= 0.99 and top1 >= 0.9


def test_nonstandard_mask_is_rejected(device):
    model = _model(device)
    cache = tl.make_turbo_cache(model)
    ids = torch.arange(8, device=device)[None]
    with torch.no_grad():
        model(ids, past_key_values=cache, use_cache=True)
        tl.patch_llama_attention(model)
        try:
            mask = torch.ones((1, 9), dtype=torch.long, device=device)
            mask[0, 2] = 0  # a padded position: not the full-history causal mask
            with pytest.raises(NotImplementedError, match="standard causal full-history masks"):
                model(torch.tensor([[3]], device=device), attention_mask=mask, past_key_values=cache, use_cache=True)
        finally:
            tl.unpatch_llama_attention(model)


def test_hook_attention_matches_oracle(device):
    """Layer 1's fused decode inside the patched model, step by step, against
    the oracle's _cpu_online_attention_dense_tail (metal.py:293-332) on the
    identical state: q after RoPE as the hook hands it over (fp16, as the
    kernel takes it), the cache's stored pages and dense tail after the
    step's append, the step's sequence length and fp16(scale).  Steps cover a
    tail-only cache, a page completed by the step and a partial tail."""
    import oracle
    from common import ATOL, RTOL_L2, max_abs, rel_l2

    model = _model(device)
    g = torch.Generator().manual_seed(3)
    tokens = torch.randint(0, 512, (1, 140), generator=g).to(device)
    prompt = 60
    seen = []
    orig = TurboPolarFastCache.decode_attention

    def capture(self, q, k_new, v_new, scale, **kw):
        out = orig(self, q, k_new, v_new, scale, **kw)
        if self is cache.fast(1):
            rt = self.runtime
            block, qv, tk, tv, _, seq = rt.get_fused_attention_inputs()
            host = lambda t: None if t is None else t.detach().cpu().numpy()  # noqa: E731
            seen.append({
                "q": q[:, :, 0].to(torch.float16).cpu().numpy(), "scale": scale, "seq": seq,
                "blk": None if block is None else {
                    "radii": host(block.radii),
                    "radii_scales": None if block.radii_scales is None else
                    host(block.radii_scales).reshape(block.radii.shape[:3] + (1, 1)),
                    "angle_codes_l1": host(block.angle_codes_l1), "angle_codes_deep": host(block.angle_codes_deep),
                    "metadata": block.metadata},
                "qv": None if qv is None else (host(qv.codes), host(qv.scales)),
                "tk": host(tk), "tv": host(tv), "out": out.float().cpu().numpy(),
            })
        return out

    cache = tl.make_turbo_cache(model)
    with torch.no_grad():
        model(tokens[:, :prompt], past_key_values=cache, use_cache=True)
        TurboPolarFastCache.decode_attention = capture
        tl.patch_llama_attention(model)
        try:
            for t in range(prompt, prompt + 75):  # 61 .. 135 tokens: 0 -> 2 pages
                model(tokens[:, t:t + 1], past_key_values=cache, use_cache=True)
        finally:
            tl.unpatch_llama_attention(model)
            TurboPolarFastCache.decode_attention = orig
    assert len(seen) == 75
    checked = 0
    for i, st in enumerate(seen):
        if i % 7 and i not in (2, 3, 67, 68):  # every 7th step, and both sides of the page completions at 64, 128
            continue
        hkv = st["tk"].shape[1] if st["tk"] is not None else st["blk"]["radii"].shape[1]
        empty = np.zeros((1, hkv, 0, 128), np.float16)
        tk = st["tk"] if st["tk"] is not None else empty
        tv = st["tv"] if st["tv"] is not None else empty
        scale = oracle.fp16_scale(st["scale"])
        if st["blk"] is None:
            ref = oracle.softmax_attention(st["q"], tk, tv, scale, st["seq"])
        else:
            ref = oracle.cpu_online_attention_dense_tail(st["q"], st["blk"], st["qv"], tk, tv, scale, st["seq"])
        ma, rl = max_abs(st["out"], ref), rel_l2(st["out"], ref)
        assert ma <= ATOL and rl <= RTOL_L2, f"step {i} (seq {st['seq']}): max_abs={ma:.3g} rel_l2={rl:.3g}"
        checked += 1
    assert checked >= 14 and seen[2]["blk"] is None and seen[3]["blk"] is not None and seen[3]["tk"] is None
    assert seen[67]["seq"] == 128 and seen[67]["tk"] is None and seen[68]["tk"].shape[2] == 1


def test_nonfinite_kv_in_one_layer_undoes_the_token_everywhere(device):
    """The hook defers each layer's non-finite verdict and reads them once per
    forward: a NaN in layer 1's K raises the reference's ValueError from the
    forward and leaves every layer at its previous length; the next finite
    step continues as if the bad one never happened."""
    model = _model(device)
    cache = tl.make_turbo_cache(model)
    twin = tl.make_turbo_cache(model)
    ids = torch.arange(20, device=device)[None] % 512
    with torch.no_grad():
        model(ids, past_key_values=cache, use_cache=True)
        model(ids, past_key_values=twin, use_cache=True)
        tl.patch_llama_attention(model)
        try:
            w = model.model.layers[1].self_attn.k_proj.weight
            saved = w.data.clone()
            w.data[3, :] = float("nan")
            with pytest.raises(ValueError, match="finite"):
                model(torch.tensor([[7]], device=device), past_key_values=cache, use_cache=True)
            w.data.copy_(saved)
            assert [cache.fast(i).offset for i in range(2)] == [20, 20]
            la = model(torch.tensor([[9]], device=device), past_key_values=cache, use_cache=True).logits
            lb = model(torch.tensor([[9]], device=device), past_key_values=twin, use_cache=True).logits
        finally:
            tl.unpatch_llama_attention(model)
    assert torch.equal(la, lb)
    assert [cache.fast(i).offset for i in range(2)] == [21, 21]


def test_local_checkpoint_decodes_through_the_fused_path(device, tmp_path):
    """A Llama saved to a local directory and loaded with load_local_llama
    (the offline counterpart of run_fast_attention_bench.py:155's
    mlx_lm.load(path)) decodes through tp_decode_attention, and its logits are
    those of the same weights run in memory through the same hook."""
    model = _model(device)
    model.save_pretrained(tmp_path)
    g = torch.Generator().manual_seed(3)
    tokens = torch.randint(0, 512, (1, 90), generator=g).to(device)
    prompt = 60
    calls = {"n": 0}
    orig = TurboPolarFastCache.decode_attention

    def counted(self, *a, **k):
        calls["n"] += 1
        return orig(self, *a, **k)

    def run(m):
        cache = tl.make_turbo_cache(m)
        with torch.no_grad():
            out = [m(tokens[:, :prompt], past_key_values=cache, use_cache=True).logits[0, -1]]
            for t in range(prompt, tokens.shape[1]):
                out.append(m(tokens[:, t:t + 1], past_key_values=cache, use_cache=True).logits[0, -1])
        torch.cuda.synchronize()
        return torch.stack(out)

    TurboPolarFastCache.decode_attention = counted
    try:
        loaded = tl.load_local_llama(tmp_path, device=device, dtype=torch.float32)  # patches the hook
        from_disk = run(loaded)
        in_memory = run(model)
    finally:
        tl.unpatch_llama_attention()
        TurboPolarFastCache.decode_attention = orig
    steps = tokens.shape[1] - prompt
    assert calls["n"] == 2 * steps * 2  # both runs, every decode step of both layers
    assert torch.isfinite(from_disk).all()
    assert (from_disk - in_memory).abs().max().item() <= 1e-4
