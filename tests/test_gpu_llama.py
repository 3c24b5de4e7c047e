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
