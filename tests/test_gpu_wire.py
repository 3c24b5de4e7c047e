"""Page snapshots on the GPU: a cache saved and restored attends bit for bit
like the original, before and after further appends (the restored pages,
tail and counters feed the same kernels)."""

import numpy as np
import pytest
import torch

from turbopolar_amd import TurboPolarConfig, TurboPolarFastCache, wire

pytestmark = pytest.mark.gpu

LAYOUTS = {"default": (False, 4, 4, 64), "fast": (True, 4, 2, 46)}


@pytest.mark.parametrize("layout", sorted(LAYOUTS))
@pytest.mark.parametrize("prefill", [318, 640])
def test_restored_cache_attends_identically(device, tmp_path, layout, prefill):
    print(f"[wire] layout={layout} prefill={prefill}", flush=True)
    int8, l1b, deepb, split = LAYOUTS[layout]
    cfg = TurboPolarConfig(num_q_heads=8, num_kv_heads=2, use_int8_radii=int8, k_angle_bits_level1=l1b,
                           k_angle_bits_deep=deepb, split_dim=split)
    rng = np.random.default_rng(prefill)

    def t(*shape):
        return torch.from_numpy(rng.standard_normal(shape).astype(np.float16)).to(device)

    a = TurboPolarFastCache(cfg)
    a.runtime.append(t(1, 2, prefill, 128), t(1, 2, prefill, 128))
    path = tmp_path / "cache.safetensors"
    wire.save(a, str(path))
    b = wire.load_fast_cache(str(path), device)
    assert b.runtime.k_storage.radii.device == device
    assert b.runtime.get_io_telemetry() == a.runtime.get_io_telemetry()
    scale = 128 ** -0.5
    for step in range(4):  # 318 + 4 crosses a page boundary; 640 starts a new tail
        q, kn, vn = t(1, 8, 1, 128), t(1, 2, 1, 128), t(1, 2, 1, 128)
        oa = a.decode_attention(q, kn, vn, scale)
        ob = b.decode_attention(q, kn, vn, scale)
        torch.cuda.synchronize()
        assert torch.isfinite(oa).all()
        assert torch.equal(oa, ob), f"step {step}"
    assert b.runtime.actual_seq_len == prefill + 4
    assert b.runtime.get_io_telemetry() == a.runtime.get_io_telemetry()
    S = a.runtime.k_storage.block_count
    assert torch.equal(a.runtime.v_storage.codes[:, :, :S], b.runtime.v_storage.codes[:, :, :S])
    assert torch.equal(a.runtime.k_storage.radii[:, :, :S], b.runtime.k_storage.radii[:, :, :S])
