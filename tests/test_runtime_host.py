"""Runtime host logic without a GPU: the append validation contract
(turbo_polar_cache.py:55-104 of the reference), dense-tail bookkeeping below one
page, telemetry, reset, the storage doubling rule, and that page flushes on a
CPU tensor fail loudly instead of falling back to a CPU path."""

import numpy as np
import pytest
import torch

from turbopolar_amd import PolarKBlockStorage, TurboPolarConfig, TurboPolarFastCache, TurboPolarKVCacheRuntime
from turbopolar_amd.storage import _doublings


def _rt(hkv=4):
    return TurboPolarKVCacheRuntime(TurboPolarConfig(num_q_heads=4, num_kv_heads=hkv))


def _x(B=1, H=4, T=1, D=128, dtype=torch.float16):
    return torch.randn((B, H, T, D)).to(dtype)


def test_rejects_non_tensors():
    with pytest.raises(TypeError):
        _rt().append(np.zeros((1, 4, 1, 128)), np.zeros((1, 4, 1, 128)))


@pytest.mark.parametrize("k,v,msg", [
    (torch.zeros(1, 4, 128), torch.zeros(1, 4, 128), "4-D inputs"),
    (torch.zeros(1, 4, 1, 128), torch.zeros(1, 4, 2, 128), "must match"),
    (torch.zeros(1, 4, 0, 128), torch.zeros(1, 4, 0, 128), "at least one token"),
    (torch.zeros(1, 4, 1, 128), torch.zeros(1, 4, 1, 128, dtype=torch.float16), "dtype"),
    (torch.zeros(1, 4, 1, 128, dtype=torch.bfloat16), torch.zeros(1, 4, 1, 128, dtype=torch.bfloat16),
     "only float16 and float32"),
    (torch.zeros(1, 2, 1, 128), torch.zeros(1, 2, 1, 128), "KV heads"),
    (torch.zeros(1, 4, 1, 64), torch.zeros(1, 4, 1, 64), "head_dim"),
])
def test_append_validation(k, v, msg):
    with pytest.raises(ValueError, match=msg):
        _rt().append(k, v)


def test_nonfinite_rejected():
    k = _x(T=2)
    k[0, 0, 0, 0] = float("inf")
    with pytest.raises(ValueError, match="finite"):
        _rt().append(k, _x(T=2))


def test_invariants_persist_and_reset():
    rt = _rt()
    rt.append(_x(T=3), _x(T=3))
    with pytest.raises(ValueError, match="batch size changed"):
        rt.append(_x(B=2), _x(B=2))
    with pytest.raises(ValueError, match="dtype changed"):
        rt.append(_x(dtype=torch.float32), _x(dtype=torch.float32))
    with pytest.raises(ValueError, match="KV head count changed"):
        rt.append(_x(H=2), _x(H=2))
    rt.reset()
    assert rt.partial_k is None and rt.actual_seq_len == 0
    rt.append(_x(B=2, T=1), _x(B=2, T=1))
    assert rt._batch_size == 2


def test_tail_bookkeeping_below_one_page():
    rt = _rt()
    ks = [_x(T=t) for t in (5, 20, 38)]
    for k in ks:
        rt.append(k, k)
    assert rt.actual_seq_len == 63
    assert torch.equal(rt.partial_k, torch.cat(ks, dim=2))
    tel = rt.get_io_telemetry()
    assert tel["partial_tokens"] == 63 and tel["total_blocks"] == 0
    assert tel["actual_cache_bytes"] == 2 * 4 * 63 * 128 * 2
    assert tel["compression_ratio"] == 1.0
    block, qv, tk, tv, qjl, seq = rt.get_fused_attention_inputs()
    assert block is None and qv is None and qjl is None and seq == 63 and tk.shape == (1, 4, 63, 128)


def test_page_flush_on_cpu_fails_loudly():
    rt = _rt()
    rt.append(_x(T=63), _x(T=63))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        rt.append(_x(T=1), _x(T=1))


def test_decode_shape_contract():
    cache_cfg = TurboPolarConfig(num_q_heads=4, num_kv_heads=2)
    v = TurboPolarFastCache._validate_decode_shape
    q = torch.zeros(1, 4, 1, 128)
    kv = torch.zeros(1, 2, 1, 128)
    with pytest.raises(NotImplementedError, match="batch size 1"):
        v(torch.zeros(2, 4, 1, 128), torch.zeros(2, 2, 1, 128), torch.zeros(2, 2, 1, 128), cache_cfg)
    with pytest.raises(ValueError, match="single query"):
        v(torch.zeros(1, 4, 2, 128), kv, kv, cache_cfg)
    with pytest.raises(NotImplementedError, match="head_dim == 128"):
        v(torch.zeros(1, 4, 1, 64), torch.zeros(1, 2, 1, 64), torch.zeros(1, 2, 1, 64), cache_cfg)
    with pytest.raises(ValueError, match="GQA ratio"):
        v(torch.zeros(1, 5, 1, 128), kv, kv, cache_cfg)
    with pytest.raises(ValueError, match="4-D"):
        v(torch.zeros(1, 4, 128), kv, kv, cache_cfg)
    v(q, kv, kv, cache_cfg)


def test_storage_doubling_rule():
    """Capacity 4 * 2^k and the reference's _grow call sequence (storage.py:57-87)."""
    assert _doublings(4, 4) == ([], 4)
    assert _doublings(4, 5) == ([4], 8)
    assert _doublings(4, 512) == ([4, 8, 16, 32, 64, 128, 256], 512)
    assert _doublings(8, 2049) == ([8, 16, 32, 64, 128, 256, 512, 1024, 2048], 4096)


def test_storage_append_and_views_on_cpu():
    """PolarKBlockStorage.append: lazy init at capacity 4, doubling, growth bytes."""
    from turbopolar_amd.payload import PolarKeyBlock

    st = PolarKBlockStorage()
    for i in range(5):
        blk = PolarKeyBlock(
            radii=torch.full((1, 2, 64, 64), float(i), dtype=torch.float16),
            angle_codes_l1=torch.full((1, 2, 64, 16), i, dtype=torch.uint8),
            angle_codes_deep=torch.full((1, 2, 64, 16), i, dtype=torch.uint8),
            shape=(1, 2, 64, 128), block_size=64, head_dim=128, metadata={"l1_bits": 4},
        )
        st.append(blk)
    assert st.block_count == 5 and st.capacity == 8 and st.reallocation_count == 1
    assert st.bytes_copied_during_growth == 4 * (1 * 2 * 64 * (64 * 2 + 16 + 16))
    u = st.to_unified_block((1, 2, 5 * 64, 128))
    assert u.radii.shape == (1, 2, 5, 64, 64)
    assert [float(u.radii[0, 0, s, 0, 0]) for s in range(5)] == [0, 1, 2, 3, 4]
