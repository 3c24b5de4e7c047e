"""TurboPolarConfig contract: the reference's validation messages
(rfsn_v11/candidates/turbo_polar_config.py:27-55; its
tests/unit/test_supported_config_contract.py and tests/test_turbo_polar_cache_runtime.py:80-88)."""

import math

import pytest

from turbopolar_amd import TurboPolarConfig


def test_supported_config_constructs():
    cfg = TurboPolarConfig(head_dim=128, block_size=64, num_q_heads=8, num_kv_heads=4, use_qjl=False,
                           storage_mode="kv_quant")
    assert cfg.head_dim == 128 and cfg.block_size == 64 and not cfg.use_qjl
    assert cfg.attention_scale == 1.0 / math.sqrt(128)
    assert TurboPolarConfig(attention_scale=0.5).attention_scale == 0.5


def test_defaults_are_the_default_layout():
    cfg = TurboPolarConfig()
    assert (cfg.k_angle_bits_level1, cfg.k_angle_bits_deep, cfg.split_dim, cfg.use_int8_radii) == (4, 4, 64, False)


@pytest.mark.parametrize("kw,msg", [
    (dict(head_dim=64), "head_dim == 128"),
    (dict(head_dim=256), "head_dim == 128"),
    (dict(block_size=32), "block_size == 64"),
    (dict(use_qjl=True), "use_qjl=False"),
    (dict(storage_mode="dense_v_debug"), "storage_mode='kv_quant'"),
    (dict(storage_mode="k_only_first"), "storage_mode='kv_quant'"),
    (dict(storage_mode="bogus"), "unknown storage_mode"),
    (dict(v_bits=4), "v_bits must be 8"),
    (dict(num_q_heads=7, num_kv_heads=4), "num_q_heads must be divisible"),
    (dict(split_dim=63), "split_dim must be even"),
    (dict(split_dim=130), "split_dim must be even"),
    (dict(block_size=0), "block_size must be positive"),
    (dict(head_dim=127), "divisible by 2"),
    (dict(qjl_proj_dim=12), "divisible by 8"),
    (dict(qjl_proj_dim=0), "qjl_proj_dim must be positive"),
])
def test_rejections(kw, msg):
    base = dict(head_dim=128, block_size=64, num_q_heads=4, num_kv_heads=4)
    base.update(kw)
    with pytest.raises(ValueError, match=msg):
        TurboPolarConfig(**base)


def test_frozen_and_replace_revalidates():
    import dataclasses

    cfg = TurboPolarConfig()
    with pytest.raises(dataclasses.FrozenInstanceError):
        cfg.head_dim = 64
    assert dataclasses.replace(cfg, attention_scale=0.25).attention_scale == 0.25
    with pytest.raises(ValueError):
        dataclasses.replace(cfg, block_size=32)
