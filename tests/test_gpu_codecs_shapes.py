"""The codecs on shapes the page encoder does not take, against the oracle.

* PolarQuantEncoder.encode_block with int8 log radii over a block of L != 64
  tokens: one log scale over the whole (b, h) row (rfsn_v11/quant/polar/
  encoder.py:34-42), through tp_log_radii_rows over the block's fp16 radii.
* GroupedVQuantizer.quantize_block / dequantize_block with any group size
  dividing the row (rfsn_v11/quant/v_quant/encoder.py:12-38), through
  tp_quantize_v_groups.

Codes and scales must be bit-exact with oracle.encode_block /
oracle.quantize_block / oracle.dequantize_block on the same inputs.
"""

import numpy as np
import pytest
import torch

import oracle
from common import LAYOUTS
from turbopolar_amd import TurboPolarConfig
from turbopolar_amd.codecs import GroupedVQuantizer, PolarQuantEncoder

pytestmark = pytest.mark.gpu


def _same(a, b):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


@pytest.mark.parametrize("layout_name", ["fast", "int8_default_angles"])
@pytest.mark.parametrize("L", [1, 37, 100, 200])
@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_int8_log_radii_any_length(device, layout_name, L, dtype):
    int8, l1b, deepb, split = LAYOUTS[layout_name]
    cfg = TurboPolarConfig(num_q_heads=4, num_kv_heads=2, use_int8_radii=int8, k_angle_bits_level1=l1b,
                           k_angle_bits_deep=deepb, split_dim=split)
    rng = np.random.default_rng(L)
    k = (rng.standard_normal((2, 2, L, 128)) * np.exp(rng.uniform(-3, 3, (1, 2, 1, 128)))).astype(dtype)
    k[0, 1, 0, :4] = 0.0  # a zero pair: log of the radius floor
    ref = oracle.encode_block(k, l1_bits=l1b, deep_bits=deepb, split_dim=split, use_int8_radii=True)
    blk = PolarQuantEncoder(cfg).encode_block(torch.from_numpy(k).to(device))
    assert _same(blk.radii.cpu().numpy(), ref["radii"])
    assert _same(blk.radii_scales.cpu().numpy().reshape(2, 2, 1, 1), ref["radii_scales"])
    assert _same(blk.angle_codes_l1.cpu().numpy(), ref["angle_codes_l1"])
    assert _same(blk.angle_codes_deep.cpu().numpy(), ref["angle_codes_deep"])


@pytest.mark.parametrize("group,D", [(1, 128), (8, 128), (16, 128), (64, 128), (128, 128), (32, 64), (24, 96)])
@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_quantize_any_group_size(device, group, D, dtype):
    rng = np.random.default_rng(group * 1000 + D)
    v = (rng.standard_normal((1, 2, 3, 5, D)) * 3).astype(dtype)
    v[0, 0, 0, 0, :group] = 0.0  # an all-zero group: the 1e-4 scale floor
    v[0, 1, 2, 4, 0] = 127.0 * 0.5  # a group whose maximum gives a round scale
    codes_ref, scales_ref = oracle.quantize_block(v, group)
    q = GroupedVQuantizer(group_size=group).quantize_block(torch.from_numpy(v).to(device))
    assert _same(q.codes.cpu().numpy(), codes_ref)
    assert _same(q.scales.cpu().numpy(), scales_ref)
    deq = GroupedVQuantizer(group_size=group).dequantize_block(q).cpu().numpy()
    assert _same(deq, oracle.dequantize_block(codes_ref, scales_ref, group))


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_int8_log_radii_nan_row(device, dtype):
    """A NaN pair in one (b, h) row: that row's max |log r| is NaN, so its scale
    is NaN and every radius code 0 (the oracle's NumPy max); the other rows are
    untouched."""
    int8, l1b, deepb, split = LAYOUTS["fast"]
    cfg = TurboPolarConfig(num_q_heads=4, num_kv_heads=2, use_int8_radii=int8, k_angle_bits_level1=l1b,
                           k_angle_bits_deep=deepb, split_dim=split)
    rng = np.random.default_rng(7)
    k = (rng.standard_normal((2, 2, 37, 128)) * 4).astype(dtype)
    k[0, 1, 5, 20] = np.nan
    ref = oracle.encode_block(k, l1_bits=l1b, deep_bits=deepb, split_dim=split, use_int8_radii=True)
    blk = PolarQuantEncoder(cfg).encode_block(torch.from_numpy(k).to(device))
    assert _same(blk.radii.cpu().numpy(), ref["radii"])
    assert _same(blk.radii_scales.cpu().numpy().reshape(2, 2, 1, 1), ref["radii_scales"])
    assert _same(blk.angle_codes_deep.cpu().numpy(), ref["angle_codes_deep"])


@pytest.mark.parametrize("group", [8, 32, 128])
@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_quantize_nan_group(device, group, dtype):
    """A NaN in a group: its scale is NaN and every code of the group 0 (the
    oracle's NumPy max); an inf elsewhere gives codes 0 around a finite v / inf."""
    rng = np.random.default_rng(group)
    v = (rng.standard_normal((1, 2, 3, 5, 128)) * 3).astype(dtype)
    v[0, 0, 1, 2, 3] = np.nan
    v[0, 1, 0, 4, 100] = np.inf
    codes_ref, scales_ref = oracle.quantize_block(v, group)
    q = GroupedVQuantizer(group_size=group).quantize_block(torch.from_numpy(v).to(device))
    assert _same(q.codes.cpu().numpy(), codes_ref)
    assert _same(q.scales.cpu().numpy(), scales_ref)
