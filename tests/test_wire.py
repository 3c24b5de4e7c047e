"""Page snapshot format (turbopolar_amd.wire) on the host: round trips, the
file's safetensors framing, and rejection of malformed snapshots.

The reference has no on-disk format (its caches live in memory only,
rfsn_v11/generation/turbo_polar_cache.py:18-395); these tests pin the format
against the safetensors file layout itself (8-byte little-endian header
length, JSON header with dtype / shape / data_offsets and __metadata__) and
against the runtime state it must restore bit for bit.  The pages are filled
with random bytes: a snapshot is layout, not arithmetic, so no encode is
needed (and none runs without a GPU)."""

import json
import struct

import numpy as np
import pytest
import torch

from turbopolar_amd import TurboPolarConfig, TurboPolarKVCacheRuntime, wire

PAGE = 64
LAYOUTS = {  # int8 radii, l1 bits, deep bits, split_dim
    "default": (False, 4, 4, 64),
    "fast": (True, 4, 2, 46),
    "all_deep": (False, 4, 8, 0),
    "all_l1": (True, 8, 4, 128),
}


def _filled_runtime(layout, pages, tail, B=2, H=4, dtype=torch.float16, seed=0):
    int8, l1b, deepb, split = LAYOUTS[layout]
    cfg = TurboPolarConfig(num_q_heads=2 * H, num_kv_heads=H, use_int8_radii=int8, k_angle_bits_level1=l1b,
                           k_angle_bits_deep=deepb, split_dim=split)
    rt = TurboPolarKVCacheRuntime(cfg)
    g = torch.Generator().manual_seed(seed)

    def fill(t):
        if t is None:
            return
        raw = torch.randint(0, 256, (t.numel() * t.element_size(),), dtype=torch.uint8, generator=g)
        t.view(-1).view(torch.uint8).copy_(raw)
        if t.dtype == torch.float16:  # keep values finite: clear the top exponent bit
            t.view(torch.int16).bitwise_and_(0x3FFF)

    if pages:
        rt.k_storage.reserve(pages, rt.polar_encoder, B, H, "cpu")
        rt.v_storage.reserve(pages, B, H, "cpu")
        for t in (rt.k_storage.radii, rt.k_storage.angle_codes_l1, rt.k_storage.angle_codes_deep,
                  rt.k_storage.radii_scales, rt.v_storage.codes, rt.v_storage.scales):
            fill(t)
        rt.k_storage.block_count = rt.v_storage.block_count = pages
    if tail:
        rt._tail_k = torch.randn((B, H, PAGE, 128), generator=g).to(dtype)
        rt._tail_v = torch.randn((B, H, PAGE, 128), generator=g).to(dtype)
        rt._tail_len = tail
    rt._batch_size, rt._num_kv_heads, rt._head_dim, rt._input_dtype = B, H, 128, dtype
    rt._initialized = True
    rt.actual_seq_len = pages * PAGE + tail
    rt.total_blocks = pages
    rt.bytes_written = 12345 + pages
    rt.bytes_read = 77
    rt.compression_time_ns = 999
    return rt


def _assert_same_state(a, b):
    S = a.k_storage.block_count
    assert b.k_storage.block_count == b.v_storage.block_count == S
    if S:
        for x, y in ((a.k_storage.radii, b.k_storage.radii), (a.k_storage.angle_codes_l1, b.k_storage.angle_codes_l1),
                     (a.k_storage.angle_codes_deep, b.k_storage.angle_codes_deep),
                     (a.v_storage.codes, b.v_storage.codes), (a.v_storage.scales, b.v_storage.scales)):
            assert x.dtype == y.dtype and x.shape == y.shape  # same capacity too
            assert torch.equal(x[:, :, :S].cpu(), y[:, :, :S].cpu())
        if a.k_storage.radii_scales is None:
            assert b.k_storage.radii_scales is None
        else:
            assert torch.equal(a.k_storage.radii_scales[:, :, :S].cpu(), b.k_storage.radii_scales[:, :, :S].cpu())
    if a._tail_len:
        assert torch.equal(a.partial_k.cpu(), b.partial_k.cpu()) and torch.equal(a.partial_v.cpu(), b.partial_v.cpu())
    else:
        assert b.partial_k is None
    for f in ("actual_seq_len", "total_blocks", "bytes_written", "bytes_read", "compression_time_ns",
              "_batch_size", "_num_kv_heads", "_head_dim", "_input_dtype", "_tail_len", "_initialized"):
        assert getattr(a, f) == getattr(b, f), f
    assert a.config == b.config
    assert a.get_io_telemetry() == b.get_io_telemetry()


@pytest.mark.parametrize("layout", sorted(LAYOUTS))
@pytest.mark.parametrize("pages,tail", [(1, 0), (5, 17), (0, 9), (9, 63)])
def test_round_trip_through_file(tmp_path, layout, pages, tail):
    rt = _filled_runtime(layout, pages, tail, seed=pages * 64 + tail)
    path = tmp_path / "cache.safetensors"
    wire.save(rt, str(path))
    back = wire.load(str(path), "cpu")
    _assert_same_state(rt, back)


def test_round_trip_float32_tail_and_growth_telemetry():
    rt = _filled_runtime("default", 3, 5, dtype=torch.float32)
    # growth history as the doubling rule leaves it after 20 single-page appends
    rt.k_storage.reserve(20, rt.polar_encoder, 2, 4, "cpu")
    rt.v_storage.reserve(20, 2, 4, "cpu")
    assert rt.k_storage.capacity == 32 and rt.k_storage.reallocation_count == 3
    back = wire.load_state_dict(*wire.state_dict(rt), "cpu")
    _assert_same_state(rt, back)
    assert back.k_storage.bytes_copied_during_growth == rt.k_storage.bytes_copied_during_growth > 0


def test_snapshot_holds_only_valid_pages(tmp_path):
    rt = _filled_runtime("fast", 5, 0)
    assert rt.k_storage.capacity == 8
    tensors, meta = wire.state_dict(rt)
    assert sorted(tensors) == ["k.angle_deep", "k.angle_l1", "k.radii", "k.radii_scales", "v.codes", "v.scales"]
    assert all(t.shape[2] == 5 for t in tensors.values())
    l1_row, deep_row = rt.polar_encoder.row_bytes()
    per_page = PAGE * (64 + l1_row + deep_row) + 2 + PAGE * 128 + PAGE * 4 * 2  # int8 radii + fp16 scale
    assert sum(t.numel() * t.element_size() for t in tensors.values()) == 2 * 4 * 5 * per_page


def test_file_is_plain_safetensors(tmp_path):
    """Parse the file by hand (the safetensors layout), independent of the library."""
    rt = _filled_runtime("default", 2, 3, B=1, H=2)
    path = tmp_path / "c.safetensors"
    wire.save(rt, str(path))
    raw = path.read_bytes()
    (n,) = struct.unpack("<Q", raw[:8])
    header = json.loads(raw[8 : 8 + n])
    body = raw[8 + n :]
    meta = header.pop("__metadata__")
    assert meta["format"] == "turbopolar-pages" and meta["version"] == "1"
    assert meta["pages"] == "2" and meta["tail_tokens"] == "3" and meta["actual_seq_len"] == "131"
    assert json.loads(meta["config"])["num_kv_heads"] == 2
    assert header["v.codes"]["dtype"] == "I8" and header["v.codes"]["shape"] == [1, 2, 2, 1, 64, 128]
    assert header["k.radii"]["dtype"] == "F16" and header["k.angle_l1"]["dtype"] == "U8"
    b, e = header["v.codes"]["data_offsets"]
    got = np.frombuffer(body[b:e], dtype=np.int8).reshape(1, 2, 2, 1, 64, 128)
    assert np.array_equal(got, rt.v_storage.codes[:, :, :2].numpy())
    b, e = header["tail.k"]["data_offsets"]
    got = np.frombuffer(body[b:e], dtype=np.float16).reshape(1, 2, 3, 128)
    assert np.array_equal(got, rt.partial_k.numpy())


def _mutated(rt, fn):
    tensors, meta = wire.state_dict(rt)
    tensors, meta = dict(tensors), dict(meta)
    fn(tensors, meta)
    return tensors, meta


@pytest.mark.parametrize("mutation,msg", [
    (lambda t, m: m.update(format="other"), "not a TurboPolar page snapshot"),
    (lambda t, m: m.update(version="2"), "unsupported snapshot version"),
    (lambda t, m: m.pop("actual_seq_len"), "malformed snapshot metadata"),
    (lambda t, m: m.update(input_dtype="torch.int8"), "malformed snapshot metadata"),
    (lambda t, m: m.update(actual_seq_len="200"), "inconsistent snapshot"),
    (lambda t, m: m.update(tail_tokens="64", actual_seq_len="256"), "inconsistent snapshot"),
    (lambda t, m: m.update(k_capacity="2"), "inconsistent snapshot"),
    (lambda t, m: m.update(head_dim="64"), "does not match its config"),
    (lambda t, m: t.pop("v.scales"), "lacks v.scales"),
    (lambda t, m: t.update({"k.radii": t["k.radii"].to(torch.float32)}), "k.radii: expected"),
    (lambda t, m: t.update({"v.codes": t["v.codes"][:, :, :2]}), "v.codes: expected"),
    (lambda t, m: t.update({"tail.k": t["tail.k"][:, :, :3]}), "tail.k: expected"),
])
def test_malformed_snapshots_are_rejected(mutation, msg):
    rt = _filled_runtime("default", 3, 7, B=1, H=2)
    tensors, meta = _mutated(rt, mutation)
    with pytest.raises(ValueError, match=msg):
        wire.load_state_dict(tensors, meta, "cpu")


def test_empty_cache_cannot_be_saved():
    rt = TurboPolarKVCacheRuntime(TurboPolarConfig())
    with pytest.raises(ValueError, match="empty cache"):
        wire.state_dict(rt)
    with pytest.raises(TypeError):
        wire.state_dict(object())


def test_snapshot_shares_no_memory_with_the_cache():
    """A full-capacity cache has contiguous page slices: the snapshot must
    still copy them, so later changes to the cache leave it alone."""
    rt = _filled_runtime("default", 4, 3)
    assert rt.k_storage.capacity == 4  # the [:, :, :4] slices are the whole buffers
    tensors, _ = wire.state_dict(rt)
    before = {k: v.clone() for k, v in tensors.items()}
    rt.k_storage.radii.zero_()
    rt.v_storage.codes.fill_(7)
    rt._tail_k.zero_()
    for k, v in tensors.items():
        assert torch.equal(v, before[k]), k
