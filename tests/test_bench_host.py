"""bench.py on the host: the algorithmic byte counts that its roofline
divides by equal the closed-form figures of the measurement plan (bytes per
step = Hkv*S*64*(Kb + 136) + Hkv*S*rs + Hkv*Tt*512 + Hq*128*2*2, tabulated
there for every BASELINE config), and the single-GPU contract holds."""

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import bench

ROOT = Path(__file__).resolve().parent.parent
D, F = bench.LAYOUTS["default"], bench.LAYOUTS["fast"]


@pytest.mark.parametrize("hq,context,layout,expected", [
    (32, 4096, D, 9_715_712), (32, 4096, F, 8_668_160),            # configs[0]
    (32, 8192, D, 19_415_040), (32, 8192, F, 17_319_936),          # configs[2] sweep
    (32, 32768, D, 77_611_008), (32, 32768, F, 69_230_592),        # configs[2] headline
    (32, 131072, D, 310_394_880), (32, 131072, F, 276_873_216),
    (64, 131072, D, 310_411_264), (64, 131072, F, 276_889_600),    # configs[4]
])
def test_decode_bytes_match_the_tabulated_figures(hq, context, layout, expected):
    assert bench.algorithmic_bytes(hq, 8, context // 64, layout) == expected


def test_layers_and_encode_bytes():
    assert 16 * bench.algorithmic_bytes(32, 8, 512, D) == 1_241_776_128  # configs[1]
    assert 16 * bench.algorithmic_bytes(32, 8, 512, F) == 1_107_689_472
    # configs[3] bulk encode: write = the compressed pages of 32k tokens x 8 heads
    assert 8 * 512 * bench.bench_page_bytes(D) == 77_594_624
    assert 8 * 512 * bench.bench_page_bytes(F) == 69_214_208
    # a dense tail adds 512 B per token and kv head (fp16 K and V)
    assert bench.algorithmic_bytes(32, 8, 512, D, tail=37) - bench.algorithmic_bytes(32, 8, 512, D) == 8 * 37 * 512


def test_k_page_bytes():
    assert bench.k_page_bytes(D) == 64 * 128 + 1024 + 1024  # fp16 radii + 4-bit l1 and deep rows
    assert bench.k_page_bytes(F) == 64 * 64 + 64 * 64 + 2  # int8 log radii + 8-bit deep row + page scale


def test_f16_ulp_gap():
    one = np.array([1.0], np.float16)
    nxt = np.nextafter(one, np.float16(2))
    assert bench._f16_ulp_gap(one, one) == 0
    assert bench._f16_ulp_gap(one, nxt) == 1
    tiny = np.array([np.float16(2.0 ** -24)])
    assert bench._f16_ulp_gap(np.array([-0.0], np.float16), np.array([0.0], np.float16)) == 0
    assert bench._f16_ulp_gap(-tiny, tiny) == 2
    assert bench._f16_ulp_gap(np.array([np.inf], np.float16), np.array([1.0], np.float16)) == 0  # non-finite skipped


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300, cwd=ROOT)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


def test_kernel_workloads_warm_up_past_the_clock_ramp():
    """The kernel workloads time their steps after tens of milliseconds of
    untimed launches (the GPU's clocks settle in between: the 32k decode step
    read about 1 us more after 20 warm-up launches than after 2000); the
    workloads that consume their warm-up steps as tokens keep short ones."""
    d = bench.WARMUP_DEFAULTS
    assert d["decode"] >= 2000 and d["qk"] >= 2000
    assert min(d["encode"], d["decompress"], d["stream"]) >= 1000
    assert d["prefill"] <= 8 and d["model"] <= 8
