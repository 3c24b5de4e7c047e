"""The committed golden fixtures (tests/golden) against the oracle on the CPU.

Inputs regenerate from the seeded generators; encoded codes and scales,
decoded V and the edge pages reproduce byte for byte; decoded K within one
fp16 ulp (the f32 cos/sin of the host's libm may differ in the last bit);
attention outputs within 1e-6 (float64 evaluation stored as float32).
"""

import numpy as np
import pytest

from common import load_golden, within_f16_ulp
from golden import make_fixtures

FILES = make_fixtures.build_all()


@pytest.mark.parametrize("fname", sorted(FILES))
def test_oracle_reproduces_fixture(fname):
    stored = load_golden(fname)
    fresh = FILES[fname]
    assert sorted(stored) == sorted(fresh)
    for key, ref in stored.items():
        got = np.asarray(fresh[key])
        assert got.shape == ref.shape and got.dtype == ref.dtype, key
        if key == "k_decoded":
            assert within_f16_ulp(got, ref), key
        elif key.startswith("out_"):
            assert np.allclose(got, ref, rtol=0, atol=1e-6), key
        else:
            assert np.array_equal(got.view(np.uint8), ref.view(np.uint8)), key


def test_fixture_coverage():
    """Tails 0/1/37/63, GQA 1/4/8, the masked suffix and both dtypes of the edge page."""
    d = load_golden("layout_default.npz")
    outs = {k for k in d if k.startswith("out_")}
    assert outs == {f"out_g{g}_t{t}" for g in (1, 4, 8) for t in (0, 1, 37, 63)} | {"out_g4_masked"}
    assert {"float16__radii", "float32__radii"} <= set(d)
    f = load_golden("layout_fast.npz")
    assert f["radii"].dtype == np.int8 and f["radii_scales"].shape == (1, 2, 2, 1, 1)
    assert f["angle_codes_l1"].shape[-1] == 0 and f["angle_codes_deep"].shape[-1] == 64
