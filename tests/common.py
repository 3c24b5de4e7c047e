"""Shared helpers for the test-suite: seeded inputs, oracle page stacks, metrics."""

from __future__ import annotations

import numpy as np

import oracle

PAGE = 64
D = 128

# (int8_radii, l1_bits, deep_bits, split_dim)
LAYOUTS = {
    "default": (False, 4, 4, 64),  # TurboPolarConfig() defaults
    "fast": (True, 4, 8, 0),  # make_turbo_caches / benchmark layout
    "deep2": (False, 4, 2, 64),
    "l1_8bit": (False, 8, 4, 32),
    "odd_split": (True, 4, 2, 46),
    "int8_default_angles": (True, 4, 4, 64),
}


def gen_kv(seed: int, B: int, H: int, T: int, kind: str = "normal", dtype=np.float16):
    """Synthetic K and V ``[B, H, T, 128]`` (numpy PCG64 generator).

    kinds: ``normal`` K, V ~ N(0,1) (configs 1, 4);
    ``loguniform`` K ~ N(0,1) * c_d, c_d log-uniform in [0.25, 4] per channel
    (config 2); ``outlier`` K ~ N(0,1) with 4 channels per head x20 (config 3);
    ``studentt`` K ~ t(3) * c_d, c_d log-uniform in [0.1, 10] (config 5).
    """
    rng = np.random.default_rng(seed)
    if kind == "normal":
        k = rng.standard_normal((B, H, T, D), dtype=np.float32)
    elif kind == "loguniform":
        c = np.exp(rng.uniform(np.log(0.25), np.log(4.0), size=(1, H, 1, D))).astype(np.float32)
        k = rng.standard_normal((B, H, T, D), dtype=np.float32) * c
    elif kind == "outlier":
        k = rng.standard_normal((B, H, T, D), dtype=np.float32)
        for h in range(H):
            ch = rng.choice(D, size=4, replace=False)
            k[:, h, :, ch] *= 20.0
    elif kind == "studentt":
        c = np.exp(rng.uniform(np.log(0.1), np.log(10.0), size=(1, H, 1, D))).astype(np.float32)
        k = (rng.standard_t(3, size=(B, H, T, D)) * c).astype(np.float32)
    else:
        raise ValueError(kind)
    v = rng.standard_normal((B, H, T, D), dtype=np.float32)
    return k.astype(dtype), v.astype(dtype)


def gen_q(seed: int, B: int, Hq: int, scale: float = 1.0):
    rng = np.random.default_rng(seed + 1000)
    return (rng.standard_normal((B, Hq, D), dtype=np.float32) * scale).astype(np.float16)


def edge_page(dtype):
    """Axis-aligned pairs, signed zeros, radii at the fp16 x*x overflow edge,
    exact V quotient ties and an all-zero V group."""
    k = np.zeros((1, 1, PAGE, 128), dtype=np.float32)
    v = np.zeros((1, 1, PAGE, 128), dtype=np.float32)
    specials = [(0, 0), (1, 0), (-1, 0.0), (-1, -0.0), (0, 1), (0, -1), (1, 1), (-1, 1), (3, 4),
                (255.9, 0), (256, 0), (255, 10), (-300, 2), (1e-7, 1e-7), (65504, 65504), (-0.0, -0.0)]
    rng = np.random.default_rng(5)
    for t in range(PAGE):
        for j in range(64):
            x, y = specials[(t * 64 + j) % len(specials)] if t < 8 else rng.standard_normal(2) * 4
            k[0, 0, t, 2 * j], k[0, 0, t, 2 * j + 1] = x, y
    # V: group 0 all zero; group 1 with many exact half-ties of v / s; group 2 huge range
    v[0, 0, :, 32:64] = np.arange(32, dtype=np.float32)[None, :] * 0.5 - 8
    v[0, 0, :, 32] = 127.0
    v[0, 0, :, 64:96] = rng.standard_normal((PAGE, 32)) * 1000
    v[0, 0, :, 96:] = rng.standard_normal((PAGE, 32)) * 1e-6
    return k.astype(dtype), v.astype(dtype)


def oracle_pages(k: np.ndarray, v: np.ndarray, layout):
    """Oracle-encode ``[B,H,S*64,D]`` inputs page by page and stack to 5-D."""
    int8, l1b, deepb, split = layout
    B, H, T, _ = k.shape
    S = T // PAGE
    enc = [
        oracle.encode_block(k[:, :, s * PAGE:(s + 1) * PAGE], l1_bits=l1b, deep_bits=deepb,
                            split_dim=split, use_int8_radii=int8)
        for s in range(S)
    ]
    blk = {
        "radii": np.stack([e["radii"] for e in enc], axis=2),
        "radii_scales": np.stack([e["radii_scales"] for e in enc], axis=2) if int8 else None,
        "angle_codes_l1": np.stack([e["angle_codes_l1"] for e in enc], axis=2),
        "angle_codes_deep": np.stack([e["angle_codes_deep"] for e in enc], axis=2),
        "metadata": enc[0]["metadata"],
    }
    codes, scales = oracle.quantize_block(v.reshape(B, H, S, PAGE, D))
    return blk, (codes, scales)


def max_abs(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-30))


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-12))


# Tolerances stated by BASELINE.json's north_star for attention outputs
# (fp16 output, fp32 accumulation): max-abs 2e-3 and relative L2 1e-3.
ATOL = 2e-3
RTOL_L2 = 1e-3


GOLDEN_DIR = __import__("pathlib").Path(__file__).resolve().parent / "golden"


def load_golden(name: str) -> dict:
    """A committed fixture file from tests/golden as a dict of arrays."""
    with np.load(GOLDEN_DIR / name, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def within_f16_ulp(got, ref) -> bool:
    """|got - ref| <= one fp16 ulp of ref, elementwise (fp16 decode outputs)."""
    ref64 = np.asarray(ref, np.float64)
    ulp = np.spacing(np.abs(np.asarray(ref, np.float16))).astype(np.float64)
    return bool(np.all(np.abs(np.asarray(got, np.float64) - ref64) <= ulp + 1e-12))
