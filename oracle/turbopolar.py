"""NumPy restatement of the reference's TurboPolar CPU path (test oracle).

TEST INFRASTRUCTURE ONLY -- imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, never by the product package.

Every function cites the reference file:line it restates (paths relative to
the reference repository root).  The reference runs these steps as MLX op
graphs; MLX is not available here, so its arithmetic is restated under four
documented assumptions:

1. *Weak Python scalars.*  ``array <op> python_float`` keeps the array's dtype,
   so ``angles + np.pi`` is an fp16 add of fp16(pi) = 3.140625 (0x4248) and
   ``/ (2*pi)`` divides by fp16(2*pi) = 6.28125 (0x4648).  A 0-d
   ``mx.array(0.0)`` is *not* weak: it is float32, so the
   ``mx.where(..., mx.array(0.0), norm)`` at ``encoder.py:51`` promotes the
   normalised fp16 angles to float32 before they are multiplied by the code
   scale.
2. *Per-op fp16 rounding.*  Each fp16 op is the correctly rounded result.
   NumPy's float16 arithmetic computes in float32 and rounds per op, which
   equals the correctly rounded fp16 result for + - * / sqrt (float32 has
   24 >= 2*11+2 significand bits).
3. *Round half to even* for ``mx.round``.
4. *Correctly rounded transcendental policy.*  ``arctan2`` and ``log`` are
   evaluated in float64 and rounded once to the output dtype.  NaN cast to
   int8 gives 0 (the AArch64 ``fcvtzs`` result the reference's host would
   produce).

The attention functions compute in float64 by default (``dtype`` argument) on
the fp16 decoded K and V, which is the "ideal" value of the reference CPU path.

How each function is pinned (tests/test_oracle_pins.py,
tests/test_oracle_attention.py, tests/test_golden.py):

* pack_4bit / pack_2bit / unpack_* / layout_bytes: closed forms and round trips.
* encode_block, angle_codes_f16, atan2_cr, log_cr: known answers of the rules in
  encoder.py:24-98, an independent exact-rational restatement
  (tests/exact_f16.py) compared bit for bit, fp32-input wrap cases.
* quantize_block: known answers (zero group, group max, half-even ties) and
  the exact-rational restatement.
* qjl_projection / qjl_pack_signs / qjl_residual_sketch / qjl_dot_estimate /
  cpu_fused_qk_qjl (tests/test_oracle_qjl.py): unit columns and the seed's
  stream, single-bit known answers of the packing, a pure-Python brute force
  of the estimator, its closed forms (equal sketches: +|E||q|, complementary:
  -|E||q|, half the bits: 0) and its consistency (with many projections it
  converges to q . E, which a wrong sign, factor or bit order breaks).
* dequantize_block: exact-rational known answers element by element, the
  exact round trip of code x power-of-two values, and the quantisation error
  bound 0.53125 s + half an fp16 ulp.
* decode_block: radius invariant sqrt(kx^2 + ky^2) ~ r, decode->encode
  idempotence.
* softmax_attention, cpu_fused_qk, cpu_online_attention[_dense_v|_dense_tail]: torch
  float64 scaled_dot_product_attention, brute-force loops on one page, the
  split-K merge algebra.

Parity unpinned at the MLX boundary (MLX is not installable here): MLX's own
ulp behaviour for fp16 arctan2 / log, its scalar promotion and rounding mode
(assumptions 1-4 above), and the reduction order inside mx.sum / mx.softmax.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "F16_PI",
    "F16_TWO_PI",
    "layout_bytes",
    "pack_4bit",
    "pack_2bit",
    "unpack_4bit",
    "unpack_2bit",
    "atan2_cr",
    "log_cr",
    "angle_codes_f16",
    "encode_block",
    "quantize_block",
    "decode_block",
    "dequantize_block",
    "cpu_fused_qk",
    "cpu_online_attention",
    "cpu_online_attention_dense_v",
    "cpu_online_attention_dense_tail",
    "softmax_attention",
    "fp16_scale",
    "qjl_projection",
    "qjl_pack_signs",
    "qjl_residual_sketch",
    "qjl_dot_estimate",
    "cpu_fused_qk_qjl",
]

F16 = np.float16
F32 = np.float32
F64 = np.float64

F16_PI = F16(np.pi)  # 3.140625, bits 0x4248
F16_TWO_PI = F16(2.0 * np.pi)  # 6.28125, bits 0x4648
F32_PI = F32(np.pi)
F32_TWO_PI = F32(2.0 * np.pi)
F16_RADIUS_FLOOR = F16(1e-6)  # bits 0x0011
F16_V_SCALE_FLOOR = F16(1e-4)  # bits 0x068E


def fp16_scale(scale: float) -> float:
    """Attention scale as the reference kernels see it.

    ``metal.py:518,692,774`` pass ``config.attention_scale`` as a 0-d fp16
    array, so 1/sqrt(128) becomes 0.08837890625 (0x2DA8).
    """
    return float(F16(scale))


def layout_bytes(l1_bits: int, deep_bits: int, split_dim: int, head_dim: int = 128):
    """Packed row lengths (bytes per token) of the l1 and deep angle codes.

    Restates ``encoder.py:56-83`` with the padding of ``_pack_4bit``/``_pack_2bit``
    (``encoder.py:101-130``) and the shape assertions of
    ``tests/benchmarks/test_turbo_polar_offline.py:27-34``.
    """
    split_half = split_dim // 2
    deep_half = head_dim // 2 - split_half
    if l1_bits == 4:
        l1 = (split_half + 1) // 2
    elif l1_bits == 8:
        l1 = split_half
    else:
        raise ValueError(f"unsupported k_angle_bits_level1: {l1_bits}")
    if deep_bits == 8:
        deep = deep_half
    elif deep_bits == 4:
        deep = (deep_half + 1) // 2
    elif deep_bits == 2:
        deep = (deep_half + 3) // 4
    else:
        raise ValueError(f"unsupported k_angle_bits_deep: {deep_bits}")
    return l1, deep


# --------------------------------------------------------------------------
# bit packing -- encoder.py:101-130, decoder.py:70-85
# --------------------------------------------------------------------------

def pack_4bit(codes: np.ndarray) -> np.ndarray:
    """``PolarQuantEncoder._pack_4bit`` (encoder.py:101-113): low nibble first."""
    n = codes.shape[-1]
    pad = (2 - n % 2) % 2
    if pad:
        codes = np.concatenate([codes, np.zeros(codes.shape[:-1] + (pad,), codes.dtype)], axis=-1)
    even = codes[..., 0::2].astype(np.uint8)
    odd = codes[..., 1::2].astype(np.uint8)
    return ((even & 0x0F) | ((odd & 0x0F) << 4)).astype(np.uint8)


def pack_2bit(codes: np.ndarray) -> np.ndarray:
    """``PolarQuantEncoder._pack_2bit`` (encoder.py:116-130): lowest pair of bits first."""
    n = codes.shape[-1]
    pad = (4 - n % 4) % 4
    if pad:
        codes = np.concatenate([codes, np.zeros(codes.shape[:-1] + (pad,), codes.dtype)], axis=-1)
    c = codes.astype(np.uint8)
    out = (c[..., 0::4] & 3) | ((c[..., 1::4] & 3) << 2) | ((c[..., 2::4] & 3) << 4) | ((c[..., 3::4] & 3) << 6)
    return out.astype(np.uint8)


def unpack_4bit(packed: np.ndarray, n: int) -> np.ndarray:
    """``PolarQuantDecoder._unpack_4bit`` (decoder.py:70-77)."""
    low = packed & 0x0F
    high = (packed >> 4) & 0x0F
    inter = np.stack([low, high], axis=-1).reshape(packed.shape[:-1] + (-1,))
    return inter[..., :n]


def unpack_2bit(packed: np.ndarray, n: int) -> np.ndarray:
    """``PolarQuantDecoder._unpack_2bit`` (decoder.py:79-85)."""
    parts = [(packed >> s) & 0x03 for s in (0, 2, 4, 6)]
    inter = np.stack(parts, axis=-1).reshape(packed.shape[:-1] + (-1,))
    return inter[..., :n]


# --------------------------------------------------------------------------
# transcendental policy (assumption 4)
# --------------------------------------------------------------------------

def atan2_cr(y: np.ndarray, x: np.ndarray, out_dtype) -> np.ndarray:
    """Correctly rounded ``arctan2`` in ``out_dtype`` (fp16 or fp32).

    Stands in for ``mx.arctan2`` at ``encoder.py:46``.  float64 atan2 is
    accurate to < 1 ulp, and NumPy's float64 -> float16/float32 casts round
    directly from the float64 value (no double rounding).
    """
    return np.arctan2(y.astype(F64), x.astype(F64)).astype(out_dtype)


def log_cr(r16: np.ndarray) -> np.ndarray:
    """Correctly rounded fp16 natural log of fp16 radii (``encoder.py:37``)."""
    with np.errstate(divide="ignore"):
        return np.log(r16.astype(F64)).astype(F16)


def angle_codes_f16(a16: np.ndarray, bits: int) -> np.ndarray:
    """Angle code of fp16 angles (encoder.py:47-55 with fp16 inputs).

    fp16 shift by fp16(pi) and fp16 divide by fp16(2*pi), clip to [0, 1], then the
    float32 product with (2^bits - 1) rounded half-even and clipped."""
    with np.errstate(invalid="ignore", over="ignore"):
        n = (a16.astype(F16) + F16_PI) / F16_TWO_PI
        n = np.clip(n, F16(0.0), F16(1.0))
        n = np.where(n > F16(1.0 - 1e-6), F32(0.0), n.astype(F32))
        lv = 2 ** bits - 1
        c = np.rint(n * F32(lv))
        c = np.where(np.isnan(c), 0, c)
        return np.clip(c, 0, lv).astype(np.uint8)


def _to_int8_nan0(q: np.ndarray) -> np.ndarray:
    q = np.where(np.isnan(q), 0, q)
    return np.clip(q, -128, 127).astype(np.int8)


# --------------------------------------------------------------------------
# encoders -- polar/encoder.py:24-98, v_quant/encoder.py:16-30
# --------------------------------------------------------------------------

def encode_block(
    k: np.ndarray,
    *,
    l1_bits: int = 4,
    deep_bits: int = 4,
    split_dim: int = 64,
    use_int8_radii: bool = False,
) -> dict:
    """``PolarQuantEncoder.encode_block`` (encoder.py:24-98).

    ``k`` is ``[B, H, L, D]`` float16 or float32.  Returns a dict with
    ``radii`` (fp16, or int8 codes), ``radii_scales`` (fp16 ``[B, H, 1, 1]`` or
    None), ``angle_codes_l1``, ``angle_codes_deep`` (uint8, packed) and
    ``metadata`` (the keys of encoder.py:85-97).
    """
    if k.dtype not in (F16, F32):
        raise ValueError(f"encode_block expects float16 or float32, got {k.dtype}")
    B, H, L, D = k.shape
    assert D % 2 == 0
    half_d = D // 2
    split_half = split_dim // 2
    l1_levels = 2 ** l1_bits
    deep_levels = 2 ** deep_bits
    x = k[..., 0::2]
    y = k[..., 1::2]
    with np.errstate(over="ignore", invalid="ignore"):
        if k.dtype == F16:
            # encoder.py:33 -- every op rounds to fp16, no fused multiply-add.
            radii_fp = np.sqrt(x * x + y * y)
            ang = atan2_cr(y, x, F16)
            shifted = ang + F16_PI  # weak scalar: fp16 add (encoder.py:47)
            norm = shifted / F16_TWO_PI  # fp16 divide (encoder.py:48)
            norm = np.clip(norm, F16(0.0), F16(1.0))  # encoder.py:49
            # encoder.py:51: threshold fp16(1 - 1e-6) == 1.0 never fires after the
            # clip; the float32 mx.array(0.0) promotes the result to float32.
            norm = np.where(norm > F16(1.0 - 1e-6), F32(0.0), norm.astype(F32))
        else:
            radii_fp = np.sqrt(x * x + y * y).astype(F16)
            ang = atan2_cr(y, x, F32)
            shifted = ang + F32_PI
            norm = shifted / F32_TWO_PI
            norm = np.clip(norm, F32(0.0), F32(1.0))
            norm = np.where(norm > F32(1.0 - 1e-6), F32(0.0), norm)

        if use_int8_radii:
            # encoder.py:34-42
            log_r = log_cr(np.maximum(radii_fp, F16_RADIUS_FLOOR)).astype(F32)
            log_scale = np.max(np.abs(log_r), axis=(2, 3), keepdims=True)
            log_scale = np.where(log_scale == 0, F32(1e-6), log_scale)
            ls16 = (log_scale / F32(127.0)).astype(F16)
            radii_codes = _to_int8_nan0(np.rint(log_r / ls16.astype(F32)))
            radii_scales = ls16
        else:
            radii_codes = radii_fp
            radii_scales = None

        norm = norm.astype(F32)
        norm_l1 = norm[..., :split_half]
        norm_deep = norm[..., split_half:]
        codes_l1 = np.clip(np.rint(norm_l1 * F32(l1_levels - 1)), 0, l1_levels - 1).astype(np.uint8)
        codes_deep = np.clip(np.rint(norm_deep * F32(deep_levels - 1)), 0, deep_levels - 1).astype(np.uint8)

    if l1_bits == 4:
        l1 = pack_4bit(codes_l1)
        l1_packed = True
    elif l1_bits == 8:
        l1 = codes_l1
        l1_packed = False
    else:
        raise ValueError(f"unsupported k_angle_bits_level1: {l1_bits}")
    if deep_bits == 8:
        deep = codes_deep
        deep_packed = False
    elif deep_bits == 4:
        deep = pack_4bit(codes_deep)
        deep_packed = True
    elif deep_bits == 2:
        deep = pack_2bit(codes_deep)
        deep_packed = True
    else:
        raise ValueError(f"unsupported k_angle_bits_deep: {deep_bits}")

    metadata = {
        "l1_scale": float(l1_levels - 1),
        "deep_scale": float(deep_levels - 1),
        "split_dim": split_dim,
        "l1_packed": l1_packed,
        "deep_packed": deep_packed,
        "deep_bits": deep_bits,
        "l1_bits": l1_bits,
        "int8_radii": use_int8_radii,
        "log_radii": use_int8_radii,
        "l1_original_len": split_half,
        "deep_original_len": half_d - split_half,
    }
    return {
        "radii": radii_codes,
        "radii_scales": radii_scales,
        "angle_codes_l1": l1,
        "angle_codes_deep": deep,
        "metadata": metadata,
    }


def quantize_block(v: np.ndarray, group_size: int = 32):
    """``GroupedVQuantizer.quantize_block`` (v_quant/encoder.py:16-30).

    ``v`` is ``[B, H, S, L, D]`` float16 or float32.  Returns ``(codes int8
    [B,H,S,L,D], scales fp16 [B,H,S,L,D//group])``.
    """
    B, H, S, L, D = v.shape
    assert D % group_size == 0
    r = v.reshape(B, H, S, L, D // group_size, group_size)
    m = np.max(np.abs(r), axis=-1, keepdims=True)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        if v.dtype == F16:
            s = m / F16(127.0)  # fp16 divide by the weak scalar
        else:
            s = (m / F32(127.0)).astype(F16)
        s = np.where(s == 0, F16_V_SCALE_FLOOR, s).astype(F16)
        if v.dtype == F16:
            qv = r / s  # fp16 quotient, rounded before mx.round
        else:
            qv = r / s.astype(F32)
        codes = _to_int8_nan0(np.rint(qv))
    return codes.reshape(B, H, S, L, D), s[..., 0]


# --------------------------------------------------------------------------
# decoders -- polar/decoder.py:7-67, v_quant/encoder.py:32-38
# --------------------------------------------------------------------------

def _angle_norms(angle_l1, angle_deep, meta, head_dim):
    split_half = meta.get("split_dim", head_dim // 2) // 2
    l1_orig = meta.get("l1_original_len", split_half)
    deep_orig = meta.get("deep_original_len", head_dim // 2 - split_half)
    l1_scale = F32(meta["l1_scale"])
    deep_scale = F32(meta["deep_scale"])
    if meta.get("l1_packed", False):
        c1 = unpack_4bit(angle_l1, l1_orig)
    else:
        c1 = angle_l1[..., :l1_orig]
    deep_bits = meta.get("deep_bits", 2)
    if meta.get("deep_packed", False):
        if deep_bits == 4:
            cd = unpack_4bit(angle_deep, deep_orig)
        elif deep_bits == 2:
            cd = unpack_2bit(angle_deep, deep_orig)
        else:
            raise ValueError(f"unsupported deep_bits: {deep_bits}")
    else:
        cd = angle_deep[..., :deep_orig]
    n1 = c1.astype(F32) / l1_scale
    nd = cd.astype(F32) / deep_scale
    return np.concatenate([n1, nd], axis=-1)


def decode_block(radii, radii_scales, angle_l1, angle_deep, meta, head_dim: int = 128) -> np.ndarray:
    """``PolarQuantDecoder.decode_block`` (decoder.py:7-67).

    Accepts 4-D ``[B,H,L,D/2]`` or 5-D ``[B,H,S,L,D/2]`` payloads (decoder.py:9-27);
    ``radii_scales`` is ``[B,H,1,1]`` / ``[B,H,S,1,1]`` or None.  Returns fp16
    ``[B, H, S*L, D]``.
    """
    if radii.ndim == 4:
        radii = radii[:, :, None]
        angle_l1 = angle_l1[:, :, None]
        angle_deep = angle_deep[:, :, None]
        if radii_scales is not None:
            radii_scales = radii_scales[:, :, None]
    B, H, S, L, _ = radii.shape
    norm = _angle_norms(angle_l1, angle_deep, meta, head_dim)
    angles = norm * F32_TWO_PI - F32_PI  # decoder.py:55: two separate f32 ops
    with np.errstate(over="ignore", invalid="ignore"):
        if radii_scales is not None:
            if meta.get("log_radii", False):
                r = np.exp(radii.astype(F32) * radii_scales.astype(F32))
            else:
                r = radii.astype(F32) * radii_scales.astype(F32)
        else:
            r = radii.astype(F32)
        kx = r * np.cos(angles)
        ky = r * np.sin(angles)
    k = np.stack([kx, ky], axis=-1)
    return k.reshape(B, H, S * L, head_dim).astype(F16)


def dequantize_block(codes: np.ndarray, scales: np.ndarray, group_size: int = 32) -> np.ndarray:
    """``GroupedVQuantizer.dequantize_block`` (v_quant/encoder.py:32-38): f16(f32(code)*f32(scale))."""
    B, H, S, L, D = codes.shape
    c = codes.reshape(B, H, S, L, D // group_size, group_size).astype(F32)
    s = scales[..., None].astype(F32)
    return (c * s).reshape(B, H, S, L, D).astype(F16)


# --------------------------------------------------------------------------
# attention -- kernels/turbo_polar/metal.py:254-332
# --------------------------------------------------------------------------

def softmax_attention(q, k, v, scale, actual_seq_len=None, dtype=F64, score_bias=None):
    """Masked softmax attention, GQA broadcast by ``repeat`` (metal.py:259,307-308).

    q ``[B,Hq,D]``; k, v ``[B,Hkv,T,D]``.  Tokens ``t >= actual_seq_len`` are
    masked (metal.py:278-279,318-319).  ``score_bias`` ``[B,Hq,T]`` is added to
    the scaled scores before the mask (the QJL correction, metal.py:273-275,310-316).
    """
    B, Hq, D = q.shape
    Hkv = k.shape[1]
    g = Hq // Hkv
    T = k.shape[2]
    # Query head h reads kv head h // g: the mx.repeat(axis=1) broadcast,
    # evaluated per kv head without materialising the repeated K/V.
    qg = q.astype(dtype).reshape(B, Hkv, g, D)
    kk = k.astype(dtype)
    vv = v.astype(dtype)
    with np.errstate(invalid="ignore", over="ignore"):
        s = np.matmul(qg, np.swapaxes(kk, -1, -2)) * dtype(scale)  # [B, Hkv, g, T]
        if score_bias is not None:
            s = s + score_bias.astype(dtype).reshape(s.shape)
        if actual_seq_len is not None and actual_seq_len < T:
            s[..., actual_seq_len:] = -np.inf
        m = np.max(s, axis=-1, keepdims=True)
        e = np.exp(s - m)
        w = e / np.sum(e, axis=-1, keepdims=True)
        return np.matmul(w, vv).reshape(B, Hq, D)


def _block_fields(block):
    return (
        block["radii"],
        block.get("radii_scales"),
        block["angle_codes_l1"],
        block["angle_codes_deep"],
        block["metadata"],
    )


def cpu_fused_qk(q, block, scale, dtype=F64):
    """``MetalKernelBridge._cpu_fused_qk`` (metal.py:254-260): scores over all S*64 slots."""
    k = decode_block(*_block_fields(block))
    B, Hq, D = q.shape
    Hkv = k.shape[1]
    qg = q.astype(dtype).reshape(B, Hkv, Hq // Hkv, D)
    with np.errstate(invalid="ignore", over="ignore"):
        s = np.matmul(qg, np.swapaxes(k.astype(dtype), -1, -2)) * dtype(scale)
        return s.reshape(B, Hq, -1)


def cpu_online_attention(q, block, quant_v, scale, actual_seq_len, dtype=F64):
    """``_cpu_online_attention`` with quantised V (metal.py:267-291, caller :661-667)."""
    codes, scales = quant_v
    k = decode_block(*_block_fields(block))
    v = dequantize_block(codes, scales)
    B, H, S, L, D = codes.shape
    return softmax_attention(q, k, v.reshape(B, H, S * L, D), scale, actual_seq_len, dtype)


def cpu_online_attention_dense_v(q, block, v_dense, scale, actual_seq_len, dtype=F64, qjl=None):
    """``execute_online_attention_dense_v``'s CPU path (metal.py:586-601: V
    reshaped to ``[B, H_kv, S*L, D]`` and repeated over the GQA group, then
    ``_cpu_online_attention``, metal.py:267-291): decoded K, dense fp16 V, the
    QJL correction times ``scale`` on every token when ``qjl`` = (packed
    signs, norms, packed query signs, proj_dim)."""
    k = decode_block(*_block_fields(block))
    B, H, T, D = k.shape
    v = np.asarray(v_dense, np.float16).reshape(B, H, T, D)
    bias = None if qjl is None else qjl_dot_estimate(q, *qjl) * F64(scale)
    return softmax_attention(q, k, v, scale, actual_seq_len, dtype, score_bias=bias)


def cpu_online_attention_dense_tail(q, block, quant_v, tail_k, tail_v, scale, actual_seq_len, dtype=F64,
                                    qjl=None):
    """``_cpu_online_attention_dense_tail`` (metal.py:293-332).  ``qjl`` =
    (packed signs, norms, packed query signs, proj_dim): use_qjl=True, the
    correction times ``scale`` on the page tokens and 0 on the tail
    (metal.py:310-316)."""
    codes, scales = quant_v
    k = decode_block(*_block_fields(block))
    v = dequantize_block(codes, scales)
    B, H, S, L, D = codes.shape
    full_k = np.concatenate([k.astype(dtype), tail_k.astype(dtype)], axis=2)
    full_v = np.concatenate([v.reshape(B, H, S * L, D).astype(dtype), tail_v.astype(dtype)], axis=2)
    bias = None
    if qjl is not None:
        corr = qjl_dot_estimate(q, *qjl) * F64(scale)
        tail = np.zeros((B, q.shape[1], tail_k.shape[2]), F64)
        bias = np.concatenate([corr, tail], axis=2)
    return softmax_attention(q, full_k, full_v, scale, actual_seq_len, dtype, score_bias=bias)


# --------------------------------------------------------------------------
# QJL -- rfsn_v11/quant/qjl/encoder.py:19-44, score_estimate.py:6-54,
# kernels/turbo_polar/metal.py:262-265
# --------------------------------------------------------------------------

def qjl_projection(seed: int = 42, head_dim: int = 128, proj_dim: int = 64) -> np.ndarray:
    """QJLResidualEncoder's W (encoder.py:20-28): float32 standard normals of
    ``np.random.default_rng(seed)``, each column over (its norm + 1e-12)."""
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((head_dim, proj_dim), dtype=np.float32)
    return w / (np.linalg.norm(w, axis=0, keepdims=True) + 1e-12)


def qjl_pack_signs(proj: np.ndarray) -> np.ndarray:
    """``proj >= 0`` packed along the last axis, bit i of byte j the sign of
    element 8j + i (encoder.py:36-39: powers 1, 2, ..., 128 summed)."""
    bits = (proj >= 0).astype(np.uint8)
    shp = bits.shape[:-1] + (bits.shape[-1] // 8, 8)
    return (bits.reshape(shp) * (1 << np.arange(8, dtype=np.uint16))).sum(axis=-1).astype(np.uint8)


def qjl_residual_sketch(e: np.ndarray, w: np.ndarray):
    """compute_residual_sketch (encoder.py:30-44): packed signs of e @ W
    (projections in float64) and the fp16 residual norms."""
    proj = e.astype(F64) @ w.astype(F64)
    norms = np.sqrt(np.sum(e.astype(F64) ** 2, axis=-1)).astype(F16)
    return qjl_pack_signs(proj), norms


def qjl_dot_estimate(q, packed, norms, q_packed, proj_dim):
    """qjl_dot_estimate (score_estimate.py:6-54) in float64: for query head h
    and token t of kv head h // g, |E_t| |q_h| sin(pi/2 * match / P), match
    the +-1 sign agreement sum.  packed ``[B,Hkv,S,L,P/8]``, norms
    ``[B,Hkv,S,L]``, q_packed ``[B,Hq,P/8]``; returns ``[B,Hq,S*L]``."""
    B, Hkv, S, L, _ = packed.shape
    Hq = q_packed.shape[1]
    g = Hq // Hkv
    kb = np.unpackbits(packed.reshape(-1, proj_dim // 8), axis=1, bitorder="little")[:, :proj_dim]
    ks = kb.reshape(B, Hkv, S * L, proj_dim).astype(np.int64) * 2 - 1
    qb = np.unpackbits(q_packed.reshape(-1, proj_dim // 8), axis=1, bitorder="little")[:, :proj_dim]
    qs = qb.reshape(B, Hq, proj_dim).astype(np.int64) * 2 - 1
    ks = np.repeat(ks, g, axis=1)
    match = np.einsum("bhp,bhtp->bht", qs, ks)
    q_norm = np.sqrt(np.sum(q.astype(F64) ** 2, axis=-1))
    n = np.repeat(norms.reshape(B, Hkv, S * L).astype(F64), g, axis=1)
    return n * q_norm[:, :, None] * np.sin((np.pi / 2.0) * match / proj_dim)


def cpu_fused_qk_qjl(q, block, qjl, scale, dtype=F64):
    """``_cpu_fused_qk_qjl`` (metal.py:262-265): the fused-QK scores plus the
    QJL estimate times ``scale``; ``qjl`` as for cpu_online_attention_dense_tail."""
    return cpu_fused_qk(q, block, scale, dtype) + qjl_dot_estimate(q, *qjl).astype(dtype) * dtype(scale)
