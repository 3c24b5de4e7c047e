// tp_encode.hip -- page encoder: polar keys + grouped int8 values.
//
// Restates PolarQuantEncoder.encode_block (rfsn_v11/quant/polar/encoder.py:24-98)
// and GroupedVQuantizer.quantize_block (rfsn_v11/quant/v_quant/encoder.py:16-30)
// bit-exactly (see tp_common.h for the fp16 rules).
//
// One 256-thread workgroup encodes one page (64 tokens of one (batch, kv head)).
// Thread (t = tid/4, q = tid%4) owns key pairs [16q, 16q+16) and value group q
// of token t, so each wave reads 16 consecutive 256-byte token rows (fp16).
// Angle codes go through LDS so that any (bits, split_dim) packs into
// dword-wide row stores; int8 log radii need one block-wide max for the
// per-page scale (encoder.py:38-41).
#include "tp_common.h"

namespace tp {

struct EncodeArgs {
  const void* k;
  const void* v;
  int64_t in_tokens;
  int64_t token_begin;
  int64_t n_tokens;
  int32_t int8_radii;
  int32_t l1_bits;
  int32_t deep_bits;
  int32_t split_half;
  int32_t l1_row;
  int32_t deep_row;
  void* radii;
  uint16_t* radii_scales;
  uint8_t* angle_l1;
  uint8_t* angle_deep;
  int8_t* v_codes;
  uint16_t* v_scales;
  int64_t capacity;
  int64_t page_begin;
};

// 32 consecutive input values of one token row: issue the loads (raw) first,
// convert to floats later, so K and V rows are in flight together.  Tokens past
// the end read as zeros (the zero padding of _maybe_encode_partial,
// turbo_polar_cache.py:280-285).
template <bool kF32>
struct RawRow32 {
  uint4 w[kF32 ? 8 : 4];
};

template <bool kF32>
__device__ __forceinline__ void load_row32(const void* base, int64_t off, bool valid, RawRow32<kF32>& r) {
  constexpr int n = kF32 ? 8 : 4;
  const uint4* p = kF32 ? reinterpret_cast<const uint4*>(static_cast<const float*>(base) + off)
                        : reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + off);
#pragma unroll
  for (int i = 0; i < n; ++i) r.w[i] = valid ? p[i] : make_uint4(0u, 0u, 0u, 0u);
}

// Element i of a raw row, and pair j = elements (2j, 2j+1); for fp16 input a
// pair is exactly one dword.
template <bool kF32>
__device__ __forceinline__ uint32_t raw_word(const RawRow32<kF32>& r, int i) {
  const uint4 w = r.w[i >> 2];
  return (i & 3) == 0 ? w.x : (i & 3) == 1 ? w.y : (i & 3) == 2 ? w.z : w.w;
}
template <bool kF32>
__device__ __forceinline__ float raw_val(const RawRow32<kF32>& r, int i) {
  if constexpr (kF32) return __uint_as_float(raw_word(r, i));
  const uint32_t w = raw_word(r, i >> 1);
  return h2f((uint16_t)((i & 1) ? (w >> 16) : (w & 0xffffu)));
}

// Packs the codes of pairs [pair0, pair0 + npairs) of all 64 tokens into rows
// of `row_bytes` bytes (low bits first, zero padded: encoder.py:101-130).
__device__ __forceinline__ void pack_rows(uint8_t* dst, int row_bytes, int bits, int pair0,
                                          int npairs, const uint8_t* codes, int tid) {
  const int words = (kPageTokens * row_bytes) >> 2;
  for (int w = tid; w < words; w += 256) {
    uint32_t word = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int idx = 4 * w + b;
      const int tt = idx / row_bytes;
      const int bb = idx - tt * row_bytes;
      const uint8_t* cr = codes + tt * kPairs + pair0;
      uint32_t byte = 0;
      if (bits == 8) {
        byte = bb < npairs ? cr[bb] : 0u;
      } else if (bits == 4) {
        const int i0 = 2 * bb;
        byte = (i0 < npairs ? cr[i0] : 0u) | ((i0 + 1 < npairs ? cr[i0 + 1] : 0u) << 4);
      } else {
        const int i0 = 4 * bb;
#pragma unroll
        for (int s = 0; s < 4; ++s) byte |= (i0 + s < npairs ? cr[i0 + s] : 0u) << (2 * s);
      }
      word |= byte << (8 * b);
    }
    reinterpret_cast<uint32_t*>(dst)[w] = word;
  }
}

// The page's max |lr| over the workgroup's 256 threads (16 fp16 values
// each) as the reference's reduction takes it: NaN propagates (a NaN log
// radius makes the maximum NaN, and with it the page scale and every radius
// code).  An integer maximum of the |lr| fp16 bit patterns orders finite
// values and inf as fmaxf does and puts every NaN above inf.  s_max: 4 words
// of LDS.
__device__ __forceinline__ float page_abs_max(const uint16_t (&lr)[16], uint32_t* s_max, int tid) {
  uint32_t m = 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) m = max(m, (uint32_t)(lr[j] & 0x7fffu));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off, 64));
  if ((tid & 63) == 0) s_max[tid >> 6] = m;
  __syncthreads();
  return h2f((uint16_t)max(max(s_max[0], s_max[1]), max(s_max[2], s_max[3])));
}

template <bool kF32>
__global__ __launch_bounds__(256) void encode_pages_kernel(EncodeArgs a) {
  __shared__ uint8_t s_codes[kPageTokens * kPairs];
  __shared__ uint32_t s_max[4];

  const int page = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int tid = threadIdx.x;
  const int t = tid >> 2;
  const int qq = tid & 3;
  const int64_t local_tok = (int64_t)page * kPageTokens + t;
  const bool valid = local_tok < a.n_tokens;
  const int64_t in_off = (bh * a.in_tokens + a.token_begin + local_tok) * kHeadDim + 32 * qq;
  const int64_t slot = bh * a.capacity + a.page_begin + page;
  const int64_t row = slot * kPageTokens + t;

  RawRow32<kF32> kraw, vraw;
  if (a.k) load_row32<kF32>(a.k, in_off, valid, kraw);

  if (a.k) {
    uint16_t r16[16];
    // Angles whose fast fp32 atan2 lands too close to an fp16 rounding
    // boundary are flagged here and recomputed in float64 after the loop, so
    // the float64 path is one loop body instead of 16 unrolled copies.
    uint32_t afix = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float x = raw_val(kraw, 2 * j);
      const float y = raw_val(kraw, 2 * j + 1);
      const int p = 16 * qq + j;
      const int bits = p < a.split_half ? a.l1_bits : a.deep_bits;
      uint32_t code;
      if constexpr (kF32) {
        r16[j] = radius_f32_in(x, y);
        code = angle_code_f32((float)atan2((double)y, (double)x), bits);
      } else {
        r16[j] = radius_f16_in(x, y);
        bool exact;
        const uint16_t a16 = atan2_f16_fast(y, x, &exact);
        afix |= exact ? 0u : (1u << j);
        code = angle_code_f16(a16, bits);
      }
      s_codes[t * kPairs + p] = (uint8_t)code;
    }
    if constexpr (!kF32) {
      const uint16_t* pin = static_cast<const uint16_t*>(a.k) + in_off;
      while (afix) {
        const int j = __builtin_ctz(afix);
        afix &= afix - 1u;
        const uint32_t xy = *reinterpret_cast<const uint32_t*>(pin + 2 * j);  // flagged pairs are never padding
        const int p = 16 * qq + j;
        const int bits = p < a.split_half ? a.l1_bits : a.deep_bits;
        s_codes[t * kPairs + p] =
            (uint8_t)angle_code_f16(atan2_f16_slow(h2f((uint16_t)(xy >> 16)), h2f((uint16_t)(xy & 0xffffu))), bits);
      }
    }

    if (a.int8_radii) {
      // encoder.py:34-42: lr = f32(f16 log(max(r, fp16(1e-6)))); per-page scale
      // f16(max|lr| / 127); codes rint(lr / scale).  Flagged logs are redone in
      // float64 by one loop body that selects its element into place.
      uint16_t lr[16];  // fp16 log radii
      uint32_t lfix = 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint16_t rb = r16[j] > kF16RadiusFloor ? r16[j] : kF16RadiusFloor;
        bool exact;
        lr[j] = log_f16_fast(h2f(rb), &exact);
        lfix |= exact ? 0u : (1u << j);
      }
      while (lfix) {
        const int j = __builtin_ctz(lfix);
        lfix &= lfix - 1u;
        uint16_t rb = 0;
#pragma unroll
        for (int k2 = 0; k2 < 16; ++k2) rb = k2 == j ? r16[k2] : rb;
        rb = rb > kF16RadiusFloor ? rb : kF16RadiusFloor;
        const uint16_t exact_lr = log_f16_slow(h2f(rb));
#pragma unroll
        for (int k2 = 0; k2 < 16; ++k2) lr[k2] = k2 == j ? exact_lr : lr[k2];
      }
      const float mx = page_abs_max(lr, s_max, tid);
      const float ls = mx == 0.0f ? 1e-6f : mx;
      const uint16_t ls16 = f2h(ls / 127.0f);
      const float lsf = h2f(ls16);
      uint32_t packed[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t c = (uint32_t)(to_int8_rne(h2f(lr[j]) / lsf) & 0xff);
        packed[j >> 2] |= c << (8 * (j & 3));
      }
      *reinterpret_cast<uint4*>(static_cast<int8_t*>(a.radii) + row * kPairs + 16 * qq) =
          make_uint4(packed[0], packed[1], packed[2], packed[3]);
      if (tid == 0) a.radii_scales[slot] = ls16;
    } else {
      uint32_t w[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) w[i] = (uint32_t)r16[2 * i] | ((uint32_t)r16[2 * i + 1] << 16);
      uint4* dst = reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.radii) + row * kPairs + 16 * qq);
      dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
      dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
    }
    __syncthreads();
    if (a.l1_row > 0)
      pack_rows(a.angle_l1 + slot * kPageTokens * a.l1_row, a.l1_row, a.l1_bits, 0, a.split_half,
                s_codes, tid);
    if (a.deep_row > 0)
      pack_rows(a.angle_deep + slot * kPageTokens * a.deep_row, a.deep_row, a.deep_bits,
                a.split_half, kPairs - a.split_half, s_codes, tid);
  }

  if (a.v) {
    load_row32<kF32>(a.v, in_off, valid, vraw);
    // v_quant/encoder.py:21-25: s = f16(max|v| / 127) (1e-4 if zero),
    // code = int8(clip(rint(v / s))) with an fp16 quotient for fp16 inputs.
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) m = max_abs_nan(m, raw_val(vraw, i));
    uint16_t s16 = f2h(m / 127.0f);
    if ((s16 & 0x7fffu) == 0) s16 = kF16VScaleFloor;
    const float s = h2f(s16);
    const float rs = __builtin_amdgcn_rcpf(s);
    uint32_t packed[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      float qv;
      if constexpr (kF32) {
        qv = raw_val(vraw, i) / s;
      } else {
        qv = div_f16(raw_val(vraw, i), s, rs);
      }
      packed[i >> 2] |= (uint32_t)(to_int8_rne(qv) & 0xff) << (8 * (i & 3));
    }
    uint4* dst = reinterpret_cast<uint4*>(a.v_codes + row * kHeadDim + 32 * qq);
    dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
    a.v_scales[row * kVGroups + qq] = s16;
  }
}

// ---- fp16 fast path for the runtime's two layouts ----------------------------
//
// encode_pages_kernel serves every layout and input type.  fp16 input in the
// default layout (4-bit l1 and deep angles, split_dim 64, fp16 radii) or the
// fast layout (8-bit deep angles, split_dim 0, int8 log radii) takes this
// kernel instead: the code widths and the pair -> row mapping are compile-time
// constants, each thread packs its 16 codes in registers and stores them
// directly (thread q of a token owns pairs [16q, 16q+16), which are bytes
// [8q, 8q+8) of the token's l1 / deep rows in the default layout and bytes
// [16q, 16q+16) of its deep row in the fast layout), and the byte conversion
// v_cvt_pk_u8_f32 rounds half to even, saturates and places the byte in one
// instruction.  Every fp32 step whose fp16 rounding is in doubt only sets a
// per-lane flag; flagged pairs and value groups are redone exactly after the
// main loop, so the output is bit-identical to encode_pages_kernel's.

constexpr int kEncDefault = 0;
constexpr int kEncFast = 1;

// x (an fp32 value holding an fp16 number) times s in fp32, rounded once: an
// explicit FMA with a +0 addend, which the backend takes as one mixed-precision
// FMA (v_fma_mix_f32) reading the fp16 operand directly.  A -0 product reads
// as +0; the callers only test the result's distance from fp16 rounding
// midpoints, which the sign of zero does not change.
__device__ __forceinline__ float mul_f16_f32(float x, float s) { return __builtin_fmaf(x, s, 0.0f); }

// fp16 (a16 + pi) as fp32, the numerator of the angle code (encoder.py:46-50).
__device__ __forceinline__ float code_numerator(uint16_t a16) { return h2f(f2h(h2f(a16) + h2f(kF16Pi))); }

// Argument of the code's byte conversion from the fp16 quotient n16 of a
// fast-path angle: n16 * (2^bits - 1), one mixed-precision FMA reading the
// fp16 value.  No clamp: a non-NaN atan2 lies in [-pi, pi], whose fp16
// rounding lies in [-fp16(pi), fp16(pi)] (pi is below the midpoint between
// fp16(pi) and the next fp16 value), so the shifted angle lies in [0,
// fp16(2 pi)] and its quotient in [0, 1]; the NaN cases are flagged and
// redone on the exact path.
template <int kBits>
__device__ __forceinline__ float code_arg(float n16) {
  return __builtin_fmaf(n16, (float)((1 << kBits) - 1), 0.0f);
}

// The fast path's angle code of pair (x, y), as the argument of the byte
// conversion, and whether it cannot be trusted: the fp32 atan2 lies near an
// fp16 rounding midpoint or is NaN (a NaN x or y, whose code is the NaN
// angle's 0, or two infinite components, an odd multiple of pi/4; atan2_poly
// propagates both as NaN).  An angle below 2^-14
// leaves fp16(a + pi) = fp16(pi) whichever way it rounds, so the guard needs
// no subnormal test, and atan2(+-0, x >= 0) = +-0 comes out of atan2_poly
// exactly.  The quotient needs no guard: for every fp16 numerator s1 the fp32
// product s1 * fp32(1 / fp16(2 pi)), rounded once, rounds to the same fp16 as
// the fp16 division s1 / fp16(2 pi) (checked over all 65536 fp16 values by
// tests/test_oracle_pins.py and, through this function, by
// atan2_exhaustive_kernel).
// xy: the pair's raw fp16 word (y in the high half), whose top bit is the
// sign of y that the angle takes (one bit-field insert).
template <int kBits>
__device__ __forceinline__ float angle_arg_fast(float x, float y, uint32_t xy, bool* flag) {
  const float a = __uint_as_float((__float_as_uint(atan2_poly_mag(y, x)) & 0x7fffffffu) | (xy & 0x80000000u));
  const float q = mul_f16_f32(code_numerator(f2h(a)), kF32InvF16TwoPi);
  *flag = near_f16_midpoint_code<kGuardAtan2>(a) | __builtin_isnan(a);
  return code_arg<kBits>(h2f(f2h(q)));
}

// Exact angle code of pair (x, y): correctly rounded fp16 atan2, except that
// the float64 atan2 runs only when the two fp16 candidates around the fast
// result's rounding midpoint give different codes.  A NaN x or y gives the
// NaN angle's code, 0 (angle_code_f16); two infinite components take the
// float64 atan2.
template <int kBits>
__device__ __forceinline__ uint32_t exact_angle_code(float y, float x) {
  if (__builtin_isunordered(x, y)) return 0u;
  const float a = atan2_poly(y, x);
  if (__builtin_isnan(a)) return angle_code_f16(atan2_f16_slow(y, x), kBits);
  const uint16_t a16 = f2h(a);
  const uint32_t c0 = angle_code_f16(a16, kBits);
  if (!near_f16_midpoint_code<kGuardAtan2>(a)) return c0;
  // The fast fp32 angle lies within kGuardAtan2 ulps of the midpoint between
  // a16 and the neighbour on its side; the correctly rounded value is one of
  // the two.
  const float d = a - h2f(a16);
  const uint16_t nb = (uint16_t)(a16 + ((d > 0.0f) == !(a16 & 0x8000u) ? 1 : -1));
  if ((a16 & 0x7fffu) == 0 || angle_code_f16(nb, kBits) != c0) return angle_code_f16(atan2_f16_slow(y, x), kBits);
  return c0;
}

// Biased byte (code + 128) of value v with scale s = 1/rs by the fast path,
// written into byte `sel` of `old`, and whether the fp32 quotient is too close
// to an fp16 midpoint to trust.
// one: 1.0f, which the caller hides from the compiler (an empty asm that
// yields it in an SGPR) so that fp16(q) * 1 + 128 stays one mixed-precision FMA
// reading the fp16 value instead of a conversion and an add; x * 1 is exact,
// so it rounds as the fp32 sum does.
__device__ __forceinline__ uint32_t vcode_fast_byte(float v, float rs, float one, uint32_t sel, uint32_t old,
                                                    bool* near) {
  const float q = mul_f16_f32(v, rs);
  *near = near_f16_midpoint_code<kGuardDiv>(q);
  return __builtin_amdgcn_cvt_pk_u8_f32(__builtin_fmaf(h2f(f2h(q)), one, 128.0f), sel, old);
}
// 1.0f in an SGPR, opaque to the compiler's constant folding.
__device__ __forceinline__ float opaque_one() {
  float one;
  asm volatile("s_mov_b32 %0, 1.0" : "=s"(one));
  return one;
}
// The same byte from the correctly rounded quotient, NaN -> code 0.
__device__ __forceinline__ uint32_t vcode_exact_byte(float v, float s) {
  const float qn = h2f(f2h(v / s));
  return __builtin_amdgcn_cvt_pk_u8_f32((qn == qn ? qn : 0.0f) + 128.0f, 0u, 0u);
}

// Biased byte (code + 128) of the int8 log-radius code rint(lr / ls) of the
// fp16 log radius lr16 by the fast path, rl = 1 / ls by v_rcp_f32, written
// into byte `sel` of `old`, and whether it must be redone.  The fast path
// forms lr * rl + 128 in one FMA: the reciprocal is within 1 ulp, so for
// |lr / ls| < 127.1 (lr is at most the page's max |lr| and ls its fp16 / 127)
// the product is within 2^-16 of the exact quotient and the rounded sum within
// 1.5 * 2^-16 of quotient + 128; rint agrees with the reference's unless the
// sum lies within 2^-13 of a half-integer.  The sum is positive, and the byte
// conversion rounds half to even.
__device__ __forceinline__ uint32_t lcode_fast_byte(uint16_t lr16, float rl, uint32_t sel, uint32_t old,
                                                    bool* near) {
  const float qb = __builtin_fmaf(h2f(lr16), rl, 128.0f);
  // v_fract_f32 is qb - floor(qb) here (0 < qb < 256; it caps just below 1).
  *near = fabsf(__builtin_amdgcn_fractf(qb) - 0.5f) <= 0x1p-13f;
  return __builtin_amdgcn_cvt_pk_u8_f32(qb, sel, old);
}
// The same byte from the correctly rounded fp32 quotient lr / ls (NaN -> code
// 0).  The quotient of two fp16 values is a half-integer exactly or lies at
// least 2^-13 from one, so adding 128 (one rounding at 2^-16) keeps rint's
// answer, and a tie stays a tie whose even neighbour is shifted by 128.
__device__ __forceinline__ uint32_t lcode_exact_byte(uint16_t lr16, float ls) {
  const float qd = h2f(lr16) / ls;
  return __builtin_amdgcn_cvt_pk_u8_f32((qd == qd ? qd : 0.0f) + 128.0f, 0u, 0u);
}

// Per-lane masks of the items the fast path cannot vouch for are built most
// significant first: push_flag shifts the mask up and ORs the new item's flag
// in (a 0/1 select and a shift-or, where a bit of its own per item would need
// a 32-bit constant in a register for every item past the sixth), so item j
// of n sits in bit n - 1 - j.
__device__ __forceinline__ uint32_t push_flag(uint32_t m, bool f) { return (m << 1) | (f ? 1u : 0u); }

template <int L>
__global__ __launch_bounds__(256) void encode_f16_kernel(EncodeArgs a) {
  constexpr bool kFastLayout = L == kEncFast;
  constexpr int kBits = kFastLayout ? 8 : 4;
  __shared__ uint32_t s_max[4];

  const int page = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int tid = threadIdx.x;
  const int t = tid >> 2;
  const int qq = tid & 3;
  const int64_t local_tok = (int64_t)page * kPageTokens + t;
  const bool valid = local_tok < a.n_tokens;
  const int64_t in_off = (bh * a.in_tokens + a.token_begin + local_tok) * kHeadDim + 32 * qq;
  const int64_t slot = bh * a.capacity + a.page_begin + page;
  const int64_t row = slot * kPageTokens + t;

  RawRow32<false> kraw;
  load_row32<false>(a.k, in_off, valid, kraw);
  uint16_t r16[16];
  uint32_t cw[kFastLayout ? 4 : 2];
#pragma unroll
  for (int i = 0; i < (kFastLayout ? 4 : 2); ++i) cw[i] = 0u;
  uint32_t fixa = 0;  // pairs whose angle code the fast path cannot vouch for
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const uint32_t w = raw_word(kraw, j);
    const half2v xy = __builtin_bit_cast(half2v, w);
    const half2v sq = xy * xy;  // fp16 products, as the reference squares in fp16 (no FMA)
    r16[j] = __builtin_bit_cast(uint16_t, __builtin_sqrtf16((f16)(sq[0] + sq[1])));  // correctly rounded
    bool flag;
    const float arg = angle_arg_fast<kBits>((float)xy[0], (float)xy[1], w, &flag);
    fixa = push_flag(fixa, flag);
    if constexpr (kFastLayout) {
      cw[j >> 2] = __builtin_amdgcn_cvt_pk_u8_f32(arg, (uint32_t)(j & 3), cw[j >> 2]);
    } else {
      cw[j >> 3] |= __builtin_amdgcn_cvt_pk_u8_f32(arg, 0u, 0u) << (4 * (j & 7));
    }
  }
  // Exact redo of the flagged codes (padding tokens are never flagged).
  const uint32_t* kin = reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.k) + in_off);
  while (fixa) {  // flagged pairs are never padding: reload the pair
    const int j = 15 - __builtin_ctz(fixa);
    fixa &= fixa - 1u;
    const uint32_t w = kin[j];
    const uint32_t c = exact_angle_code<kBits>(h2f((uint16_t)(w >> 16)), h2f((uint16_t)(w & 0xffffu)));
    if constexpr (kFastLayout) {
      const uint32_t sh = 8u * (uint32_t)(j & 3);
#pragma unroll
      for (int k2 = 0; k2 < 4; ++k2)
        cw[k2] = k2 == (j >> 2) ? (cw[k2] & ~(0xffu << sh)) | (c << sh) : cw[k2];
    } else {
      const uint32_t sh = 4u * (uint32_t)(j & 7);
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2)
        cw[k2] = k2 == (j >> 3) ? (cw[k2] & ~(0xfu << sh)) | (c << sh) : cw[k2];
    }
  }

  if constexpr (kFastLayout) {
    // encoder.py:34-42: lr = f32(f16 log(max(r, fp16(1e-6)))); per-page scale
    // f16(max|lr| / 127); codes rint(lr / scale).
    // The log radii stay fp16 (the reference's f16 log, widened exactly
    // wherever it is used).
    uint16_t lr[16];
    uint32_t lfix = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint16_t rb = r16[j] > kF16RadiusFloor ? r16[j] : kF16RadiusFloor;
      bool exact;
      lr[j] = log_f16_fast(h2f(rb), &exact);
      lfix = push_flag(lfix, !exact);
    }
    while (lfix) {
      const int j = 15 - __builtin_ctz(lfix);
      lfix &= lfix - 1u;
      uint16_t rb = 0;
#pragma unroll
      for (int k2 = 0; k2 < 16; ++k2) rb = k2 == j ? r16[k2] : rb;
      rb = rb > kF16RadiusFloor ? rb : kF16RadiusFloor;
      const uint16_t exact_lr = log_f16_slow(h2f(rb));
#pragma unroll
      for (int k2 = 0; k2 < 16; ++k2) lr[k2] = k2 == j ? exact_lr : lr[k2];
    }
    const float mx = page_abs_max(lr, s_max, tid);
    const float ls = mx == 0.0f ? 1e-6f : mx;
    const uint16_t ls16 = f2h(ls / 127.0f);
    const float lsf = h2f(ls16);
    // code = int8(clip(rint(f32(lr / ls)))) by lcode_fast_byte, the flagged
    // ones redone by lcode_exact_byte.  NaN quotients give code 0, and they
    // come only from a scale that is 0 (every lr is 0: 0 / 0), inf (lr / inf
    // is 0 or NaN) or NaN (a NaN lr): then every code of the page is 0, and
    // otherwise every lr is finite.
    const float rl = __builtin_amdgcn_rcpf(lsf);
    const bool zero_codes = !(lsf != 0.0f && fabsf(lsf) < INFINITY);  // uniform over the page
    uint32_t packed[4] = {0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u};
    uint32_t dfix = 0;
    if (!zero_codes) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        bool near;
        packed[j >> 2] = lcode_fast_byte(lr[j], rl, (uint32_t)(j & 3), packed[j >> 2], &near);
        dfix = push_flag(dfix, near);
      }
    }
    while (dfix) {
      const int j = 15 - __builtin_ctz(dfix);
      dfix &= dfix - 1u;
      uint16_t lj = 0;
#pragma unroll
      for (int k2 = 0; k2 < 16; ++k2) lj = k2 == j ? lr[k2] : lj;
      const uint32_t b = lcode_exact_byte(lj, lsf);
      const uint32_t sh = 8u * (uint32_t)(j & 3);
#pragma unroll
      for (int k2 = 0; k2 < 4; ++k2) packed[k2] = k2 == (j >> 2) ? (packed[k2] & ~(0xffu << sh)) | (b << sh) : packed[k2];
    }
#pragma unroll
    for (int k2 = 0; k2 < 4; ++k2) packed[k2] ^= 0x80808080u;  // biased bytes -> int8
    *reinterpret_cast<uint4*>(static_cast<int8_t*>(a.radii) + row * kPairs + 16 * qq) =
        make_uint4(packed[0], packed[1], packed[2], packed[3]);
    if (tid == 0) a.radii_scales[slot] = ls16;
    *reinterpret_cast<uint4*>(a.angle_deep + row * kPairs + 16 * qq) = make_uint4(cw[0], cw[1], cw[2], cw[3]);
  } else {
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = (uint32_t)r16[2 * i] | ((uint32_t)r16[2 * i + 1] << 16);
    uint4* dst = reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.radii) + row * kPairs + 16 * qq);
    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
    uint8_t* crow = (qq < 2 ? a.angle_l1 : a.angle_deep) + row * 16 + 8 * (qq & 1);
    *reinterpret_cast<uint2*>(crow) = make_uint2(cw[0], cw[1]);
  }

  // Values (v_quant/encoder.py:21-25): s = f16(max|v| / 127) (1e-4 if zero),
  // code = int8(clip(rint(f16(v / s)), -128, 127)).  The group maximum is an
  // integer maximum of the |v| bit patterns, which orders finite fp16 values
  // and inf like fmaxf and puts every NaN above inf: a NaN makes the maximum
  // NaN (nan_max, tp_common.h), so the scale is NaN and every code 0.
  RawRow32<false> vraw;
  load_row32<false>(a.v, in_off, valid, vraw);
  // Both halves of each word at once (v_pk_max_u16), then the two halves.
  u16x2 m2 = {0, 0};
#pragma unroll
  for (int i = 0; i < 16; ++i)
    m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, raw_word(vraw, i) & 0x7fff7fffu));
  const uint32_t mbits = max((uint32_t)m2[0], (uint32_t)m2[1]);
  // inf or NaN in the group: exact path (v / inf and NaN quotients give code 0).
  const bool nonfinite = mbits >= 0x7c00u;
  uint16_t s16 = f2h(h2f((uint16_t)mbits) / 127.0f);
  if ((s16 & 0x7fffu) == 0) s16 = kF16VScaleFloor;
  const float s = h2f(s16);
  const float rs = __builtin_amdgcn_rcpf(s);
  const float one = opaque_one();
  uint32_t vw[8];
  uint32_t vfix = 0;  // values whose quotient the fast path cannot vouch for (value i in bit 31 - i)
#pragma unroll
  for (int i = 0; i < 8; ++i) vw[i] = 0u;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    bool near;
    vw[i >> 2] = vcode_fast_byte(raw_val(vraw, i), rs, one, (uint32_t)(i & 3), vw[i >> 2], &near);
    vfix = push_flag(vfix, near);
  }
  if (nonfinite) vfix = 0xffffffffu;  // inf or NaN in the group: every value on the exact path
  const uint16_t* vin = static_cast<const uint16_t*>(a.v) + in_off;
  while (vfix) {  // exact quotients of the flagged values, reloaded (never padding)
    const int i = 31 - __builtin_ctz(vfix);
    vfix &= vfix - 1u;
    const uint32_t b = vcode_exact_byte(h2f(vin[i]), s);
    const uint32_t sh = 8u * (uint32_t)(i & 3);
#pragma unroll
    for (int k2 = 0; k2 < 8; ++k2) vw[k2] = k2 == (i >> 2) ? (vw[k2] & ~(0xffu << sh)) | (b << sh) : vw[k2];
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) vw[i] ^= 0x80808080u;  // biased bytes -> int8
  uint4* vdst = reinterpret_cast<uint4*>(a.v_codes + row * kHeadDim + 32 * qq);
  vdst[0] = make_uint4(vw[0], vw[1], vw[2], vw[3]);
  vdst[1] = make_uint4(vw[4], vw[5], vw[6], vw[7]);
  a.v_scales[row * kVGroups + qq] = s16;
}

// ---- codec entry points for shapes outside the page encoder ----------------------
//
// GroupedVQuantizer.quantize_block for any group size dividing the row and any
// row length, and the int8 log radii of an L-token block with one scale per
// (b, h) row (PolarQuantEncoder.encode_block with use_int8_radii and L != 64).
// Off the decode path: plain, exact per-element arithmetic, no fast paths.

// One thread per group of `group` values of a row of `dim` (v_quant/encoder.py:
// 16-30): s = f16(max|v| / 127) (fp16(1e-4) if zero), code = int8(clip(rint(v
// / s))), the quotient rounded to fp16 first for fp16 input.  A NaN in the
// group makes the maximum NaN (nan_max), as in the page encoder.
template <bool F32IN>
__global__ __launch_bounds__(256) void quantize_groups_kernel(const void* v, int64_t n_groups, int32_t group,
                                                              int8_t* codes, uint16_t* scales) {
  const int64_t gi = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gi >= n_groups) return;
  const int64_t base = gi * group;
  auto val = [&](int i) -> float {
    if constexpr (F32IN) return static_cast<const float*>(v)[base + i];
    else return h2f(static_cast<const uint16_t*>(v)[base + i]);
  };
  float m = 0.0f;
  for (int i = 0; i < group; ++i) m = max_abs_nan(m, val(i));
  uint16_t s16 = f2h(m / 127.0f);
  if ((s16 & 0x7fffu) == 0) s16 = kF16VScaleFloor;
  const float s = h2f(s16);
  for (int i = 0; i < group; ++i) {
    const float q = F32IN ? val(i) / s : h2f(f2h(val(i) / s));
    codes[base + i] = (int8_t)to_int8_rne(q);
  }
  scales[gi] = s16;
}

// One workgroup per (b, h) row of n fp16 radii (encoder.py:34-42): lr =
// f32(f16 log(max(r, fp16(1e-6)))), scale = f16(max|lr| / 127) (max 0 ->
// 1e-6), code = int8(clip(rint(lr / scale))).  A NaN log radius makes the
// maximum NaN (nan_max), as in the page encoder.
__global__ __launch_bounds__(256) void log_radii_rows_kernel(const uint16_t* radii, int64_t n, int8_t* codes,
                                                             uint16_t* scales) {
  __shared__ float s_max[256];
  const int64_t row = blockIdx.x;
  const uint16_t* r = radii + row * n;
  auto log_r = [&](int64_t i) -> float {
    const uint16_t rb = r[i] > kF16RadiusFloor ? r[i] : kF16RadiusFloor;
    return h2f(log_f16(h2f(rb)));
  };
  float m = 0.0f;
  for (int64_t i = threadIdx.x; i < n; i += 256) m = max_abs_nan(m, log_r(i));
  s_max[threadIdx.x] = m;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) s_max[threadIdx.x] = nan_max(s_max[threadIdx.x], s_max[threadIdx.x + w]);
    __syncthreads();
  }
  const float mx = s_max[0];
  const uint16_t ls16 = f2h((mx == 0.0f ? 1e-6f : mx) / 127.0f);
  const float ls = h2f(ls16);
  for (int64_t i = threadIdx.x; i < n; i += 256) codes[row * n + i] = (int8_t)to_int8_rne(log_r(i) / ls);
  if (threadIdx.x == 0) scales[row] = ls16;
}

// ---- self-test kernels -------------------------------------------------------

__global__ __launch_bounds__(256) void f16_tables_kernel(uint16_t* sqrt_out, uint16_t* log_out,
                                                         uint8_t* codes_out) {
  const uint32_t b = blockIdx.x * 256u + threadIdx.x;
  const uint16_t hb = (uint16_t)b;
  sqrt_out[b] = sqrt_f16(h2f(hb));
  const uint16_t rb = (hb < 0x8000u && hb < kF16RadiusFloor) ? kF16RadiusFloor : hb;
  log_out[b] = log_f16(h2f(rb));
  codes_out[3 * b + 0] = (uint8_t)angle_code_f16(hb, 2);
  codes_out[3 * b + 1] = (uint8_t)angle_code_f16(hb, 4);
  codes_out[3 * b + 2] = (uint8_t)angle_code_f16(hb, 8);
}

__global__ __launch_bounds__(256) void atan2_exhaustive_kernel(unsigned long long* mismatches,
                                                               int32_t x_begin) {
  const uint32_t xb = (uint32_t)(x_begin + (int32_t)blockIdx.y) & 0xffffu;
  const uint32_t yb = blockIdx.x * 256u + threadIdx.x;
  uint32_t bad = 0;
  if ((xb & 0x7c00u) != 0x7c00u && (yb & 0x7c00u) != 0x7c00u) {
    const float x = h2f((uint16_t)xb);
    const float y = h2f((uint16_t)yb);
    const uint16_t fast = atan2_f16(y, x);
    const uint16_t ref = d2h(atan2((double)y, (double)x));
    bad = fast != ref ? 1u : 0u;
    // The specialised encoder's codes: the fast path where it vouches for its
    // result, else exact_angle_code (which skips the float64 atan2 when both
    // fp16 candidates give one code).
    bool f4, f8;
    const float g4 = angle_arg_fast<4>(x, y, (yb << 16) | xb, &f4);
    const float g8 = angle_arg_fast<8>(x, y, (yb << 16) | xb, &f8);
    const uint32_t c4 = f4 ? exact_angle_code<4>(y, x) : __builtin_amdgcn_cvt_pk_u8_f32(g4, 0u, 0u);
    const uint32_t c8 = f8 ? exact_angle_code<8>(y, x) : __builtin_amdgcn_cvt_pk_u8_f32(g8, 0u, 0u);
    bad |= c4 != angle_code_f16(ref, 4) ? 1u : 0u;
    bad |= c8 != angle_code_f16(ref, 8) ? 1u : 0u;
  }
  const unsigned long long ballot = __ballot(bad);
  if ((threadIdx.x & 63) == 0 && ballot) atomicAdd(mismatches, (unsigned long long)__popcll(ballot));
}

__global__ __launch_bounds__(256) void div_exhaustive_kernel(unsigned long long* mismatches, int32_t s_begin) {
  const uint32_t sb = (uint32_t)(s_begin + (int32_t)blockIdx.y) & 0x7fffu;
  const uint32_t vb = blockIdx.x * 256u + threadIdx.x;
  uint32_t bad = 0;
  if (sb != 0 && (sb & 0x7c00u) != 0x7c00u && (vb & 0x7c00u) != 0x7c00u) {
    const float s = h2f((uint16_t)sb);
    const float v = h2f((uint16_t)vb);
    const uint16_t fast = f2h(div_f16(v, s, __builtin_amdgcn_rcpf(s)));
    const uint16_t ref = f2h(v / s);
    bad = fast != ref ? 1u : 0u;
  }
  const unsigned long long ballot = __ballot(bad);
  if ((threadIdx.x & 63) == 0 && ballot) atomicAdd(mismatches, (unsigned long long)__popcll(ballot));
}

// Every finite value v against one positive finite scale per blockIdx.y: the
// fast V code byte (with its exact fallback) against the exact one.
__global__ __launch_bounds__(256) void vcode_exhaustive_kernel(unsigned long long* mismatches, int32_t s_begin) {
  const uint32_t sb = (uint32_t)(s_begin + (int32_t)blockIdx.y) & 0x7fffu;
  const uint32_t vb = blockIdx.x * 256u + threadIdx.x;
  uint32_t bad = 0;
  if (sb != 0 && (sb & 0x7c00u) != 0x7c00u && (vb & 0x7c00u) != 0x7c00u) {
    const float s = h2f((uint16_t)sb);
    const float v = h2f((uint16_t)vb);
    bool near;
    uint32_t fast = vcode_fast_byte(v, __builtin_amdgcn_rcpf(s), opaque_one(), 0u, 0u, &near);
    if (near) fast = vcode_exact_byte(v, s);
    const int32_t ref = to_int8_rne(h2f(f2h(v / s)));
    bad = (int32_t)(int8_t)(uint8_t)(fast ^ 0x80u) != ref ? 1u : 0u;
  }
  const unsigned long long ballot = __ballot(bad);
  if ((threadIdx.x & 63) == 0 && ballot) atomicAdd(mismatches, (unsigned long long)__popcll(ballot));
}

// Every finite fp16 log radius lr against one positive finite fp16 scale ls
// per blockIdx.y, over the quotients the encoder forms (|lr / ls| < 127.1):
// the fast log-radius code byte (with its exact fallback) against
// int8(clip(rint(f32(lr / ls)), -128, 127)).
__global__ __launch_bounds__(256) void lcode_exhaustive_kernel(unsigned long long* mismatches, int32_t s_begin) {
  const uint32_t sb = (uint32_t)(s_begin + (int32_t)blockIdx.y) & 0x7fffu;
  const uint32_t lb = blockIdx.x * 256u + threadIdx.x;
  uint32_t bad = 0;
  if (sb != 0 && (sb & 0x7c00u) != 0x7c00u && (lb & 0x7c00u) != 0x7c00u) {
    const float ls = h2f((uint16_t)sb);
    const float lr = h2f((uint16_t)lb);
    if (fabsf(lr) < 127.1f * ls) {
      bool near;
      uint32_t fast = lcode_fast_byte((uint16_t)lb, __builtin_amdgcn_rcpf(ls), 0u, 0u, &near);
      if (near) fast = lcode_exact_byte((uint16_t)lb, ls);
      const int32_t ref = to_int8_rne(lr / ls);
      bad = (int32_t)(int8_t)(uint8_t)(fast ^ 0x80u) != ref ? 1u : 0u;
    }
  }
  const unsigned long long ballot = __ballot(bad);
  if ((threadIdx.x & 63) == 0 && ballot) atomicAdd(mismatches, (unsigned long long)__popcll(ballot));
}

}  // namespace tp

using namespace tp;

extern "C" {

int32_t tp_encode_pages(const void* k, const void* v, int32_t in_dtype, int64_t bh,
                        int64_t in_tokens, int64_t token_begin, int64_t n_tokens,
                        const tp_page_layout* layout, const tp_pages* pages, int64_t page_begin,
                        void* stream) {
  clear_error();
  int l1_row = 0, deep_row = 0;
  if (!check_layout(layout, &l1_row, &deep_row)) return TP_ERR_UNSUPPORTED;
  if (!pages) {
    set_error("pages is NULL");
    return TP_ERR_INVALID;
  }
  if (in_dtype != 0 && in_dtype != 1) {
    set_error("in_dtype must be 0 (float16) or 1 (float32), got %d", in_dtype);
    return TP_ERR_INVALID;
  }
  if (!k && !v) {
    set_error("k and v are both NULL");
    return TP_ERR_INVALID;
  }
  if (n_tokens == 0) return TP_OK;
  if (bh < 1 || bh > 65535 || n_tokens < 0 || token_begin < 0 || in_tokens < 0 ||
      token_begin + n_tokens > in_tokens) {
    set_error("bad token range: bh=%lld in_tokens=%lld token_begin=%lld n_tokens=%lld",
              (long long)bh, (long long)in_tokens, (long long)token_begin, (long long)n_tokens);
    return TP_ERR_INVALID;
  }
  const int64_t n_pages = (n_tokens + kPageTokens - 1) / kPageTokens;
  if (page_begin < 0 || page_begin + n_pages > pages->capacity || n_pages > 0x7fffffff) {
    set_error("page slots [%lld, %lld) exceed capacity %lld", (long long)page_begin,
              (long long)(page_begin + n_pages), (long long)pages->capacity);
    return TP_ERR_INVALID;
  }
  if (k) {
    if (!pages->radii || (l1_row > 0 && !pages->angle_l1) || (deep_row > 0 && !pages->angle_deep) ||
        (layout->int8_radii && !pages->radii_scales)) {
      set_error("key page buffers missing for this layout");
      return TP_ERR_INVALID;
    }
    if (((uintptr_t)k & 15u) || ((uintptr_t)pages->radii & 15u) ||
        ((uintptr_t)pages->angle_l1 & 3u) || ((uintptr_t)pages->angle_deep & 3u)) {
      set_error("k / key page buffers are not 16-byte aligned");
      return TP_ERR_INVALID;
    }
  }
  if (v) {
    if (!pages->v_codes || !pages->v_scales) {
      set_error("value page buffers missing");
      return TP_ERR_INVALID;
    }
    if (((uintptr_t)v & 15u) || ((uintptr_t)pages->v_codes & 15u) ||
        ((uintptr_t)pages->v_scales & 1u)) {
      set_error("v / value page buffers are not aligned");
      return TP_ERR_INVALID;
    }
  }
  EncodeArgs a;
  a.k = k;
  a.v = v;
  a.in_tokens = in_tokens;
  a.token_begin = token_begin;
  a.n_tokens = n_tokens;
  a.int8_radii = layout->int8_radii;
  a.l1_bits = layout->l1_bits;
  a.deep_bits = layout->deep_bits;
  a.split_half = layout->split_dim / 2;
  a.l1_row = l1_row;
  a.deep_row = deep_row;
  a.radii = pages->radii;
  a.radii_scales = static_cast<uint16_t*>(pages->radii_scales);
  a.angle_l1 = pages->angle_l1;
  a.angle_deep = pages->angle_deep;
  a.v_codes = pages->v_codes;
  a.v_scales = static_cast<uint16_t*>(pages->v_scales);
  a.capacity = pages->capacity;
  a.page_begin = page_begin;
  const dim3 grid((unsigned)n_pages, (unsigned)bh);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // fp16 K and V in the runtime's two layouts take the specialised kernel.
  const bool is_default = !layout->int8_radii && layout->l1_bits == 4 && layout->deep_bits == 4 &&
                          layout->split_dim == 64 && !(((uintptr_t)pages->angle_l1 | (uintptr_t)pages->angle_deep) & 7u);
  const bool is_fast = layout->int8_radii && layout->deep_bits == 8 && layout->split_dim == 0 &&
                       !((uintptr_t)pages->angle_deep & 15u);
  if (in_dtype == 0 && k && v && is_default)
    hipLaunchKernelGGL(encode_f16_kernel<kEncDefault>, grid, dim3(256), 0, s, a);
  else if (in_dtype == 0 && k && v && is_fast)
    hipLaunchKernelGGL(encode_f16_kernel<kEncFast>, grid, dim3(256), 0, s, a);
  else if (in_dtype == 1)
    hipLaunchKernelGGL(encode_pages_kernel<true>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(encode_pages_kernel<false>, grid, dim3(256), 0, s, a);
  return launch_status("tp_encode_pages");
}

int32_t tp_selftest_f16_tables(uint16_t* sqrt_out, uint16_t* log_out, uint8_t* codes_out,
                               void* stream) {
  clear_error();
  if (!sqrt_out || !log_out || !codes_out) {
    set_error("output buffers must not be NULL");
    return TP_ERR_INVALID;
  }
  hipLaunchKernelGGL(f16_tables_kernel, dim3(256), dim3(256), 0, static_cast<hipStream_t>(stream),
                     sqrt_out, log_out, codes_out);
  return launch_status("tp_selftest_f16_tables");
}

int32_t tp_selftest_atan2_exhaustive(unsigned long long* mismatches, int32_t x_begin,
                                     int32_t x_count, void* stream) {
  clear_error();
  if (!mismatches || x_begin < 0 || x_count < 1 || x_begin + x_count > 65536 || x_count > 65535) {
    set_error("bad self-test range");
    return TP_ERR_INVALID;
  }
  hipLaunchKernelGGL(atan2_exhaustive_kernel, dim3(256, (unsigned)x_count), dim3(256), 0,
                     static_cast<hipStream_t>(stream), mismatches, x_begin);
  return launch_status("tp_selftest_atan2_exhaustive");
}

int32_t tp_quantize_v_groups(const void* v, int32_t in_dtype, int64_t rows, int32_t dim, int32_t group_size,
                             int8_t* codes, uint16_t* scales, void* stream) {
  clear_error();
  if (in_dtype != 0 && in_dtype != 1) {
    set_error("in_dtype must be 0 (float16) or 1 (float32), got %d", in_dtype);
    return TP_ERR_INVALID;
  }
  if (!v || !codes || !scales || rows < 1 || dim < 1 || group_size < 1 || dim % group_size) {
    set_error("bad arguments: rows=%lld dim=%d group_size=%d (the group size must divide dim)", (long long)rows,
              dim, group_size);
    return TP_ERR_INVALID;
  }
  const int64_t n_groups = rows * (dim / group_size);
  const unsigned blocks = (unsigned)((n_groups + 255) / 256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (in_dtype)
    hipLaunchKernelGGL(quantize_groups_kernel<true>, dim3(blocks), dim3(256), 0, s, v, n_groups, group_size, codes,
                       scales);
  else
    hipLaunchKernelGGL(quantize_groups_kernel<false>, dim3(blocks), dim3(256), 0, s, v, n_groups, group_size, codes,
                       scales);
  return launch_status("tp_quantize_v_groups");
}

int32_t tp_log_radii_rows(const void* radii, int64_t rows, int64_t n, int8_t* codes, uint16_t* scales,
                          void* stream) {
  clear_error();
  if (!radii || !codes || !scales || rows < 1 || rows > INT32_MAX || n < 1) {
    set_error("bad arguments: rows=%lld n=%lld", (long long)rows, (long long)n);
    return TP_ERR_INVALID;
  }
  hipLaunchKernelGGL(log_radii_rows_kernel, dim3((unsigned)rows), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(radii), n, codes, scales);
  return launch_status("tp_log_radii_rows");
}

int32_t tp_selftest_vcode_exhaustive(unsigned long long* mismatches, int32_t s_begin, int32_t s_count,
                                     void* stream) {
  clear_error();
  if (!mismatches || s_begin < 0 || s_count < 1 || s_begin + s_count > 32768 || s_count > 65535) {
    set_error("bad self-test range");
    return TP_ERR_INVALID;
  }
  hipLaunchKernelGGL(vcode_exhaustive_kernel, dim3(256, (unsigned)s_count), dim3(256), 0,
                     static_cast<hipStream_t>(stream), mismatches, s_begin);
  return launch_status("tp_selftest_vcode_exhaustive");
}

int32_t tp_selftest_lcode_exhaustive(unsigned long long* mismatches, int32_t s_begin, int32_t s_count,
                                     void* stream) {
  clear_error();
  if (!mismatches || s_begin < 0 || s_count < 1 || s_begin + s_count > 32768 || s_count > 65535) {
    set_error("bad self-test range");
    return TP_ERR_INVALID;
  }
  hipLaunchKernelGGL(lcode_exhaustive_kernel, dim3(256, (unsigned)s_count), dim3(256), 0,
                     static_cast<hipStream_t>(stream), mismatches, s_begin);
  return launch_status("tp_selftest_lcode_exhaustive");
}

int32_t tp_selftest_div_f16_exhaustive(unsigned long long* mismatches, int32_t s_begin, int32_t s_count,
                                       void* stream) {
  clear_error();
  if (!mismatches || s_begin < 0 || s_count < 1 || s_begin + s_count > 32768) {
    set_error("bad self-test range");
    return TP_ERR_INVALID;
  }
  hipLaunchKernelGGL(div_exhaustive_kernel, dim3(256, (unsigned)s_count), dim3(256), 0,
                     static_cast<hipStream_t>(stream), mismatches, s_begin);
  return launch_status("tp_selftest_div_f16_exhaustive");
}

}  // extern "C"
