// tp_common.h -- shared device helpers of the TurboPolar gfx950 kernels.
//
// Bit-exactness of the encoder rests on these scalar helpers.  They restate
// the fp16 semantics of the reference encoder
// (rfsn_v11/quant/polar/encoder.py:24-98, rfsn_v11/quant/v_quant/encoder.py:16-30):
//   * every fp16 op is correctly rounded: computed in fp32 and rounded once to
//     fp16 (exact for + - * / sqrt because fp32 has >= 2*11+2 significand bits),
//     which requires IEEE fp32 divide/sqrt and no FMA contraction -- the library
//     is compiled with -ffp-contract=off -fhip-fp32-correctly-rounded-divide-sqrt;
//   * round-half-to-even (rintf -> v_rndne_f32);
//   * atan2 and log are correctly rounded to the output type: a fast fp32 path,
//     with a float64 recomputation whenever the fp32 result lies within a few
//     ulps of an fp16 rounding midpoint (checked exhaustively over every pair of
//     fp16 inputs by tp_selftest_atan2_exhaustive).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "turbopolar.h"

namespace tp {

typedef _Float16 f16;
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

constexpr int kPageTokens = 64;
constexpr int kHeadDim = 128;
constexpr int kPairs = 64;
constexpr int kVGroups = 4;
constexpr int kVGroupSize = 32;

// fp16 constants of the reference's weak-scalar arithmetic.
constexpr uint16_t kF16Pi = 0x4248;            // fp16(pi) = 3.140625
constexpr uint16_t kF16TwoPi = 0x4648;         // fp16(2*pi) = 6.28125
constexpr uint16_t kF16RadiusFloor = 0x0011;   // fp16(1e-6)
constexpr uint16_t kF16VScaleFloor = 0x068E;   // fp16(1e-4)
// float32 constants: f32(pi), f32(2*pi), f32(1 - 1e-6)
constexpr float kF32Pi = 3.14159274101257324f;
constexpr float kF32TwoPi = 6.28318548202514648f;
constexpr float kF32OneMinusEps = 0.999998986721038818f;
// fp32(1 / 6.28125), the reciprocal of fp16(2*pi) (0.5 fp32 ulp from exact).
constexpr float kF32InvF16TwoPi = 0.159203976392745972f;

// fp32 ulps around an fp16 rounding midpoint inside which a fast fp32 result
// is not trusted and the exact path decides.  Each guard exceeds the fast
// path's error: a v_rcp_f32 product is within 2 ulps, atan2_poly and logf
// within a few; the atan2, log, quotient and angle-code paths are checked over
// every fp16 input by the self-test kernels.
constexpr int kGuardAtan2 = 6;
constexpr int kGuardLog = 16;
constexpr int kGuardDiv = 3;

__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(f16, b); }
__device__ __forceinline__ uint16_t f2h(float x) { return __builtin_bit_cast(uint16_t, (f16)x); }

// float64 -> fp16, round to nearest even, without double rounding:
// round to fp32 toward zero, make it sticky (round-to-odd), then RNE to fp16.
__device__ __forceinline__ uint16_t d2h(double d) {
  float f = __double2float_rz(d);
  if ((double)f != d) f = __uint_as_float(__float_as_uint(f) | 1u);
  return f2h(f);
}

// True when the fp32 value `v` is within kGuard fp32 ulps of an fp16 rounding
// midpoint, for a value that only feeds the round-half-even of a code: below
// the fp16 normal range (|v| < 2^-14) every code candidate rounds to 0, so no
// subnormal test is needed.  ((u - 0x1000 + kGuard) mod 2^13) <= 2 kGuard is
// |low 13 bits - 0x1000| <= kGuard.
// The low 13 bits are tested in the top of the word: (x << 19) < (2 kGuard +
// 1) << 19 is (x mod 2^13) <= 2 kGuard, one shift-add and one compare.
template <int kGuard>
__device__ __forceinline__ bool near_f16_midpoint_code(float v) {
  return ((__float_as_uint(v) + (uint32_t)(kGuard - 0x1000)) << 19) < ((uint32_t)(2 * kGuard + 1) << 19);
}

// True when the fp32 value `v` is too close to an fp16 rounding boundary (or in
// the fp16 subnormal range) for its rounding to be trusted.
template <int kGuard>
__device__ __forceinline__ bool near_f16_midpoint(float v) {
  const uint32_t u = __float_as_uint(v) & 0x7fffffffu;
  const int low = (int)(u & 0x1fffu) - 0x1000;
  return u < 0x38800000u || (low <= kGuard && low >= -kGuard);
}

// Running maxima of group and page scales take NaN as NumPy's max does (the
// reference's max reductions are restated with it): a NaN element makes the
// maximum NaN, and the scale and every code of the group or page follow.
// nan_max(m, x) for m, x >= 0 or NaN; max_abs_nan(m, x) = nan_max(m, |x|).
__device__ __forceinline__ float nan_max(float m, float x) { return (x > m || x != x) ? x : m; }
__device__ __forceinline__ float max_abs_nan(float m, float x) { return nan_max(m, fabsf(x)); }

// fp32 |atan2(y, x)| for fp16-representable x, y: octant reduction to t =
// min(|x|,|y|)/max in [0, 1], atan(t) = t * P(t^2) with a degree-9
// polynomial in t^2 fitted here for least maximum relative error on [0, 1]
// (Lawson-weighted least squares over Chebyshev nodes), evaluated as t + (t
// t^2) * P1(t^2) with P = 1 + t^2 P1 (the leading term exact), then the
// quadrant: pi/2 - a and pi - a with single fp32 constants (each 0.37 to 0.73
// ulp of the result from the true constant).  Within a few fp32 ulps of the
// true angle; atan2_f16 below only trusts it away from fp16 rounding
// boundaries, and the result and the encoder's codes built on it are checked
// against float64 over all fp16 pairs.
//
// NaN: a NaN x or y gives a NaN angle (IEEE maximum / minimum, v_maximum3_f32
// and v_minimum3_f32, propagate it), and so do two infinite components, whose
// ratio is inf * rcp(inf) = NaN; one infinite component gives the ratio 0 and
// the exact angle.
__device__ __forceinline__ float atan2_poly_mag(float y, float x) {
  const float ax = fabsf(x);
  const float ay = fabsf(y);
  const float mx = __builtin_elementwise_maximum(ax, ay);
  const float mn = __builtin_elementwise_minimum(ax, ay);
  // mx >= 2^-24 for any non-zero fp16 input; for x = y = 0 the clamp keeps t = 0.
  const float t = mn * __builtin_amdgcn_rcpf(__builtin_elementwise_maximum(mx, 0x1p-30f));
  const float u = t * t;
  float p = -0.0017539079999551177f;
  p = __builtin_fmaf(p, u, 0.010726844891905785f);
  p = __builtin_fmaf(p, u, -0.030804410576820374f);
  p = __builtin_fmaf(p, u, 0.05755191296339035f);
  p = __builtin_fmaf(p, u, -0.08377303928136826f);
  p = __builtin_fmaf(p, u, 0.10942026972770691f);
  p = __builtin_fmaf(p, u, -0.142619326710701f);
  p = __builtin_fmaf(p, u, 0.1999826580286026f);
  p = __builtin_fmaf(p, u, -0.3333328366279602f);
  float r = __builtin_fmaf(t * u, p, t);
  constexpr float kHalfPi = 1.57079637050628662f;  // fp32(pi/2)
  constexpr float kPi = 3.14159274101257324f;      // fp32(pi)
  if (ay > ax) r = kHalfPi - r;
  if (__builtin_signbit(x)) r = kPi - r;
  return r;
}
__device__ __forceinline__ float atan2_poly(float y, float x) { return __builtin_copysignf(atan2_poly_mag(y, x), y); }

// fp16 atan2(y, x) for fp16-representable x, y from the fp32 atan2_poly; *exact
// is cleared when the result is too close to an fp16 rounding boundary to be
// trusted (the caller then uses atan2_f16_slow).
__device__ __forceinline__ uint16_t atan2_f16_fast(float y, float x, bool* exact) {
  // A NaN angle (a NaN x or y, or two infinite components) takes the float64
  // path, whose atan2 is NaN, or an odd multiple of pi/4 for two infinities.
  if (y == 0.0f && !__builtin_signbit(x) && !__builtin_isnan(x)) {  // exact +-0
    *exact = true;
    return f2h(y);
  }
  const float a = atan2_poly(y, x);
  *exact = !__builtin_isnan(a) && !near_f16_midpoint<kGuardAtan2>(a);
  return f2h(a);
}
// The float64 fallbacks are real calls: inlined, the compiler hoists their
// float64 constants out of the callers' rare redo loops into the main path
// (some 40 register moves and 40 VGPRs per encoder thread).
__device__ inline __attribute__((noinline)) uint16_t atan2_f16_slow(float y, float x) { return d2h(atan2((double)y, (double)x)); }

// Correctly rounded fp16 atan2(y, x) for fp16-representable x, y.
__device__ __forceinline__ uint16_t atan2_f16(float y, float x) {
  bool exact;
  const uint16_t a = atan2_f16_fast(y, x, &exact);
  return exact ? a : atan2_f16_slow(y, x);
}

// Correctly rounded fp16 natural log of a positive fp16 value (or +inf); the
// fast/slow split mirrors atan2_f16.
__device__ __forceinline__ uint16_t log_f16_fast(float r, bool* exact) {
  // ln r = log2(r) * ln 2: v_log_f32 and one fp32 product, within a few fp32
  // ulps of ln r over the fp16 radii (r >= fp16(1e-6)); the guard hands every
  // result near an fp16 rounding boundary to the float64 path, and
  // tp_selftest_f16_tables checks the outcome for every fp16 input.
  // No subnormal test: the only fp16 r whose ln lies below 2^-14 in magnitude
  // is r = 1 (its neighbours are 1 - 2^-11 and 1 + 2^-10), and log2(1) is 0
  // exactly, so every other result is an fp16-normal value.
  const float l = __builtin_amdgcn_logf(r) * 0.693147180559945309f;
  *exact = !near_f16_midpoint_code<kGuardLog>(l);
  return f2h(l);
}
__device__ inline __attribute__((noinline)) uint16_t log_f16_slow(float r) { return d2h(log((double)r)); }
__device__ __forceinline__ uint16_t log_f16(float r) {
  bool exact;
  const uint16_t l = log_f16_fast(r, &exact);
  return exact ? l : log_f16_slow(r);
}

// Correctly rounded fp16 sqrt of a non-negative fp16 value s: v_sqrt_f16, which
// on gfx950 returns the correctly rounded root for every non-negative fp16
// input (tp_selftest_f16_tables checks all of them against the fp16 rounding of
// the correctly rounded fp32 root, itself exact to fp16: 24 >= 2 * 11 + 2).
__device__ __forceinline__ uint16_t sqrt_f16(float s) {
  return __builtin_bit_cast(uint16_t, __builtin_sqrtf16((f16)s));
}

// fp16(v / s) for fp16-representable v and s > 0 (rs = v_rcp_f32(s)): the
// reciprocal product is within 2 fp32 ulps of v / s, so its fp16 rounding is
// the correctly rounded quotient's unless it is near an fp16 rounding
// boundary; then the correctly rounded fp32 division decides.
__device__ __forceinline__ float div_f16(float v, float s, float rs) {
  const float q = v * rs;
  if (q != 0.0f && near_f16_midpoint<kGuardDiv>(q)) return h2f(f2h(v / s));
  return h2f(f2h(q));
}

// encoder.py:33 for fp16 inputs: f16(sqrt(f16(f16(x*x) + f16(y*y)))).
__device__ __forceinline__ uint16_t radius_f16_in(float x, float y) {
  const float xx = h2f(f2h(x * x));
  const float yy = h2f(f2h(y * y));
  return sqrt_f16(h2f(f2h(xx + yy)));
}

// encoder.py:33 for fp32 inputs: f16(sqrt(x*x + y*y)) with fp32 ops.
__device__ __forceinline__ uint16_t radius_f32_in(float x, float y) {
  const float xx = x * x;
  const float yy = y * y;
  return f2h(sqrtf(xx + yy));
}

// encoder.py:47-55 for an fp16 angle: fp16 shift and divide, clip, then the
// float32 product with (2^bits - 1) rounded half-even.
__device__ __forceinline__ uint32_t angle_code_f16(uint16_t a16, int bits) {
  const float s1 = h2f(f2h(h2f(a16) + h2f(kF16Pi)));
  const float q = s1 * kF32InvF16TwoPi;
  const float n16 = near_f16_midpoint_code<kGuardDiv>(q) ? h2f(f2h(s1 / h2f(kF16TwoPi))) : h2f(f2h(q));
  const float n = fminf(fmaxf(n16, 0.0f), 1.0f);  // NaN -> 0
  // n * (2^bits - 1) lies in [0, 2^bits - 1]: the byte conversion rounds half
  // to even (the reference's mx.round) and saturation never triggers.
  return __builtin_amdgcn_cvt_pk_u8_f32(n * (float)((1 << bits) - 1), 0u, 0u);
}

// encoder.py:47-55 for an fp32 angle: fp32 ops, and the near-one wrap to 0.
__device__ __forceinline__ uint32_t angle_code_f32(float a, int bits) {
  float n = (a + kF32Pi) / kF32TwoPi;
  n = fminf(fmaxf(n, 0.0f), 1.0f);
  if (n > kF32OneMinusEps) n = 0.0f;
  const float lv = (float)((1 << bits) - 1);
  const float c = rintf(n * lv);
  return (uint32_t)fminf(fmaxf(c, 0.0f), lv);
}

// Round-half-even to int8 with clipping; NaN maps to 0.
__device__ __forceinline__ int32_t to_int8_rne(float q) {
  if (q != q) return 0;
  return (int32_t)fminf(fmaxf(rintf(q), -128.0f), 127.0f);
}

// Angle of a code, as PolarQuantDecoder computes it (decoder.py:37-55):
// f32(code)/f32(levels-1) * f32(2*pi) - f32(pi), three separate fp32 ops
// (never contracted, also in sources compiled with FMA contraction).
__device__ __forceinline__ float code_angle(uint32_t code, int bits) {
#pragma clang fp contract(off)
  const float n = (float)code / (float)((1 << bits) - 1);
  const float t = n * kF32TwoPi;
  return t - kF32Pi;
}

// Extract code `idx` of a packed angle-code row (encoder.py:101-130 packing).
__device__ __forceinline__ uint32_t packed_code(const uint8_t* row, int idx, int bits) {
  if (bits == 8) return row[idx];
  if (bits == 4) return (row[idx >> 1] >> ((idx & 1) * 4)) & 15u;
  return (row[idx >> 2] >> ((idx & 3) * 2)) & 3u;
}

// Packed row length in bytes of n codes of `bits` bits.
__host__ __device__ inline int packed_row_bytes(int n, int bits) {
  if (bits == 8) return n;
  if (bits == 4) return (n + 1) / 2;
  return (n + 3) / 4;
}

// Workgroup barrier that orders LDS only: global loads already in flight stay
// in flight (a full __syncthreads() would wait for them).
// Orders one wave's LDS accesses against its other lanes' (the wave's own
// LDS operations complete at the workgroup-scope fences); no other wave takes
// part, so waves may run different iteration counts around it.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace tp

// Host-side error reporting shared by the C-ABI translation units.
namespace tp {
void set_error(const char* fmt, ...);
void clear_error();
bool check_layout(const tp_page_layout* layout, int* l1_row, int* deep_row);
int32_t launch_status(const char* what);
}  // namespace tp
