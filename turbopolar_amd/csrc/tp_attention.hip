// tp_attention.hip -- fused dequant.QK and split-K decode attention on gfx950.
//
// Work decomposition (decode, batch b, kv head kv, GQA group g <= 16 per head
// block): a 256-thread workgroup owns `pages_per_split` consecutive pages of one
// kv head and scores ALL g query heads of that kv head from a single read of the
// page codes.  Each of its 4 wave64s walks its own pages with a private online
// softmax; the waves are merged through LDS, then the workgroup's partial
// (m, l, acc[128]) per head goes to the workspace and the last workgroup of the
// kv head to arrive (atomic ticket) combines all partials -- one launch per step.
//
// Per page (64 tokens) a wave runs two MFMA chains (v_mfma_f32_16x16x32_f16):
//   QK: S[t][h] = sum_d Khat[t][d] Q[h][d]; A = Khat decoded in registers from
//       the radius + angle codes (cos/sin from an LDS table indexed by code),
//       B = Q (loaded once), 4 token blocks x 4 k-steps.
//   PV: O[d][h] += sum_t Vhat[t][d] P[h][t]; A = Vhat = f16(code * scale)
//       (exact: the dequantised V of v_quant/encoder.py:32-38), B = P in fp16,
//       8 row tiles x 2 k-steps.
// Lane mapping (l16 = lane % 16, l4 = lane / 16):
//   QK A: token 16*mt + l16, pairs 16*l4 + 4*kk + {0..3}   (radii row chunk)
//   QK C: head l16, tokens 16*mt + 4*l4 + {0..3}           (= PV B layout)
//   PV A: d = 8*l16 + j, tokens 32*ks + 4*l4 + {0..3} and +16 (8-byte V loads)
//   PV C: head l16, d = 32*l4 + 8*i + j                    (32 contiguous d)
// so scores never leave registers between the two MFMA chains.
//
// Semantics follow the reference kernels tqpolar_online_attention_quant_v and
// _dense_tail (tqpolar_online_attention.metal:197-390,393-629): tokens with
// global index >= actual_seq_len are masked, the dense fp16 tail follows the
// pages, fp32 softmax statistics and accumulation, fp16 output.
#include "tp_common.h"

namespace tp {

enum LayoutKind { kKindDefault = 0, kKindFast = 1, kKindGeneric = 2 };

struct AttnArgs {
  const uint16_t* q;
  uint16_t* out;
  uint16_t* scores;
  int32_t hq;
  int32_t hkv;
  int32_t g;
  int32_t head_blocks;
  int32_t n_pages;
  int64_t capacity;
  const void* radii;
  const uint16_t* radii_scales;
  const uint8_t* angle_l1;
  const uint8_t* angle_deep;
  const int8_t* v_codes;
  const uint16_t* v_scales;
  int32_t l1_row;
  int32_t deep_row;
  int32_t split_half;
  int32_t l1_bits;
  int32_t deep_bits;
  const uint16_t* tail_k;
  const uint16_t* tail_v;
  int32_t tail_len;
  int64_t tail_stride;
  int64_t seq_len;
  float scale;
  float scale_log2;
  int32_t pages_per_split;
  int32_t n_splits;
  uint32_t* counters;
  float* part_ml;
  float* part_acc;
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ half8v as_half8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const u32x4 v = {a, b, c, d};
  return __builtin_bit_cast(half8v, v);
}

__device__ __forceinline__ uint32_t pack_h2(half2v v) { return __builtin_bit_cast(uint32_t, v); }

__device__ __forceinline__ half2v lo_lo(uint32_t w) {
  const f16 r = __builtin_bit_cast(f16, (uint16_t)(w & 0xffffu));
  return half2v{r, r};
}
__device__ __forceinline__ half2v hi_hi(uint32_t w) {
  const f16 r = __builtin_bit_cast(f16, (uint16_t)(w >> 16));
  return half2v{r, r};
}

// (cos, sin) of a code's decoded angle, rounded to fp16 and packed.
__device__ __forceinline__ uint32_t make_cs(uint32_t code, int bits) {
  const float th = code_angle(code, bits);
  const half2v cs = {(f16)cosf(th), (f16)sinf(th)};
  return pack_h2(cs);
}

// Four int8 codes -> two exact fp16 pairs: bias the byte into the mantissa of
// 1024.0 (0x64xx) after flipping its sign bit, then subtract 1152.
__device__ __forceinline__ void i8x4_to_f16(uint32_t w, half2v& lo, half2v& hi) {
  const uint32_t x = w ^ 0x80808080u;
  const uint32_t a = __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);
  const uint32_t b = __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u);
  const half2v bias = {(f16)1152.0f, (f16)1152.0f};
  lo = __builtin_bit_cast(half2v, a) - bias;
  hi = __builtin_bit_cast(half2v, b) - bias;
}

struct Lut {
  uint32_t l1[256];
  uint32_t deep[256];
};

template <int KIND>
__device__ __forceinline__ void build_lut(Lut& lut, const AttnArgs& a, int tid) {
  const uint32_t c = (uint32_t)tid;
  if constexpr (KIND == kKindDefault) {
    if (c < 16) lut.deep[c] = make_cs(c, 4);
  } else if constexpr (KIND == kKindFast) {
    lut.deep[c] = make_cs(c, 8);
  } else {
    if (c < (1u << a.l1_bits)) lut.l1[c] = make_cs(c, a.l1_bits);
    if (c < (1u << a.deep_bits)) lut.deep[c] = make_cs(c, a.deep_bits);
  }
}

// Q rows of the head block as MFMA B operands: lane (h = l16, l4) holds
// q[h][32*l4 + 8*kk .. +8] for kk = 0..3.
__device__ __forceinline__ void load_q(const AttnArgs& a, int b, int kv, int h0, int nh, int l16,
                                       int l4, half8v* qb) {
  const uint16_t* qrow = a.q + ((int64_t)b * a.hq + (int64_t)kv * a.g + h0 + l16) * kHeadDim + 32 * l4;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    uint4 w = make_uint4(0u, 0u, 0u, 0u);
    if (l16 < nh) w = *reinterpret_cast<const uint4*>(qrow + 8 * kk);
    qb[kk] = as_half8(w.x, w.y, w.z, w.w);
  }
}

// QK over one compressed page: s[mt][i] = score(token 16*mt + 4*l4 + i, head l16).
template <int KIND>
__device__ __forceinline__ void qk_page(const AttnArgs& a, const Lut& lut, int64_t slot,
                                        const half8v* qb, int l16, int l4, float4v* s) {
  if constexpr (KIND == kKindDefault) {
    // fp16 radii; 4-bit l1 codes for pairs 0..31, 4-bit deep codes for 32..63.
    const uint16_t* rbase = static_cast<const uint16_t*>(a.radii) + slot * (kPageTokens * kPairs) + 16 * l4;
    const uint8_t* cbase = (l4 < 2 ? a.angle_l1 + 8 * l4 : a.angle_deep + 8 * (l4 - 2)) +
                           slot * (kPageTokens * 16);
    uint4 rv[4][2];
    uint2 cv[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int t = 16 * mt + l16;
      const uint4* rp = reinterpret_cast<const uint4*>(rbase + t * kPairs);
      rv[mt][0] = rp[0];
      rv[mt][1] = rp[1];
      cv[mt] = *reinterpret_cast<const uint2*>(cbase + t * 16);
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const uint32_t rw[8] = {rv[mt][0].x, rv[mt][0].y, rv[mt][0].z, rv[mt][0].w,
                              rv[mt][1].x, rv[mt][1].y, rv[mt][1].z, rv[mt][1].w};
      const uint32_t cw[2] = {cv[mt].x, cv[mt].y};
      float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        uint32_t e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = 4 * kk + i;
          const uint32_t code = (cw[j >> 3] >> (4 * (j & 7))) & 15u;
          const half2v cs = __builtin_bit_cast(half2v, lut.deep[code]);
          const half2v rr = (j & 1) ? hi_hi(rw[j >> 1]) : lo_lo(rw[j >> 1]);
          e[i] = pack_h2(rr * cs);
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(e[0], e[1], e[2], e[3]), qb[kk], acc, 0, 0, 0);
      }
      s[mt] = acc;
    }
  } else if constexpr (KIND == kKindFast) {
    // int8 log radii with one fp16 scale per page; 8-bit deep codes, split 0.
    const int8_t* rbase = static_cast<const int8_t*>(a.radii) + slot * (kPageTokens * kPairs) + 16 * l4;
    const uint8_t* cbase = a.angle_deep + slot * (kPageTokens * kPairs) + 16 * l4;
    const float ls = h2f(a.radii_scales[slot]);
    uint4 rv[4], cv[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int t = 16 * mt + l16;
      rv[mt] = *reinterpret_cast<const uint4*>(rbase + t * kPairs);
      cv[mt] = *reinterpret_cast<const uint4*>(cbase + t * kPairs);
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const uint32_t rw[4] = {rv[mt].x, rv[mt].y, rv[mt].z, rv[mt].w};
      const uint32_t cw[4] = {cv[mt].x, cv[mt].y, cv[mt].z, cv[mt].w};
      float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        uint32_t e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int rc = (int)(int8_t)((rw[kk] >> (8 * i)) & 0xffu);
          const uint32_t code = (cw[kk] >> (8 * i)) & 0xffu;
          const f16 r = (f16)expf((float)rc * ls);
          const half2v cs = __builtin_bit_cast(half2v, lut.deep[code]);
          e[i] = pack_h2(half2v{r, r} * cs);
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(e[0], e[1], e[2], e[3]), qb[kk], acc, 0, 0, 0);
      }
      s[mt] = acc;
    }
  } else {
    // Any supported layout: per-pair code extraction.
    const int64_t row0 = slot * kPageTokens;
    const float ls = a.radii_scales ? h2f(a.radii_scales[slot]) : 1.0f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int64_t row = row0 + 16 * mt + l16;
      const uint8_t* l1row = a.angle_l1 + row * a.l1_row;
      const uint8_t* deeprow = a.angle_deep + row * a.deep_row;
      float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        uint32_t e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int p = 16 * l4 + 4 * kk + i;
          f16 r;
          if (a.radii_scales) {
            const int rc = static_cast<const int8_t*>(a.radii)[row * kPairs + p];
            r = (f16)expf((float)rc * ls);
          } else {
            r = __builtin_bit_cast(f16, static_cast<const uint16_t*>(a.radii)[row * kPairs + p]);
          }
          uint32_t csw;
          if (p < a.split_half)
            csw = lut.l1[packed_code(l1row, p, a.l1_bits)];
          else
            csw = lut.deep[packed_code(deeprow, p - a.split_half, a.deep_bits)];
          e[i] = pack_h2(half2v{r, r} * __builtin_bit_cast(half2v, csw));
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(e[0], e[1], e[2], e[3]), qb[kk], acc, 0, 0, 0);
      }
      s[mt] = acc;
    }
  }
}

// QK over the dense fp16 tail (tokens >= tail_len read as zero).
__device__ __forceinline__ void qk_tail(const AttnArgs& a, int64_t bkv, const half8v* qb, int l16,
                                        int l4, float4v* s) {
  const uint16_t* tk = a.tail_k + bkv * a.tail_stride * kHeadDim + 32 * l4;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int t = 16 * mt + l16;
    float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      uint4 w = make_uint4(0u, 0u, 0u, 0u);
      if (t < a.tail_len) w = *reinterpret_cast<const uint4*>(tk + t * kHeadDim + 8 * kk);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(w.x, w.y, w.z, w.w), qb[kk], acc, 0, 0, 0);
    }
    s[mt] = acc;
  }
}

// PV over one compressed page: acc[j] += Vhat^T tile j  x  P.
__device__ __forceinline__ void pv_page(const AttnArgs& a, int64_t slot, const half8v* pb, int l16,
                                        int l4, float4v* acc) {
  const int8_t* vbase = a.v_codes + slot * (kPageTokens * kHeadDim) + 8 * l16;
  const uint16_t* sbase = a.v_scales + slot * (kPageTokens * kVGroups) + (l16 >> 2);
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    uint2 vw[8];
    uint16_t sc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int t = 32 * ks + 4 * l4 + (e & 3) + 16 * (e >> 2);
      vw[e] = *reinterpret_cast<const uint2*>(vbase + t * kHeadDim);
      sc[e] = sbase[t * kVGroups];
    }
    // vals[e][0..3]: fp16 pairs (d 0,1), (2,3), (4,5), (6,7) of token e, scaled.
    half2v vals[8][4];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const f16 sv = __builtin_bit_cast(f16, sc[e]);
      const half2v s2 = {sv, sv};
      half2v c0, c1, c2, c3;
      i8x4_to_f16(vw[e].x, c0, c1);
      i8x4_to_f16(vw[e].y, c2, c3);
      vals[e][0] = c0 * s2;
      vals[e][1] = c1 * s2;
      vals[e][2] = c2 * s2;
      vals[e][3] = c3 * s2;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      half8v A;
#pragma unroll
      for (int e = 0; e < 8; ++e) A[e] = (j & 1) ? vals[e][j >> 1].y : vals[e][j >> 1].x;
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, pb[ks], acc[j], 0, 0, 0);
    }
  }
}

// PV over the dense fp16 tail.
__device__ __forceinline__ void pv_tail(const AttnArgs& a, int64_t bkv, const half8v* pb, int l16,
                                        int l4, float4v* acc) {
  const uint16_t* tv = a.tail_v + bkv * a.tail_stride * kHeadDim + 8 * l16;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    half8v rows[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int t = 32 * ks + 4 * l4 + (e & 3) + 16 * (e >> 2);
      uint4 w = make_uint4(0u, 0u, 0u, 0u);
      if (t < a.tail_len) w = *reinterpret_cast<const uint4*>(tv + t * kHeadDim);
      rows[e] = as_half8(w.x, w.y, w.z, w.w);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      half8v A;
#pragma unroll
      for (int e = 0; e < 8; ++e) A[e] = rows[e][j];
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, pb[ks], acc[j], 0, 0, 0);
    }
  }
}

constexpr int kWaves = 4;
constexpr int kRedStride = 132;  // padded LDS row of one head's 128 accumulators

template <int KIND>
__global__ __launch_bounds__(256, 2) void decode_attention_kernel(AttnArgs a) {
  __shared__ Lut lut;
  __shared__ float red_m[kWaves][16];
  __shared__ float red_l[kWaves][16];
  __shared__ float red_acc[kWaves][16 * kRedStride];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l16 = lane & 15;
  const int l4 = lane >> 4;
  const int split = blockIdx.x;
  const int64_t bkv = blockIdx.y;
  const int hb = blockIdx.z;
  const int b = (int)(bkv / a.hkv);
  const int kv = (int)(bkv - (int64_t)b * a.hkv);
  const int h0 = hb * 16;
  const int nh = min(16, a.g - h0);

  build_lut<KIND>(lut, a, tid);
  half8v qb[4];
  load_q(a, b, kv, h0, nh, l16, l4, qb);
  __syncthreads();

  float m_run = -INFINITY;
  float l_run = 0.0f;
  float4v acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

  const int p_begin = split * a.pages_per_split;
  int p_end = min(p_begin + a.pages_per_split, a.n_pages);
  if (split == a.n_splits - 1 && a.tail_len > 0) p_end = a.n_pages + 1;  // tail = virtual page

  for (int page = p_begin + wave; page < p_end; page += kWaves) {
    const int64_t tok0 = (int64_t)page * kPageTokens;
    if (tok0 >= a.seq_len) continue;
    const bool is_tail = page >= a.n_pages;
    const int64_t rem = a.seq_len - tok0;
    const int valid = (int)min((int64_t)(is_tail ? a.tail_len : kPageTokens), rem);
    const int64_t slot = bkv * a.capacity + page;

    float4v s[4];
    if (is_tail)
      qk_tail(a, bkv, qb, l16, l4, s);
    else
      qk_page<KIND>(a, lut, slot, qb, l16, l4, s);

    // Online softmax in the log2 domain; lane (h = l16) owns 16 tokens.
    float p[16];
    float pm = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * mt + 4 * l4 + i;
        const float v = t < valid ? s[mt][i] * a.scale_log2 : -INFINITY;
        p[4 * mt + i] = v;
        pm = fmaxf(pm, v);
      }
    }
    pm = fmaxf(pm, __shfl_xor(pm, 16, 64));
    pm = fmaxf(pm, __shfl_xor(pm, 32, 64));
    const float m_new = fmaxf(m_run, pm);
    const float alpha = exp2f(m_run - m_new);
    float lsum = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      p[k] = exp2f(p[k] - m_new);
      lsum += p[k];
    }
    l_run = l_run * alpha + lsum;
    m_run = m_new;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] *= alpha;

    half8v pb[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[ks][e] = (f16)p[4 * (2 * ks + (e >> 2)) + (e & 3)];
    }
    if (is_tail)
      pv_tail(a, bkv, pb, l16, l4, acc);
    else
      pv_page(a, slot, pb, l16, l4, acc);
  }

  // Merge the 4 waves through LDS.
  float l_tot = l_run + __shfl_xor(l_run, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  if (l4 == 0) {
    red_m[wave][l16] = m_run;
    red_l[wave][l16] = l_tot;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) red_acc[wave][l16 * kRedStride + 32 * l4 + 8 * i + j] = acc[j][i];
  }
  __syncthreads();

  const int h = tid >> 4;
  const int c = tid & 15;
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) M = fmaxf(M, red_m[w][h]);
  float L = 0.0f;
  float ACC[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const float mw = red_m[w][h];
    const float sc = mw == -INFINITY ? 0.0f : exp2f(mw - M);
    L += red_l[w][h] * sc;
#pragma unroll
    for (int d = 0; d < 8; ++d) ACC[d] += red_acc[w][h * kRedStride + 8 * c + d] * sc;
  }

  uint16_t* orow = a.out + ((int64_t)b * a.hq + (int64_t)kv * a.g + h0 + h) * kHeadDim + 8 * c;
  if (a.n_splits == 1) {
    if (h < nh) {
      uint32_t w[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) w[d] = (uint32_t)f2h(ACC[2 * d] / L) | ((uint32_t)f2h(ACC[2 * d + 1] / L) << 16);
      *reinterpret_cast<uint4*>(orow) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    return;
  }

  const int64_t unit = bkv * a.head_blocks + hb;
  const int64_t pbase = (unit * a.n_splits + split) * 16 + h;
  if (h < nh) {
    if (c == 0) {
      a.part_ml[pbase * 2 + 0] = M;
      a.part_ml[pbase * 2 + 1] = L;
    }
    float4* pa = reinterpret_cast<float4*>(a.part_acc + pbase * kHeadDim + 8 * c);
    pa[0] = make_float4(ACC[0], ACC[1], ACC[2], ACC[3]);
    pa[1] = make_float4(ACC[4], ACC[5], ACC[6], ACC[7]);
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = atomicAdd(&a.counters[unit], 1u);
    s_last = prev == (uint32_t)(a.n_splits - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  // Last workgroup of this (b, kv, head block): combine all splits.
  if (h < nh) {
    const float* pm = a.part_ml + (unit * a.n_splits * 16 + h) * 2;
    const float* pacc = a.part_acc + (unit * a.n_splits * 16 + h) * kHeadDim + 8 * c;
    float Mg = -INFINITY;
    for (int sp = 0; sp < a.n_splits; ++sp) Mg = fmaxf(Mg, pm[sp * 32]);
    float Lg = 0.0f;
    float A[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int sp = 0; sp < a.n_splits; ++sp) {
      const float ms = pm[sp * 32];
      const float wgt = ms == -INFINITY ? 0.0f : exp2f(ms - Mg);
      Lg += pm[sp * 32 + 1] * wgt;
      const float4* pa = reinterpret_cast<const float4*>(pacc + (int64_t)sp * 16 * kHeadDim);
      const float4 x0 = pa[0];
      const float4 x1 = pa[1];
      A[0] += x0.x * wgt;
      A[1] += x0.y * wgt;
      A[2] += x0.z * wgt;
      A[3] += x0.w * wgt;
      A[4] += x1.x * wgt;
      A[5] += x1.y * wgt;
      A[6] += x1.z * wgt;
      A[7] += x1.w * wgt;
    }
    uint32_t w[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) w[d] = (uint32_t)f2h(A[2 * d] / Lg) | ((uint32_t)f2h(A[2 * d + 1] / Lg) << 16);
    *reinterpret_cast<uint4*>(orow) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  if (tid == 0) a.counters[unit] = 0u;
}

template <int KIND>
__global__ __launch_bounds__(256) void fused_qk_kernel(AttnArgs a) {
  __shared__ Lut lut;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l16 = lane & 15;
  const int l4 = lane >> 4;
  const int64_t bkv = blockIdx.y;
  const int hb = blockIdx.z;
  const int b = (int)(bkv / a.hkv);
  const int kv = (int)(bkv - (int64_t)b * a.hkv);
  const int h0 = hb * 16;
  const int nh = min(16, a.g - h0);
  build_lut<KIND>(lut, a, tid);
  half8v qb[4];
  load_q(a, b, kv, h0, nh, l16, l4, qb);
  __syncthreads();
  const int page = blockIdx.x * kWaves + wave;
  if (page >= a.n_pages) return;
  float4v s[4];
  qk_page<KIND>(a, lut, bkv * a.capacity + page, qb, l16, l4, s);
  if (l16 >= nh) return;
  const int64_t hq_idx = (int64_t)b * a.hq + (int64_t)kv * a.g + h0 + l16;
  uint16_t* srow = a.scores + hq_idx * ((int64_t)a.n_pages * kPageTokens) + (int64_t)page * kPageTokens + 4 * l4;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const uint32_t w0 = (uint32_t)f2h(s[mt][0] * a.scale) | ((uint32_t)f2h(s[mt][1] * a.scale) << 16);
    const uint32_t w1 = (uint32_t)f2h(s[mt][2] * a.scale) | ((uint32_t)f2h(s[mt][3] * a.scale) << 16);
    *reinterpret_cast<uint2*>(srow + 16 * mt) = make_uint2(w0, w1);
  }
}

// ---- host side ----------------------------------------------------------------

static int layout_kind(const tp_page_layout* L) {
  if (!L->int8_radii && L->l1_bits == 4 && L->deep_bits == 4 && L->split_dim == 64) return kKindDefault;
  if (L->int8_radii && L->deep_bits == 8 && L->split_dim == 0) return kKindFast;
  return kKindGeneric;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static int32_t head_blocks_of(int32_t hq, int32_t hkv) { return (hq / hkv + 15) / 16; }

static int32_t n_splits_of(int32_t n_pages, int32_t pps) {
  return n_pages <= 0 ? 1 : (n_pages + pps - 1) / pps;
}

static bool fill_common(AttnArgs& a, const void* q, int64_t batch, int32_t hq, int32_t hkv,
                        const tp_page_layout* layout, const tp_pages* pages, int32_t n_pages,
                        bool need_v) {
  int l1_row = 0, deep_row = 0;
  if (!check_layout(layout, &l1_row, &deep_row)) return false;
  if (!q || batch < 1 || hq < 1 || hkv < 1 || hq % hkv != 0) {
    set_error("bad query shape: batch=%lld hq=%d hkv=%d (hq must be a multiple of hkv)",
              (long long)batch, hq, hkv);
    return false;
  }
  if (batch * hkv > 65535) {
    set_error("batch * hkv must be <= 65535");
    return false;
  }
  if (n_pages < 0 || (n_pages > 0 && (!pages || pages->capacity < n_pages))) {
    set_error("n_pages=%d exceeds page capacity", n_pages);
    return false;
  }
  if (n_pages > 0) {
    if (!pages->radii || (need_v && (!pages->v_codes || !pages->v_scales)) || (l1_row > 0 && !pages->angle_l1) ||
        (deep_row > 0 && !pages->angle_deep) || (layout->int8_radii && !pages->radii_scales)) {
      set_error("page buffers missing for this layout");
      return false;
    }
    if (((uintptr_t)pages->radii & 15u) || (need_v && ((uintptr_t)pages->v_codes & 15u)) ||
        ((uintptr_t)pages->angle_l1 & 7u) || ((uintptr_t)pages->angle_deep & 15u) ||
        ((uintptr_t)pages->v_scales & 1u)) {
      set_error("page buffers are not aligned");
      return false;
    }
  }
  if ((uintptr_t)q & 15u) {
    set_error("q is not 16-byte aligned");
    return false;
  }
  a = AttnArgs{};
  a.q = static_cast<const uint16_t*>(q);
  a.hq = hq;
  a.hkv = hkv;
  a.g = hq / hkv;
  a.head_blocks = head_blocks_of(hq, hkv);
  a.n_pages = n_pages;
  if (n_pages > 0) {
    a.capacity = pages->capacity;
    a.radii = pages->radii;
    a.radii_scales = layout->int8_radii ? static_cast<const uint16_t*>(pages->radii_scales) : nullptr;
    a.angle_l1 = pages->angle_l1;
    a.angle_deep = pages->angle_deep;
    a.v_codes = pages->v_codes;
    a.v_scales = static_cast<const uint16_t*>(pages->v_scales);
  }
  a.l1_row = l1_row;
  a.deep_row = deep_row;
  a.split_half = layout->split_dim / 2;
  a.l1_bits = layout->l1_bits;
  a.deep_bits = layout->deep_bits;
  return true;
}

}  // namespace tp

using namespace tp;

extern "C" {

int32_t tp_default_pages_per_split(int64_t batch, int32_t hq, int32_t hkv, int32_t n_pages) {
  if (batch < 1 || hq < 1 || hkv < 1 || n_pages < 1) return 4;
  const int64_t units = batch * hkv * (int64_t)head_blocks_of(hq, hkv);
  const int64_t target_wgs = 512;  // two 256-thread workgroups per CU on 256 CUs
  int64_t pps = (n_pages * units + target_wgs - 1) / target_wgs;
  if (pps < 4) pps = 4;
  const int64_t min_pps = (n_pages + 255) / 256;  // at most 256 splits per head
  if (pps < min_pps) pps = min_pps;
  return (int32_t)pps;
}

size_t tp_decode_counter_bytes(int64_t batch, int32_t hq, int32_t hkv) {
  if (batch < 1 || hq < 1 || hkv < 1) return 0;
  return align256((size_t)batch * hkv * head_blocks_of(hq, hkv) * sizeof(uint32_t));
}

size_t tp_decode_workspace_bytes(int64_t batch, int32_t hq, int32_t hkv, int32_t n_pages,
                                 int32_t tail_len, int32_t pages_per_split) {
  (void)tail_len;
  if (batch < 1 || hq < 1 || hkv < 1) return 0;
  if (pages_per_split <= 0) pages_per_split = tp_default_pages_per_split(batch, hq, hkv, n_pages);
  const size_t units = (size_t)batch * hkv * head_blocks_of(hq, hkv);
  const size_t splits = (size_t)n_splits_of(n_pages, pages_per_split);
  return tp_decode_counter_bytes(batch, hq, hkv) + align256(units * splits * 16 * 2 * sizeof(float)) +
         align256(units * splits * 16 * kHeadDim * sizeof(float));
}

int32_t tp_fused_qk(const void* q, int64_t batch, int32_t hq, int32_t hkv,
                    const tp_page_layout* layout, const tp_pages* pages, int32_t n_pages, float scale,
                    void* scores, void* stream) {
  clear_error();
  AttnArgs a;
  if (!fill_common(a, q, batch, hq, hkv, layout, pages, n_pages, false)) return TP_ERR_INVALID;
  if (n_pages == 0) return TP_OK;
  if (!scores || ((uintptr_t)scores & 7u)) {
    set_error("scores must be a non-NULL 8-byte aligned buffer");
    return TP_ERR_INVALID;
  }
  a.scores = static_cast<uint16_t*>(scores);
  a.scale = scale;
  const dim3 grid((unsigned)((n_pages + kWaves - 1) / kWaves), (unsigned)(batch * hkv), (unsigned)a.head_blocks);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (layout_kind(layout)) {
    case kKindDefault: hipLaunchKernelGGL(fused_qk_kernel<kKindDefault>, grid, dim3(256), 0, s, a); break;
    case kKindFast: hipLaunchKernelGGL(fused_qk_kernel<kKindFast>, grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(fused_qk_kernel<kKindGeneric>, grid, dim3(256), 0, s, a); break;
  }
  return launch_status("tp_fused_qk");
}

int32_t tp_decode_attention(const void* q, int64_t batch, int32_t hq, int32_t hkv,
                            const tp_page_layout* layout, const tp_pages* pages, int32_t n_pages,
                            const void* tail_k, const void* tail_v, int32_t tail_len,
                            int64_t tail_stride, int64_t actual_seq_len, float scale,
                            int32_t pages_per_split, void* workspace, size_t workspace_bytes,
                            void* out, void* stream) {
  clear_error();
  AttnArgs a;
  if (!fill_common(a, q, batch, hq, hkv, layout, pages, n_pages, true)) return TP_ERR_INVALID;
  if (!out || ((uintptr_t)out & 15u)) {
    set_error("out must be a non-NULL 16-byte aligned buffer");
    return TP_ERR_INVALID;
  }
  if (tail_len < 0 || tail_len >= kPageTokens) {
    set_error("tail_len must be in [0, 64), got %d", tail_len);
    return TP_ERR_INVALID;
  }
  if (tail_len > 0 && (!tail_k || !tail_v || tail_stride < tail_len ||
                       ((uintptr_t)tail_k & 15u) || ((uintptr_t)tail_v & 15u))) {
    set_error("tail buffers missing, misaligned or tail_stride < tail_len");
    return TP_ERR_INVALID;
  }
  if (n_pages == 0 && tail_len == 0) {
    set_error("nothing to attend: no pages and no tail");
    return TP_ERR_INVALID;
  }
  const int64_t total = (int64_t)n_pages * kPageTokens + tail_len;
  if (actual_seq_len < 1 || actual_seq_len > total) {
    set_error("actual_seq_len=%lld outside [1, %lld]", (long long)actual_seq_len, (long long)total);
    return TP_ERR_INVALID;
  }
  if (pages_per_split <= 0) pages_per_split = tp_default_pages_per_split(batch, hq, hkv, n_pages);
  const int32_t n_splits = n_splits_of(n_pages, pages_per_split);
  if (n_splits > 65535) {
    set_error("too many splits (%d); raise pages_per_split", n_splits);
    return TP_ERR_INVALID;
  }
  a.out = static_cast<uint16_t*>(out);
  a.tail_k = static_cast<const uint16_t*>(tail_k);
  a.tail_v = static_cast<const uint16_t*>(tail_v);
  a.tail_len = tail_len;
  a.tail_stride = tail_stride;
  a.seq_len = actual_seq_len;
  a.scale = scale;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.pages_per_split = pages_per_split;
  a.n_splits = n_splits;
  if (n_splits > 1) {
    const size_t need = tp_decode_workspace_bytes(batch, hq, hkv, n_pages, tail_len, pages_per_split);
    if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255u)) {
      set_error("workspace of %zu bytes (256-byte aligned) required, got %zu", need, workspace_bytes);
      return TP_ERR_WORKSPACE;
    }
    const size_t units = (size_t)batch * hkv * a.head_blocks;
    char* ws = static_cast<char*>(workspace);
    a.counters = reinterpret_cast<uint32_t*>(ws);
    ws += tp_decode_counter_bytes(batch, hq, hkv);
    a.part_ml = reinterpret_cast<float*>(ws);
    ws += align256(units * n_splits * 16 * 2 * sizeof(float));
    a.part_acc = reinterpret_cast<float*>(ws);
  }
  const dim3 grid((unsigned)n_splits, (unsigned)(batch * hkv), (unsigned)a.head_blocks);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (n_pages > 0 ? layout_kind(layout) : (int)kKindGeneric) {
    case kKindDefault: hipLaunchKernelGGL(decode_attention_kernel<kKindDefault>, grid, dim3(256), 0, s, a); break;
    case kKindFast: hipLaunchKernelGGL(decode_attention_kernel<kKindFast>, grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(decode_attention_kernel<kKindGeneric>, grid, dim3(256), 0, s, a); break;
  }
  return launch_status("tp_decode_attention");
}

}  // extern "C"
