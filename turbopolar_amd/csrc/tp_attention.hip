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

// ---- key pages ----------------------------------------------------------------
//
// A wave's registers for the key codes of one page (loaded ahead of use so the
// next page's loads overlap the current page's math).

template <int KIND>
struct KRegs;

template <>
struct KRegs<kKindDefault> {  // fp16 radii, 4-bit l1 (pairs 0..31) + 4-bit deep (32..63)
  uint4 r[4][2];
  uint2 c[4];
};

template <>
struct KRegs<kKindFast> {  // int8 log radii + fp16 page scale, 8-bit deep codes, split 0
  uint4 r[4];
  uint4 c[4];
  float ls;
};

template <>
struct KRegs<kKindGeneric> {  // any layout: codes are gathered during the math
  int64_t slot;
};

template <int KIND>
__device__ __forceinline__ void load_k(const AttnArgs& a, int64_t slot, int l16, int l4, KRegs<KIND>& k) {
  if constexpr (KIND == kKindDefault) {
    const uint16_t* rbase = static_cast<const uint16_t*>(a.radii) + slot * (kPageTokens * kPairs) + 16 * l4;
    const uint8_t* cbase = (l4 < 2 ? a.angle_l1 + 8 * l4 : a.angle_deep + 8 * (l4 - 2)) +
                           slot * (kPageTokens * 16);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int t = 16 * mt + l16;
      const uint4* rp = reinterpret_cast<const uint4*>(rbase + t * kPairs);
      k.r[mt][0] = rp[0];
      k.r[mt][1] = rp[1];
      k.c[mt] = *reinterpret_cast<const uint2*>(cbase + t * 16);
    }
  } else if constexpr (KIND == kKindFast) {
    const int8_t* rbase = static_cast<const int8_t*>(a.radii) + slot * (kPageTokens * kPairs) + 16 * l4;
    const uint8_t* cbase = a.angle_deep + slot * (kPageTokens * kPairs) + 16 * l4;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int t = 16 * mt + l16;
      k.r[mt] = *reinterpret_cast<const uint4*>(rbase + t * kPairs);
      k.c[mt] = *reinterpret_cast<const uint4*>(cbase + t * kPairs);
    }
    k.ls = h2f(a.radii_scales[slot]);
  } else {
    k.slot = slot;
  }
}

// QK over one compressed page: s[mt][i] = score(token 16*mt + 4*l4 + i, head l16).
template <int KIND>
__device__ __forceinline__ void qk_regs(const AttnArgs& a, const Lut& lut, const KRegs<KIND>& k,
                                        const half8v* qb, int l16, int l4, float4v* s) {
  if constexpr (KIND == kKindDefault) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const uint32_t rw[8] = {k.r[mt][0].x, k.r[mt][0].y, k.r[mt][0].z, k.r[mt][0].w,
                              k.r[mt][1].x, k.r[mt][1].y, k.r[mt][1].z, k.r[mt][1].w};
      const uint32_t cw[2] = {k.c[mt].x, k.c[mt].y};
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
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const uint32_t rw[4] = {k.r[mt].x, k.r[mt].y, k.r[mt].z, k.r[mt].w};
      const uint32_t cw[4] = {k.c[mt].x, k.c[mt].y, k.c[mt].z, k.c[mt].w};
      float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        uint32_t e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int rc = (int)(int8_t)((rw[kk] >> (8 * i)) & 0xffu);
          const uint32_t code = (cw[kk] >> (8 * i)) & 0xffu;
          const f16 r = (f16)expf((float)rc * k.ls);
          const half2v cs = __builtin_bit_cast(half2v, lut.deep[code]);
          e[i] = pack_h2(half2v{r, r} * cs);
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(e[0], e[1], e[2], e[3]), qb[kk], acc, 0, 0, 0);
      }
      s[mt] = acc;
    }
  } else {
    const int64_t row0 = k.slot * kPageTokens;
    const float ls = a.radii_scales ? h2f(a.radii_scales[k.slot]) : 1.0f;
    for (int mt = 0; mt < 4; ++mt) {
      const int64_t row = row0 + 16 * mt + l16;
      const uint8_t* l1row = a.angle_l1 + row * a.l1_row;
      const uint8_t* deeprow = a.angle_deep + row * a.deep_row;
      float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
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

// ---- value pages --------------------------------------------------------------
//
// Lane (n = l16, l4) owns dims [8n, 8n+8) (group n/4) of the 16 tokens
// 32*ks + 4*l4 + (e&3) + 16*(e>>2), ks = 0..1, e = 0..7.

struct VRegs {
  uint2 w[16];
  uint16_t s[16];
};

__device__ __forceinline__ int v_token(int ks, int l4, int e) { return 32 * ks + 4 * l4 + (e & 3) + 16 * (e >> 2); }

__device__ __forceinline__ void load_v(const AttnArgs& a, int64_t slot, int l16, int l4, VRegs& v) {
  const int8_t* vbase = a.v_codes + slot * (kPageTokens * kHeadDim) + 8 * l16;
  const uint16_t* sbase = a.v_scales + slot * (kPageTokens * kVGroups) + (l16 >> 2);
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int t = v_token(ks, l4, e);
      v.w[8 * ks + e] = *reinterpret_cast<const uint2*>(vbase + t * kHeadDim);
      v.s[8 * ks + e] = sbase[t * kVGroups];
    }
  }
}

// acc[j] += Vhat^T tile j x P, Vhat = f16(code * scale) exactly.
__device__ __forceinline__ void pv_regs(const VRegs& v, const half8v* pb, float4v* acc) {
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    half2v vals[8][4];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const f16 sv = __builtin_bit_cast(f16, v.s[8 * ks + e]);
      const half2v s2 = {sv, sv};
      half2v c0, c1, c2, c3;
      i8x4_to_f16(v.w[8 * ks + e].x, c0, c1);
      i8x4_to_f16(v.w[8 * ks + e].y, c2, c3);
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
      const int t = v_token(ks, l4, e);
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

// ---- online softmax ------------------------------------------------------------

// Folds one page of scores into the running (m, l, acc) of the lane's head and
// returns P (fp16) as the PV B operands.  Scores of tokens >= valid are masked.
__device__ __forceinline__ void softmax_page(const float4v* s, int valid, float scale_log2, int l4,
                                             float& m_run, float& l_run, float4v* acc, half8v* pb) {
  float p[16];
  float pm = -INFINITY;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * mt + 4 * l4 + i;
      const float v = t < valid ? s[mt][i] * scale_log2 : -INFINITY;
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
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int e = 0; e < 8; ++e) pb[ks][e] = (f16)p[4 * (2 * ks + (e >> 2)) + (e & 3)];
  }
}

// ---- cross-workgroup exchange ----------------------------------------------------
//
// Partials are written with agent-scope relaxed atomic stores (coherent across
// the XCDs' L2s without an L2 write-back) and each wave waits for them to be
// acknowledged before the workgroup barrier; the ticket is an agent-scope
// atomic; the combining workgroup reads partials with agent-scope loads.

__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

constexpr int kRedStride = 132;  // padded LDS row of one head's 128 accumulators

template <int WAVES>
struct AttnShared {
  Lut lut;
  float m[WAVES][16];
  float l[WAVES][16];
  float acc[WAVES][16 * kRedStride];
  int last;
};

// ---- decode attention kernel ---------------------------------------------------

template <int KIND, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void decode_attention_kernel(AttnArgs a) {
  __shared__ AttnShared<WAVES> sh;

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

  if (tid < 256) build_lut<KIND>(sh.lut, a, tid);
  half8v qb[4];
  load_q(a, b, kv, h0, nh, l16, l4, qb);
  __syncthreads();

  float m_run = -INFINITY;
  float l_run = 0.0f;
  float4v acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

  // Compressed pages of this split that hold at least one unmasked token.
  const int p_begin = split * a.pages_per_split;
  const int64_t live_pages = (a.seq_len + kPageTokens - 1) / kPageTokens;
  const int p_end = (int)min((int64_t)min(p_begin + a.pages_per_split, a.n_pages), live_pages);

  int page = p_begin + wave;
  KRegs<KIND> kr;
  if (page < p_end) load_k<KIND>(a, bkv * a.capacity + page, l16, l4, kr);
  while (page < p_end) {
    const int64_t slot = bkv * a.capacity + page;
    VRegs vr;
    load_v(a, slot, l16, l4, vr);
    float4v s[4];
    qk_regs<KIND>(a, sh.lut, kr, qb, l16, l4, s);
    const int next = page + WAVES;
    if (next < p_end) load_k<KIND>(a, bkv * a.capacity + next, l16, l4, kr);
    const int valid = (int)min((int64_t)kPageTokens, a.seq_len - (int64_t)page * kPageTokens);
    half8v pb[2];
    softmax_page(s, valid, a.scale_log2, l4, m_run, l_run, acc, pb);
    pv_regs(vr, pb, acc);
    page = next;
  }

  // The dense tail follows the last page; the last split's least loaded wave takes it.
  if (split == a.n_splits - 1 && a.tail_len > 0) {
    const int n_local = max(p_end - p_begin, 0);
    if (wave == n_local % WAVES) {
      const int64_t tok0 = (int64_t)a.n_pages * kPageTokens;
      const int valid = (int)min((int64_t)a.tail_len, a.seq_len - tok0);
      if (valid > 0) {
        float4v s[4];
        qk_tail(a, bkv, qb, l16, l4, s);
        half8v pb[2];
        softmax_page(s, valid, a.scale_log2, l4, m_run, l_run, acc, pb);
        pv_tail(a, bkv, pb, l16, l4, acc);
      }
    }
  }

  // Merge the waves through LDS.
  float l_tot = l_run + __shfl_xor(l_run, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  if (l4 == 0) {
    sh.m[wave][l16] = m_run;
    sh.l[wave][l16] = l_tot;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) sh.acc[wave][l16 * kRedStride + 32 * l4 + 8 * i + j] = acc[j][i];
  }
  __syncthreads();

  // Thread (h = item / 16, c = item % 16) owns dims [8c, 8c+8) of head h.
  const int item = tid & 255;
  const int h = item >> 4;
  const int c = item & 15;
  float M = -INFINITY, L = 0.0f;
  float ACC[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (tid < 256) {
#pragma unroll
    for (int w = 0; w < WAVES; ++w) M = fmaxf(M, sh.m[w][h]);
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float mw = sh.m[w][h];
      const float sc = mw == -INFINITY ? 0.0f : exp2f(mw - M);
      L += sh.l[w][h] * sc;
#pragma unroll
      for (int d = 0; d < 8; ++d) ACC[d] += sh.acc[w][h * kRedStride + 8 * c + d] * sc;
    }
  }
  uint16_t* orow = a.out + ((int64_t)b * a.hq + (int64_t)kv * a.g + h0 + h) * kHeadDim + 8 * c;
  if (a.n_splits == 1) {
    if (tid < 256 && h < nh) {
      uint32_t w[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) w[d] = (uint32_t)f2h(ACC[2 * d] / L) | ((uint32_t)f2h(ACC[2 * d + 1] / L) << 16);
      *reinterpret_cast<uint4*>(orow) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    return;
  }

  const int64_t unit = bkv * a.head_blocks + hb;
  if (tid < 256 && h < nh) {
    const int64_t pbase = (unit * a.n_splits + split) * 16 + h;
    if (c == 0) {
      st_agent(a.part_ml + pbase * 2 + 0, M);
      st_agent(a.part_ml + pbase * 2 + 1, L);
    }
    float* pa = a.part_acc + pbase * kHeadDim + 8 * c;
#pragma unroll
    for (int d = 0; d < 8; ++d) st_agent(pa + d, ACC[d]);
  }
  wait_stores();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(a.counters + unit, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sh.last = prev == (uint32_t)(a.n_splits - 1);
  }
  __syncthreads();
  if (!sh.last) return;

  // Last workgroup of this (b, kv, head block): combine all splits.  Thread
  // (item, sg) folds splits sg, sg + SG, ... of item (h, c); the SG partial
  // results are then merged through LDS.
  const int n_items = nh * 16;
  const int SG = max(1, (WAVES * 64) / n_items);
  const int it = tid % n_items;
  const int sg = tid / n_items;
  const int hh = it >> 4;
  const int cc = it & 15;
  float Mp = -INFINITY, Lp = 0.0f;
  float Ap[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (sg < SG) {
    const float* pm = a.part_ml + (unit * a.n_splits * 16 + hh) * 2;
    const float* pacc = a.part_acc + (unit * a.n_splits * 16 + hh) * kHeadDim + 8 * cc;
#pragma unroll 4
    for (int sp = sg; sp < a.n_splits; sp += SG) {
      const float ms = ld_agent(pm + (int64_t)sp * 32);
      const float ls = ld_agent(pm + (int64_t)sp * 32 + 1);
      float x[8];
#pragma unroll
      for (int d = 0; d < 8; ++d) x[d] = ld_agent(pacc + (int64_t)sp * 16 * kHeadDim + d);
      if (ms == -INFINITY) continue;
      const float mn = fmaxf(Mp, ms);
      const float so = exp2f(Mp - mn);  // 0 while Mp is -inf
      const float sn = exp2f(ms - mn);
      Lp = Lp * so + ls * sn;
#pragma unroll
      for (int d = 0; d < 8; ++d) Ap[d] = Ap[d] * so + x[d] * sn;
      Mp = mn;
    }
  }
  __syncthreads();  // sh.acc is reused below
  float* red = &sh.acc[0][0];  // [SG][n_items][10]
  if (sg < SG) {
    float* r = red + ((int64_t)sg * n_items + it) * 10;
    r[0] = Mp;
    r[1] = Lp;
#pragma unroll
    for (int d = 0; d < 8; ++d) r[2 + d] = Ap[d];
  }
  __syncthreads();
  if (sg == 0) {
    float Mg = -INFINITY;
    for (int g2 = 0; g2 < SG; ++g2) Mg = fmaxf(Mg, red[((int64_t)g2 * n_items + it) * 10]);
    float Lg = 0.0f;
    float Ag[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int g2 = 0; g2 < SG; ++g2) {
      const float* r = red + ((int64_t)g2 * n_items + it) * 10;
      const float sc = r[0] == -INFINITY ? 0.0f : exp2f(r[0] - Mg);
      Lg += r[1] * sc;
#pragma unroll
      for (int d = 0; d < 8; ++d) Ag[d] += r[2 + d] * sc;
    }
    uint16_t* orow2 = a.out + ((int64_t)b * a.hq + (int64_t)kv * a.g + h0 + hh) * kHeadDim + 8 * cc;
    uint32_t w[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) w[d] = (uint32_t)f2h(Ag[2 * d] / Lg) | ((uint32_t)f2h(Ag[2 * d + 1] / Lg) << 16);
    *reinterpret_cast<uint4*>(orow2) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  if (tid == 0) __hip_atomic_store(a.counters + unit, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- standalone fused QK -----------------------------------------------------------

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
  const int page = blockIdx.x * 4 + wave;
  if (page >= a.n_pages) return;
  KRegs<KIND> kr;
  load_k<KIND>(a, bkv * a.capacity + page, l16, l4, kr);
  float4v s[4];
  qk_regs<KIND>(a, lut, kr, qb, l16, l4, s);
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

constexpr int kDecodeWaves = 8;  // wave64s per decode workgroup
constexpr int kTargetWorkgroups = 256;  // one decode workgroup per CU

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
  int64_t pps = (n_pages * units + kTargetWorkgroups - 1) / kTargetWorkgroups;
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
  const dim3 grid((unsigned)((n_pages + 3) / 4), (unsigned)(batch * hkv), (unsigned)a.head_blocks);
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
    case kKindDefault:
      hipLaunchKernelGGL((decode_attention_kernel<kKindDefault, kDecodeWaves>), grid, dim3(kDecodeWaves * 64), 0, s, a);
      break;
    case kKindFast:
      hipLaunchKernelGGL((decode_attention_kernel<kKindFast, kDecodeWaves>), grid, dim3(kDecodeWaves * 64), 0, s, a);
      break;
    default:
      hipLaunchKernelGGL((decode_attention_kernel<kKindGeneric, kDecodeWaves>), grid, dim3(kDecodeWaves * 64), 0, s, a);
      break;
  }
  return launch_status("tp_decode_attention");
}

}  // extern "C"
