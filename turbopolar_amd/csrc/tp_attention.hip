// tp_attention.hip -- fused dequant.QK and split-K decode attention on gfx950.
//
// Work decomposition (decode, batch b, kv head kv, GQA group g <= 16 per head
// block): a 512-thread workgroup (8 wave64s) owns `pages_per_split`
// consecutive pages of one kv head and scores ALL g query heads of that kv head
// from a single read of the page codes.  Each wave walks its own pages with a
// private online softmax; the waves are merged through LDS, then the
// workgroup's partial per head -- (m, l) and its normalised output acc / l in
// fp16 -- goes to the workspace and the last workgroup of the kv head to
// arrive (atomic ticket) combines all partials -- one launch per step.  Above 64 splits per kv head the combine
// has two tiers: groups of 16 splits combine first, and the last group's
// combiner folds the group results.  The grid is (hkv, batch x head blocks,
// splits), kv head fastest, so with the hardware's round-robin dispatch over
// the 8 XCDs every split of one kv head of a batch-1 step runs on the same XCD
// (a locality choice only: correctness does not depend on placement).
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
#include <algorithm>
#include <cstdio>
#include <mutex>
#include <type_traits>

#include "tp_common.h"

namespace tp {

#ifdef TP_TIMELINE
// Phase stamps of the decode kernel (s_memrealtime, 100 MHz), written by
// thread 0 of workgroups < kTimelineGroups; read by tp_timeline_address().
// Built only into the timeline library (TP_TIMELINE defined), never into the
// product.
constexpr int kTimelineGroups = 2048;
constexpr int kTimelineStamps = 80;
__device__ unsigned long long g_timeline[kTimelineGroups][kTimelineStamps];
#define TP_STAMP(k)                                                                            \
  do {                                                                                          \
    const unsigned lin_ = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;       \
    if (threadIdx.x == 0 && lin_ < kTimelineGroups)                                             \
      g_timeline[lin_][(k)] = __builtin_amdgcn_s_memrealtime();                                 \
  } while (0)
#else
#define TP_STAMP(k) \
  do {              \
  } while (0)
#endif
// Stamp slots (thread 0, i.e. wave 0, of each workgroup): 0 start, 59 kernel
// arguments loaded, 60 q loads issued, 1 its first page loads issued, 3 its share of the code tables built, 2 the barrier
// after them passed, 4 + 4i QK of wave 0's page i done (its
// codes arrived), 5 + 4i its PV done, 52 wave 0's pages done; then for the
// whole workgroup 53 records stored, 54 stores complete, 55 ticket drawn; the
// last workgroup of a unit: 64 its combine entered (ticket read from LDS), 65
// its record addresses computed, 66 a second stamp right after 65 (the cost of
// one stamp), 61 its first batch of record loads issued, 62 that batch's (m, l)
// pairs arrived, 57 its record loads folded (thread 0's), 63 every wave's fold
// in LDS, 58 split groups merged, 56 output stored.

// kKindDefaultHR: default-layout pages in the half-row token order (below),
// the decode kernel's form of the default layout for head blocks of at most 8
// query heads.
enum LayoutKind { kKindDefault = 0, kKindFast = 1, kKindGeneric = 2, kKindDefaultHR = 3 };

// Division by a launch constant d as a multiply and a shift: for n < 2^31,
// l = ceil(log2 d) and m = floor(2^(31+l) / d) + 1 (< 2^32), floor(n / d) =
// (n * m) >> (31 + l) (Granlund and Montgomery, PLDI 1994, theorem 4.2:
// 2^(31+l) < m d <= 2^(31+l) + 2^l).  Three scalar instructions instead of
// the ~30-instruction integer division, on the decode kernel's critical
// path before its first page load.
struct FastDiv {
  uint32_t m;
  uint32_t sh;
};

static inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  return FastDiv{(uint32_t)(((1ull << (31 + l)) / d) + 1), 31 + l};
}

__host__ __device__ __forceinline__ uint32_t fast_div(uint32_t n, FastDiv f) {
  return (uint32_t)(((uint64_t)n * f.m) >> f.sh);
}

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
  int32_t live_end;        // min(n_pages, pages holding a token below seq_len)
  FastDiv div_head_blocks; // division by head_blocks
  int32_t counter_stride;  // u32 words between two ticket counters
  int32_t counter_slots;   // ticket counters per unit: 1, or 1 + tier_groups
  uint32_t* counters;
  // Split records: (m, l) of each head in fp32 (part_ml) and the split's
  // normalised output acc / l of each head in fp16 (part_acc).
  float* part_ml;
  uint16_t* part_acc;
  // Two-tier combine (tier_splits > 0): splits [g * tier_splits, ...) form
  // group g of tier_groups; group records in the same layout as part_ml /
  // part_acc with tier_groups records per unit.
  int32_t tier_splits;
  int32_t tier_groups;
  float* tier_ml;
  uint16_t* tier_acc;
  // QJL (tp_fused_qk_qjl, tp_decode_attention_qjl): per-token sketch and
  // residual norm in the page slots, the queries' sketches.
  const uint64_t* qjl_signs;
  const uint16_t* qjl_norms;
  const uint64_t* q_signs;
  int64_t qjl_capacity;  // sketch slots per bh
  int32_t qjl_bits;      // sketch bits P (a multiple of 8, 8 .. 256)
  // Dense fp16 values instead of the V codes (tp_decode_attention_dense_v):
  // [bkv][v_capacity pages][64][128].  Last, so the other fields keep their
  // argument offsets.
  const uint16_t* v_dense;
  int64_t v_capacity;
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Page loads carry the non-temporal hint: every page byte is read once per
// step, and streaming them past the caches measured faster (32k: 20.4 -> 19.7
// us, 131k: 58.5 -> 54.3 us per step).
__device__ __forceinline__ uint4 ldnt4(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ldnt2(const void* p) {
  const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ldnt1(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}

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

// (cos, sin) of a code's decoded angle, rounded to fp16 and packed: the
// reference's fp32 angle (code_angle, decoder.py:37-55) through accurate fp32
// cosf / sinf.  At half a turn the reference's sin(f32(pi)) is -8.7e-8, whose
// fp16 rounding -5.96e-8 is not zero, so an inf radius decodes to -inf there
// as in the reference (decoder.py:57-67); the hardware sine in revolutions
// returns an exact 0 at half a turn, which would turn that product into NaN.
// No code of 2, 4 or 8 bits has a cosine or sine that rounds to fp16 zero.
__device__ __forceinline__ uint32_t make_cs(uint32_t code, int bits) {
  const float th = code_angle(code, bits);
  const half2v cs = {(f16)cosf(th), (f16)sinf(th)};
  return pack_h2(cs);
}

// Two int8 codes (byte B of `lo` and of `hi`) -> an exact fp16 pair, one SDWA
// convert per element (sign-extended byte select, word-select destination).
#define TP_I8PAIR_TO_F16(B)                                                                   \
  __device__ __forceinline__ uint32_t i8pair_f16_b##B(uint32_t lo, uint32_t hi) {            \
    uint32_t d;                                                                               \
    asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_" #B \
        : "=v"(d)                                                                             \
        : "v"(lo));                                                                           \
    asm("v_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_" #B \
        : "=v"(d)                                                                             \
        : "0"(d), "v"(hi));                                                                   \
    return d;                                                                                 \
  }
TP_I8PAIR_TO_F16(0)
TP_I8PAIR_TO_F16(1)
TP_I8PAIR_TO_F16(2)
TP_I8PAIR_TO_F16(3)
#undef TP_I8PAIR_TO_F16

template <int B>
__device__ __forceinline__ uint32_t i8pair_f16(uint32_t lo, uint32_t hi) {
  if constexpr (B == 0) return i8pair_f16_b0(lo, hi);
  if constexpr (B == 1) return i8pair_f16_b1(lo, hi);
  if constexpr (B == 2) return i8pair_f16_b2(lo, hi);
  return i8pair_f16_b3(lo, hi);
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
  uint2 pair[256];  // 4-bit layouts: (cos, sin) of both nibbles of a code byte
};

template <int KIND>
__device__ __forceinline__ void build_lut(Lut& lut, const AttnArgs& a, int tid) {
  const uint32_t c = (uint32_t)tid;
  if constexpr (KIND == kKindDefault || KIND == kKindDefaultHR) {
    lut.pair[c] = make_uint2(make_cs(c & 15u, 4), make_cs(c >> 4, 4));
  } else if constexpr (KIND == kKindFast) {
    lut.deep[c] = make_cs(c, 8);
  } else {
    if (c < (1u << a.l1_bits)) lut.l1[c] = make_cs(c, a.l1_bits);
    if (c < (1u << a.deep_bits)) lut.deep[c] = make_cs(c, a.deep_bits);
  }
}

// Word 3 of a raw buffer resource on gfx9-family GPUs: DATA_FORMAT 32-bit
// (bits 18:15 = 4), every other field 0 (untyped loads, no swizzle).
constexpr int kRawBufferWord3 = 0x00020000;

// Q rows of the head block as MFMA B operands.  Row order: lane (h = l16,
// l4) holds q[h][32*l4 + 8*kk .. +8] for kk = 0..3.  Half-row order (at most
// 8 heads): column l16 is head l16 & 7, half l16 >> 3, and the lane holds
// q[h][64*(l16>>3) + 16*l4 + 8*kk .. +8] for kk = 0, 1.  Heads past the
// block's own (>= nh) hold zeros.  The rows are read as raw buffer loads
// bounded to the block's nh rows, so those lanes read zeros by the buffer's
// range check: no branch around the loads.  Under a branch, the compiler
// waited for q (s_waitcnt vmcnt) at the branch's join, before any page load
// was issued, so every launch paid a memory round trip for q before its first
// page request.
template <bool HR>
__device__ __forceinline__ void load_q(const AttnArgs& a, int b, int kv, int h0, int nh, int l16,
                                       int l4, half8v* qb) {
  const uint16_t* qblk = a.q + ((int64_t)b * a.hq + (int64_t)kv * a.g + h0) * kHeadDim;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(qblk), (short)0, nh * kHeadDim * (int)sizeof(uint16_t), kRawBufferWord3);
  const int off = HR ? ((l16 & 7) * kHeadDim + 64 * (l16 >> 3) + 16 * l4) * (int)sizeof(uint16_t)
                     : (l16 * kHeadDim + 32 * l4) * (int)sizeof(uint16_t);
#pragma unroll
  for (int kk = 0; kk < (HR ? 2 : 4); ++kk) {
    const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 * kk, 0, 0);
    qb[kk] = as_half8(w.x, w.y, w.z, w.w);
  }
}

// ---- load addresses ------------------------------------------------------------------
//
// Byte offsets, from each page field's base pointer, of one lane's loads of
// page slot `slot` (slot = bkv * capacity + page), as a per-lane base plus a
// per-load offset.  The kernels form their load pointers from these
// functions, and the host-side bounds check (tp_selftest_decode_bounds)
// enumerates the same functions over every lane, wave and workgroup of a
// launch, so the check sees the kernels' own address arithmetic.

// Token orders.  A lane (l16, l4) holds the page scores s[mt][i] of tokens
// score_token(mt, i, l4) for the head of its column l16:
//   row order (every kind but kKindDefaultHR): 16*mt + 4*l4 + i, the QK rows
//     being 16 tokens of 128 dims;
//   half-row order (kKindDefaultHR): 16*mt + 8*(i>>1) + 2*l4 + (i&1), the QK
//     rows being 8 tokens x 2 halves of 64 dims (qk_regs).
// The PV operands take the lane's scores in the order v_token(ks, l4, e) =
// score_token(2 ks + e/4, e%4, l4), and V rows follow it.
__host__ __device__ inline int score_token(int mt, int i, int l4, bool hr) {
  return hr ? 16 * mt + 8 * (i >> 1) + 2 * l4 + (i & 1) : 16 * mt + 4 * l4 + i;
}
__host__ __device__ inline int v_token(int ks, int l4, int e, bool hr = false) {
  return score_token(2 * ks + (e >> 2), e & 3, l4, hr);
}

// Key radii: default layout (fp16), the 32 bytes of pairs 16*l4 .. +15 of
// token t = 16*mt + l16 at base + k_radii_row(t) (two 16-byte loads); fast
// layout (int8 codes), 16 bytes at fast_radii_base + fast_row(t).
__host__ __device__ inline int64_t k_radii_base(int64_t slot, int l4) { return (slot * (kPageTokens * kPairs) + 16 * l4) * 2; }
__host__ __device__ inline int k_radii_row(int t) { return t * kPairs * 2; }
// Half-row order: load g (0..7) of lane (l16, l4) reads the 16 bytes of pairs
// 32*(l16&1) + 8*l4 .. +7 of token 8*g + l16/2, so one load instruction covers
// 8 whole 128-byte token rows (the row order's loads cover half of each of 16
// rows: 13.53 -> 12.99 us for a step's page loads alone at 32k); the codes of
// those 8 pairs are 4 bytes of the token's level-1 row (l16 even: pairs 0..31)
// or deep row (odd: pairs 32..63).
__host__ __device__ inline int64_t hr_radii_base(int64_t slot, int l16, int l4) {
  return slot * (kPageTokens * kPairs * 2) + 128 * (l16 >> 1) + 64 * (l16 & 1) + 16 * l4;
}
__host__ __device__ inline int hr_radii_row(int g) { return g * 8 * kPairs * 2; }
__host__ __device__ inline bool hr_code_from_l1(int l16) { return (l16 & 1) == 0; }
__host__ __device__ inline int64_t hr_code_base(int64_t slot, int l16, int l4) {
  return slot * (kPageTokens * 16) + 16 * (l16 >> 1) + 4 * l4;
}
__host__ __device__ inline int hr_code_row(int g) { return g * 8 * 16; }
// Key angle codes, default layout: 8 bytes of token t from angle_l1 (l4 < 2)
// or angle_deep, at k_code_base + k_code_row(t).
__host__ __device__ inline bool k_code_from_l1(int l4) { return l4 < 2; }
__host__ __device__ inline int64_t k_code_base(int64_t slot, int l4) { return 8 * (l4 & 1) + slot * (kPageTokens * 16); }
__host__ __device__ inline int k_code_row(int t) { return t * 16; }
// Fast layout: int8 log radii and 8-bit angle codes share the row layout
// (64 bytes per token): 16 bytes of token t at fast_base + fast_row(t); the
// page's fp16 radius scale at fast_scale(slot).
__host__ __device__ inline int64_t fast_base(int64_t slot, int l4) { return slot * (kPageTokens * kPairs) + 16 * l4; }
__host__ __device__ inline int fast_row(int t) { return t * kPairs; }
__host__ __device__ inline int64_t fast_scale(int64_t slot) { return slot * 2; }
// Value codes: 8 bytes of token v_token(ks, l4, e), dims 8*l16 .. +7, at
// v_code_base + v_code_row(ks, l4, e); the page's 512 bytes of scales as the
// dwords `lane` and `lane + 64` at v_scale_base + 4*lane (+256).
__host__ __device__ inline int64_t v_code_base(int64_t slot, int l16) { return slot * (kPageTokens * kHeadDim) + 8 * l16; }
__host__ __device__ inline int v_code_row(int ks, int l4, int e, bool hr = false) { return v_token(ks, l4, e, hr) * kHeadDim; }
__host__ __device__ inline int64_t v_scale_base(int64_t slot) { return slot * (kPageTokens * kVGroups) * 2; }
// Dense fp16 V rows (tp_decode_attention_dense_v): 16 bytes of the same rows.
__host__ __device__ inline int64_t dense_v_base(int64_t slot, int l16) { return (slot * (kPageTokens * kHeadDim) + 8 * l16) * 2; }
__host__ __device__ inline int dense_v_row(int ks, int l4, int e, bool hr = false) { return v_token(ks, l4, e, hr) * kHeadDim * 2; }
// QJL sketches (8 bytes per token) and fp16 norms of a lane's scored tokens.
// Row order, tokens 16*mt + 4*l4 .. +3: 32 bytes of sketches at
// qjl_sign_base + 128*mt and 8 bytes of norms at qjl_norm_base + 32*mt.
// Half-row order, tokens 16*mt + 2*l4 + {0, 1} and those + 8: 16 bytes of
// sketches at qjl_sign_base + 128*mt and at + 64 more, 4 bytes of norms at
// qjl_norm_base + 32*mt and at + 16 more.
__host__ __device__ inline int64_t qjl_sign_base(int64_t slot, int l4, bool hr = false) {
  return (slot * kPageTokens + (hr ? 2 : 4) * l4) * 8;
}
__host__ __device__ inline int64_t qjl_norm_base(int64_t slot, int l4, bool hr = false) {
  return (slot * kPageTokens + (hr ? 2 : 4) * l4) * 2;
}
// Any sketch width (nb = P/8 bytes per token): token t's sketch starts at byte
// qjl_any_row(slot, t, nb); its loads are the qjl_any_dwords(row & 3, nb)
// dwords from row - (row & 3); its fp16 norm is at byte 2 * (slot * 64 + t).
__host__ __device__ inline int64_t qjl_any_row(int64_t slot, int t, int nb) { return (slot * kPageTokens + t) * nb; }
__host__ __device__ inline int qjl_any_dwords(int sh, int nb) { return (sh + nb + 3) >> 2; }

// A wave's first page loads: a wave with a page of its own (page < p_end)
// loads it; a wave without one issues the same loads with every lane on lane
// 0's addresses of the split's first page (one cache line per load) instead
// of branching around them.  The specialised layouts always have pages
// (p_begin < n_pages).
__host__ __device__ inline void first_page_load(int page, int p_begin, int p_end, int lane, int& p_load,
                                                int& lane_e) {
  const bool has_page = page < p_end;
  p_load = has_page ? page : p_begin;
  lane_e = has_page ? lane : 0;
}

// Split records in the workspace: record r of unit `unit` (S_area records per
// unit, (m, l) rows of Sp_area pairs per head) holds head h's (m, l) at float
// offset record_ml(unit, h, Sp_area, r) and its normalised output (128 fp16)
// at half offset record_acc(unit, S_area, r, h).  Both are head-major: one
// head's records are consecutive, its outputs consecutive 256-byte rows
// (kRecordAccStride halves apart), so a combine that walks one head's records
// addresses them from one base with immediate offsets.
constexpr int64_t kRecordAccStride = kHeadDim;
__host__ __device__ inline int64_t record_ml(int64_t unit, int h, int Sp_area, int r) {
  return ((unit * 16 + h) * Sp_area + r) * 2;
}
__host__ __device__ inline int64_t record_acc(int64_t unit, int S_area, int r, int h) {
  return ((unit * 16 + h) * S_area + r) * kRecordAccStride;
}
// The combine's record of batch position u (records r0 + u past the thread's
// `mine` reread its last one, then weigh 0).
__host__ __device__ inline int fold_record(int r0, int u, int mine) { return r0 + u < mine - 1 ? r0 + u : mine - 1; }

// ---- QJL correction ---------------------------------------------------------------
//
// tqpolar_fused_qk.metal:200-231, metal.py:262-275 and score_estimate.py:6-54:
// the score of token t for query head h gains |E_t| |q_h| sin(pi/2 (P - 2
// hamming(sketch_t, sketch_h)) / P) (before the attention scale), P sketch
// bits (qjl/encoder.py:19-44 packs them little-endian, P/8 bytes per token).
// The sine of the P + 1 possible Hamming distances is a table in LDS.  Two
// kernel forms: kQjl64 (P = 64, the default; one 8-byte word per token, 16-byte
// loads of two tokens) and kQjlAny (any multiple of 8 up to kQjlMaxBits: the
// dwords covering a token's P/8 bytes, byte-aligned in registers).

constexpr int kQjlOff = 0;
constexpr int kQjl64 = 1;
constexpr int kQjlAny = 2;
constexpr int kQjlBits = 64;
constexpr int kQjlMaxBits = 256;
constexpr int kQjlMaxWords = kQjlMaxBits / 32;

__device__ __forceinline__ void build_qjl_sin(float* tab, int tid, int P) {
  for (int t = tid; t <= P; t += blockDim.x) tab[t] = sinf(1.57079632679489662f * (float)(P - 2 * t) / (float)P);
}

// |q| of the lane's head from its MFMA B operands (row order: 32 dims per
// lane, lane groups l4 = 0..3 hold the four quarters; half-row order: 16 dims
// per lane, the four lane groups of columns l16 and l16 ^ 8 hold the two
// halves) and, for kQjl64, the head's sketch.
template <bool HR, int QJL>
__device__ __forceinline__ void qjl_query(const AttnArgs& a, int b, int kv, int h0, int nh, int l16, const half8v* qb,
                                          uint64_t& qsig, float& qnorm) {
  float ss = 0.0f;
#pragma unroll
  for (int kk = 0; kk < (HR ? 2 : 4); ++kk) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = (float)qb[kk][e];
      ss = __builtin_fmaf(x, x, ss);
    }
  }
  ss += __shfl_xor(ss, 16, 64);
  ss += __shfl_xor(ss, 32, 64);
  if constexpr (HR) ss += __shfl_xor(ss, 8, 64);
  qnorm = sqrtf(ss);
  if constexpr (QJL == kQjl64)
    qsig = a.q_signs[(int64_t)b * a.hq + (int64_t)kv * a.g + h0 + min(l16, nh - 1)];  // unconditional, as load_q
}

// kQjlAny: the sketches of the block's heads as words in LDS, qw[8 h + w] =
// bytes 4w .. 4w+3 of head h's P/8 (zero past them), one word per thread.
__device__ __forceinline__ void qjl_query_words(const AttnArgs& a, int b, int kv, int h0, int nh, int tid,
                                                uint32_t* qw) {
  if (tid < 16 * kQjlMaxWords) {
    const int h = tid / kQjlMaxWords, w = tid % kQjlMaxWords;
    const int nb = a.qjl_bits >> 3;
    const uint8_t* row = reinterpret_cast<const uint8_t*>(a.q_signs) + ((int64_t)b * a.hq + (int64_t)kv * a.g + h0 + h) * nb;
    uint32_t word = 0;
    if (h < nh) {
      for (int j = 0; j < 4; ++j) {
        if (4 * w + j < nb) word |= (uint32_t)row[4 * w + j] << (8 * j);
      }
    }
    qw[tid] = word;
  }
}

// Adds the correction to one page's scores s[mt][i] (token score_token(mt,
// i, l4, HR), head l16) of page slot `slot`, P = 64.
template <bool HR>
__device__ __forceinline__ void qjl_correct(const AttnArgs& a, int64_t slot, int l4, uint64_t qsig, float qnorm,
                                            const float* sin_tab, float4v* s) {
  const char* sg = reinterpret_cast<const char*>(a.qjl_signs) + qjl_sign_base(slot, l4, HR);
  const char* nm = reinterpret_cast<const char*>(a.qjl_norms) + qjl_norm_base(slot, l4, HR);
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    // Sketches and norms of tokens i = 0..3 of s[mt] (consecutive pairs i = 0, 1 and 2, 3).
    const u32x4 w01 = *reinterpret_cast<const u32x4*>(sg + 128 * mt);
    const u32x4 w23 = *reinterpret_cast<const u32x4*>(sg + 128 * mt + (HR ? 64 : 16));
    uint2 nn;
    if constexpr (HR)
      nn = make_uint2(*reinterpret_cast<const uint32_t*>(nm + 32 * mt), *reinterpret_cast<const uint32_t*>(nm + 32 * mt + 16));
    else
      nn = *reinterpret_cast<const uint2*>(nm + 32 * mt);
    const uint64_t k[4] = {((uint64_t)w01.y << 32) | w01.x, ((uint64_t)w01.w << 32) | w01.z,
                           ((uint64_t)w23.y << 32) | w23.x, ((uint64_t)w23.w << 32) | w23.z};
    const float n[4] = {h2f((uint16_t)(nn.x & 0xffffu)), h2f((uint16_t)(nn.x >> 16)), h2f((uint16_t)(nn.y & 0xffffu)),
                        h2f((uint16_t)(nn.y >> 16))};
#pragma unroll
    for (int i = 0; i < 4; ++i) s[mt][i] += n[i] * qnorm * sin_tab[__builtin_popcountll(k[i] ^ qsig)];
  }
}

// The same for any P (kQjlAny).  Token t's sketch is the P/8 bytes at byte
// (slot * 64 + t) * P/8; the lane loads the dwords covering them (a page's
// 64 * P/8 bytes start and end on a dword boundary, so they never leave the
// page's sketches) and aligns them by the byte offset.  qw: the block's query
// words (qjl_query_words), head_row: the lane's head in them.
template <bool HR>
__device__ __forceinline__ void qjl_correct_any(const AttnArgs& a, int64_t slot, int l4, const uint32_t* qw,
                                                int head_row, float qnorm, const float* sin_tab, float4v* s) {
  const int nb = a.qjl_bits >> 3;
  const int nw = (nb + 3) >> 2;
  const uint32_t last_mask = (nb & 3) ? (1u << (8 * (nb & 3))) - 1u : 0xffffffffu;
  uint32_t q[kQjlMaxWords];
#pragma unroll
  for (int w = 0; w < kQjlMaxWords; ++w) q[w] = qw[kQjlMaxWords * head_row + w];
  const char* sg = reinterpret_cast<const char*>(a.qjl_signs);
  const uint16_t* nm = a.qjl_norms + slot * kPageTokens;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = score_token(mt, i, l4, HR);
      const int64_t o = qjl_any_row(slot, t, nb);
      const int sh = (int)(o & 3);
      const uint32_t* p = reinterpret_cast<const uint32_t*>(sg + (o - sh));
      const int cnt = qjl_any_dwords(sh, nb);
      uint32_t d[kQjlMaxWords + 1];
#pragma unroll
      for (int k = 0; k <= kQjlMaxWords; ++k) d[k] = k < cnt ? p[k] : 0u;
      int ham = 0;
#pragma unroll
      for (int w = 0; w < kQjlMaxWords; ++w) {
        if (w < nw) {
          uint32_t tw = __builtin_amdgcn_alignbyte(d[w + 1], d[w], (uint32_t)sh);
          if (w == nw - 1) tw &= last_mask;
          ham += __builtin_popcount(tw ^ q[w]);
        }
      }
      s[mt][i] += h2f(nm[t]) * qnorm * sin_tab[ham];
    }
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
struct KRegs<kKindDefaultHR> {  // the default layout's page, half-row order: load g of hr_radii_row / hr_code_row
  uint4 r[8];
  uint32_t c[8];
};

template <>
struct KRegs<kKindFast> {  // int8 log radii + fp16 page scale, 8-bit deep codes, split 0
  uint4 r[4];
  uint4 c[4];
  uint32_t ls_bits;  // fp16 page scale, converted at use so its load is not waited on early
};

template <>
struct KRegs<kKindGeneric> {  // any layout: codes are gathered during the math
  int64_t slot;
};

template <int KIND>
__device__ __forceinline__ void load_k(const AttnArgs& a, int64_t slot, int l16, int l4, KRegs<KIND>& k) {
  if constexpr (KIND == kKindDefault) {
    const char* rbase = static_cast<const char*>(a.radii) + k_radii_base(slot, l4);
    const char* cbase = reinterpret_cast<const char*>(k_code_from_l1(l4) ? a.angle_l1 : a.angle_deep) +
                        k_code_base(slot, l4);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int t = 16 * mt + l16;
      const char* rp = rbase + k_radii_row(t);
      k.r[mt][0] = ldnt4(rp);
      k.r[mt][1] = ldnt4(rp + 16);
      k.c[mt] = ldnt2(cbase + k_code_row(t));
    }
  } else if constexpr (KIND == kKindDefaultHR) {
    const char* rbase = static_cast<const char*>(a.radii) + hr_radii_base(slot, l16, l4);
    const char* cbase = reinterpret_cast<const char*>(hr_code_from_l1(l16) ? a.angle_l1 : a.angle_deep) +
                        hr_code_base(slot, l16, l4);
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      k.r[g] = ldnt4(rbase + hr_radii_row(g));
      k.c[g] = ldnt1(cbase + hr_code_row(g));
    }
  } else if constexpr (KIND == kKindFast) {
    const char* rbase = static_cast<const char*>(a.radii) + fast_base(slot, l4);
    const char* cbase = reinterpret_cast<const char*>(a.angle_deep) + fast_base(slot, l4);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int t = 16 * mt + l16;
      k.r[mt] = ldnt4(rbase + fast_row(t));
      k.c[mt] = ldnt4(cbase + fast_row(t));
    }
    k.ls_bits = *reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(a.radii_scales) + fast_scale(slot));
  } else {
    k.slot = slot;
  }
}

// The four 16-lane rows of the wave (lanes l, l ^ 16, l ^ 32 and l ^ 48)
// combined in every lane as op(op(row 0, row 1), op(row 2, row 3)):
// v_permlane16_swap pairs rows 0-1 and 2-3 and v_permlane32_swap the halves,
// both register to register (no LDS round trip, unlike a lane shuffle).
template <class Op>
__device__ __forceinline__ float across_rows(float x, Op op) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float s = op(__uint_as_float(p[0]), __uint_as_float(p[1]));
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  return op(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
__device__ __forceinline__ float sum_rows(float x) {
  return across_rows(x, [](float u, float v) { return u + v; });
}
__device__ __forceinline__ float max_rows(float x) {
  return across_rows(x, [](float u, float v) { return fmaxf(u, v); });
}

// Half-row QK output of one group of 8 tokens: the MFMA's rows are (token
// 8g + r/2, half r&1) and its columns (head c&7, half c>>3), so lane (l16, l4)
// holds D[(2*l4 + u, half h)][l16] in acc[2u + h].  The score of token
// 8g + 2*l4 + u for head l16 < 8 is D[(., 0)][(head, 0)] + D[(., 1)][(head,
// 1)]: acc[2u] plus acc[2u + 1] of lane l16 + 8 (a row rotation by 8 lanes).
// Lanes l16 >= 8 end with unused sums.  The scores go to s[mt][j], s[mt][j+1]
// (token order score_token(mt, i, l4, true)).
__device__ __forceinline__ float from_lane_xor8(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, true));  // row_ror:8
}
__device__ __forceinline__ void fold_halves(const float4v& acc, float4v& s, int j) {
  s[j] = acc[0] + from_lane_xor8(acc[1]);
  s[j + 1] = acc[2] + from_lane_xor8(acc[3]);
}

// QK over one compressed page: s[mt][i] = score(token score_token(mt, i, l4,
// KIND == kKindDefaultHR), head l16).
template <int KIND>
__device__ __forceinline__ void qk_regs(const AttnArgs& a, const Lut& lut, const KRegs<KIND>& k,
                                        const half8v* qb, int l16, int l4, float4v* s) {
  if constexpr (KIND == kKindDefaultHR) {
    // Load g: 8 pairs of one token half (A operand row l16 = (8g + l16/2,
    // half l16&1)); k-step kk takes its pairs 4kk .. 4kk+3, code bytes 2kk
    // and 2kk+1 (low nibble first).
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const uint32_t rw[4] = {k.r[g].x, k.r[g].y, k.r[g].z, k.r[g].w};
      const uint32_t cw = k.c[g];
      float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const uint2 cs01 = lut.pair[(cw >> (16 * kk)) & 0xffu];
        const uint2 cs23 = lut.pair[(cw >> (16 * kk + 8)) & 0xffu];
        uint32_t e[4];
        e[0] = pack_h2(lo_lo(rw[2 * kk]) * __builtin_bit_cast(half2v, cs01.x));
        e[1] = pack_h2(hi_hi(rw[2 * kk]) * __builtin_bit_cast(half2v, cs01.y));
        e[2] = pack_h2(lo_lo(rw[2 * kk + 1]) * __builtin_bit_cast(half2v, cs23.x));
        e[3] = pack_h2(hi_hi(rw[2 * kk + 1]) * __builtin_bit_cast(half2v, cs23.y));
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(e[0], e[1], e[2], e[3]), qb[kk], acc, 0, 0, 0);
      }
      fold_halves(acc, s[g >> 1], 2 * (g & 1));
    }
  } else if constexpr (KIND == kKindDefault) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const uint32_t rw[8] = {k.r[mt][0].x, k.r[mt][0].y, k.r[mt][0].z, k.r[mt][0].w,
                              k.r[mt][1].x, k.r[mt][1].y, k.r[mt][1].z, k.r[mt][1].w};
      const uint32_t cw[2] = {k.c[mt].x, k.c[mt].y};
      float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        // Code bytes 2kk and 2kk+1 hold the nibbles of pairs 4kk .. 4kk+3.
        const uint32_t b0 = (cw[kk >> 1] >> (16 * (kk & 1))) & 0xffu;
        const uint32_t b1 = (cw[kk >> 1] >> (16 * (kk & 1) + 8)) & 0xffu;
        const uint2 cs01 = lut.pair[b0];
        const uint2 cs23 = lut.pair[b1];
        uint32_t e[4];
        e[0] = pack_h2(lo_lo(rw[2 * kk]) * __builtin_bit_cast(half2v, cs01.x));
        e[1] = pack_h2(hi_hi(rw[2 * kk]) * __builtin_bit_cast(half2v, cs01.y));
        e[2] = pack_h2(lo_lo(rw[2 * kk + 1]) * __builtin_bit_cast(half2v, cs23.x));
        e[3] = pack_h2(hi_hi(rw[2 * kk + 1]) * __builtin_bit_cast(half2v, cs23.y));
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(e[0], e[1], e[2], e[3]), qb[kk], acc, 0, 0, 0);
      }
      s[mt] = acc;
    }
  } else if constexpr (KIND == kKindFast) {
    // r = exp(code * ls) = 2^(code * ls * log2(e)) on v_exp_f32: code * ls is
    // exact in fp32 (8 x 11 significant bits), so the result matches the
    // reference's f32 exp to ~1e-6 relative, far below the fp16 rounding of r.
    const float ls2 = h2f((uint16_t)k.ls_bits) * 1.44269504088896341f;
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
          const f16 r = (f16)__builtin_amdgcn_exp2f((float)rc * ls2);
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

// ---- value pages --------------------------------------------------------------
//
// Lane (n = l16, l4) owns dims [8n, 8n+8) (group n/4) of the 16 tokens
// v_token(ks, l4, e, HR), ks = 0..1, e = 0..7 (row order: 32*ks + 4*l4 +
// (e&3) + 16*(e>>2); half-row order: 32*ks + 16*(e>>2) + 8*((e>>1)&1) +
// 2*l4 + (e&1)); tokens e and e+1 (e even) are consecutive in both.

struct VRegs {
  uint2 w[16];
  uint32_t sd[2];  // dwords `lane` and `lane + 64` of the page's 128-dword scale block
};

// Issues the V code loads of one page and loads its 512 bytes of scales as
// two coalesced dwords per lane (the scale of token t, group g is half g & 1
// of dword 2t + g / 2); PV gathers each lane's scales from these with lane
// permutes, so the scales hold two registers, not one per token.
template <bool HR>
__device__ __forceinline__ void load_v(const AttnArgs& a, int64_t slot, int l16, int l4, int lane, VRegs& v) {
  const char* vbase = reinterpret_cast<const char*>(a.v_codes) + v_code_base(slot, l16);
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v.w[8 * ks + e] = ldnt2(vbase + v_code_row(ks, l4, e, HR));
  }
  const char* sbase = reinterpret_cast<const char*>(a.v_scales) + v_scale_base(slot);
  v.sd[0] = ldnt1(sbase + 4 * lane);
  v.sd[1] = ldnt1(sbase + 4 * (lane + 64));
}

// acc[j] += Vhat^T tile j x P, Vhat = f16(code * scale) exactly: codes become
// fp16 pairs (tokens e, e+1) by SDWA converts, then one packed multiply by the
// pair's scales.
template <int J>
__device__ __forceinline__ void pv_tile(const VRegs& v, int ks, const half2v* sp, const half8v& pb,
                                        float4v& acc) {
  uint32_t e[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint2 wa = v.w[8 * ks + 2 * q];
    const uint2 wb = v.w[8 * ks + 2 * q + 1];
    const uint32_t c = (J < 4) ? i8pair_f16<J & 3>(wa.x, wb.x) : i8pair_f16<J & 3>(wa.y, wb.y);
    e[q] = pack_h2(__builtin_bit_cast(half2v, c) * sp[q]);
  }
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(e[0], e[1], e[2], e[3]), pb, acc, 0, 0, 0);
}

// sbase4: byte index of the lane holding the scale dword of token
// v_token(0, l4, 0, HR) of the lane's group g (4 * (2 * that token + g/2));
// ssel: v_perm selector taking half g & 1 of two dwords.
template <bool HR>
__device__ __forceinline__ void pv_regs(const VRegs& v, int sbase4, uint32_t ssel, const half8v* pb,
                                        float4v* acc) {
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    // Scales of tokens (2q, 2q+1) of this k-step as fp16 pairs: tokens
    // v_token(0, l4, 0) + t0 and one more (row order t0 = 0, 2, 16, 18;
    // half-row order 0, 8, 16, 24) sit in the dwords of lanes sbase4/4 + 2*t0
    // and two lanes further, in register ks.
    half2v sp[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int t0 = v_token(0, 0, 2 * q, HR);
      const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute(sbase4 + 8 * t0, (int)v.sd[ks]);
      const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute(sbase4 + 8 * t0 + 8, (int)v.sd[ks]);
      sp[q] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(hi, lo, ssel));
    }
    pv_tile<0>(v, ks, sp, pb[ks], acc[0]);
    pv_tile<1>(v, ks, sp, pb[ks], acc[1]);
    pv_tile<2>(v, ks, sp, pb[ks], acc[2]);
    pv_tile<3>(v, ks, sp, pb[ks], acc[3]);
    pv_tile<4>(v, ks, sp, pb[ks], acc[4]);
    pv_tile<5>(v, ks, sp, pb[ks], acc[5]);
    pv_tile<6>(v, ks, sp, pb[ks], acc[6]);
    pv_tile<7>(v, ks, sp, pb[ks], acc[7]);
  }
}

// ---- dense tail -------------------------------------------------------------------
//
// The dense fp16 tail's K and V rows of this (b, kv), all in registers at
// once: raw buffer loads bounded to the tail's tail_len rows, so rows past it
// read as zero by the buffer's range check and no load sits under a branch.
// (Loads under a per-row branch were each waited for before their MFMA: up to
// 32 memory round trips in a row on the last split's critical path.)
// The QK A operands: row order k[4 mt + kk] = K[16 mt + l16][32 l4 + 8 kk ..
// +8]; half-row order k[2 g + kk] = K[8 g + l16/2][64 (l16&1) + 16 l4 + 8 kk ..
// +8].  v[8 ks + e] = V[v_token(ks, l4, e, HR)][8 l16 .. +8] (the PV rows).
struct TailRegs {
  u32x4 k[16];
  u32x4 v[16];
};

template <bool HR>
__device__ __forceinline__ void load_tail(const AttnArgs& a, int64_t bkv, int l16, int l4, TailRegs& r) {
  const int64_t plane = bkv * a.tail_stride * kHeadDim;
  const int bytes = a.tail_len * kHeadDim * (int)sizeof(uint16_t);
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.tail_k + plane),
                                                                      (short)0, bytes, kRawBufferWord3);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.tail_v + plane),
                                                                      (short)0, bytes, kRawBufferWord3);
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int elem = HR ? (8 * (j >> 1) + (l16 >> 1)) * kHeadDim + 64 * (l16 & 1) + 16 * l4 + 8 * (j & 1)
                        : (16 * (j >> 2) + l16) * kHeadDim + 32 * l4 + 8 * (j & 3);
    r.k[j] = __builtin_amdgcn_raw_buffer_load_b128(rk, elem * (int)sizeof(uint16_t), 0, 0);
  }
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int off = (v_token(ks, l4, e, HR) * kHeadDim + 8 * l16) * (int)sizeof(uint16_t);
      r.v[8 * ks + e] = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0);
    }
  }
}

// QK over the dense tail (rows past tail_len are zero), in the token order
// of the pages' scores.
template <bool HR>
__device__ __forceinline__ void qk_tail(const TailRegs& r, const half8v* qb, float4v* s) {
  if constexpr (HR) {
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const u32x4 w = r.k[2 * g + kk];
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(w.x, w.y, w.z, w.w), qb[kk], acc, 0, 0, 0);
      }
      fold_halves(acc, s[g >> 1], 2 * (g & 1));
    }
  } else {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const u32x4 w = r.k[4 * mt + kk];
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(w.x, w.y, w.z, w.w), qb[kk], acc, 0, 0, 0);
      }
      s[mt] = acc;
    }
  }
}

// PV over 64 dense fp16 V rows held as in TailRegs::v (row v_token(ks, l4, e,
// HR) in element 8 ks + e, dims 8 l16 .. +8).
__device__ __forceinline__ void pv_rows(const u32x4* v, const half8v* pb, float4v* acc) {
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    half8v rows[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const u32x4 w = v[8 * ks + e];
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

// PV over the dense fp16 tail.
__device__ __forceinline__ void pv_tail(const TailRegs& r, const half8v* pb, float4v* acc) { pv_rows(r.v, pb, acc); }

// ---- dense values (execute_online_attention_dense_v, metal.py:586-649) --------------
//
// The pages' V as fp16 rows instead of codes and scales: a page's rows in the
// PV layout of the dense tail, 16-byte non-temporal loads.
struct DenseVRegs {
  u32x4 w[16];
};

template <bool HR>
__device__ __forceinline__ void load_v(const AttnArgs& a, int64_t slot, int l16, int l4, int lane, DenseVRegs& v) {
  (void)lane;
  const char* vbase = reinterpret_cast<const char*>(a.v_dense) + dense_v_base(slot, l16);
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint4 w = ldnt4(vbase + dense_v_row(ks, l4, e, HR));
      v.w[8 * ks + e] = u32x4{w.x, w.y, w.z, w.w};
    }
  }
}

template <bool HR>
__device__ __forceinline__ void pv_regs(const DenseVRegs& v, int sbase4, uint32_t ssel, const half8v* pb,
                                        float4v* acc) {
  (void)sbase4;
  (void)ssel;
  pv_rows(v.w, pb, acc);
}

// ---- online softmax ------------------------------------------------------------

// Folds one page of scores into the running (m, l, acc) of the lane's head and
// returns P (fp16) as the PV B operands.  Scores of tokens >= valid are masked.
// The running max is raised lazily: only when some head's page max exceeds it
// by more than kLazyRescale (log2 units), so P stays <= 2^kLazyRescale (exact
// enough in fp16) and the 32-register accumulator rescale is rare.
constexpr float kLazyRescale = 8.0f;

template <bool HR>
__device__ __forceinline__ void softmax_page(const float4v* s, int valid, float scale_log2, int l4,
                                             float& m_run, float& l_run, float4v* acc, half8v* pb) {
  float x[16];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[4 * mt + i] = s[mt][i] * scale_log2;
  }
  if (valid < kPageTokens) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (score_token(mt, i, l4, HR) >= valid) x[4 * mt + i] = -INFINITY;
      }
    }
  }
  float pm = x[0];
#pragma unroll
  for (int k = 1; k < 16; ++k) pm = fmaxf(pm, x[k]);
  pm = max_rows(pm);
  if (__builtin_amdgcn_ballot_w64(pm > m_run + kLazyRescale)) {
    const float m_new = fmaxf(m_run, pm);
    // From an empty state (m_run = -inf) the factor is 0: l and acc are 0,
    // or NaN after a page whose scores were all NaN, and NaN must survive.
    const float alpha = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] *= alpha;
    m_run = m_new;
  }
  // m_run is still -inf only if every score of this page is -inf or NaN: then
  // -inf scores weigh 0 and NaN scores stay NaN, as in the reference's softmax.
  const float m_use = m_run == -INFINITY ? 0.0f : m_run;
  float lsum = 0.0f;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    x[k] = __builtin_amdgcn_exp2f(x[k] - m_use);
    lsum += x[k];
  }
  l_run += lsum;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int e = 0; e < 8; ++e) pb[ks][e] = (f16)x[4 * (2 * ks + (e >> 2)) + (e & 3)];
  }
}

// ---- cross-workgroup exchange ----------------------------------------------------
//
// Records are written with sc1 vector stores: agent-scope stores, written
// through to the level that all XCDs see.  Each wave waits for their
// acknowledgements (s_waitcnt vmcnt(0)) before the workgroup barrier that
// precedes the ticket (finish_unit), so every record is complete at agent
// scope before its ticket is drawn.  No release fence is issued: on gfx950 an
// agent-scope release writes back the whole L2 of the XCD (buffer_wbl2),
// which measured 1.0-1.7 us per step here, while these stores leave nothing
// of the record in any cache to write back.

// fp16 pair of two fp32 values (round to nearest even).
__device__ __forceinline__ uint32_t pack_f2h2(float x, float y) {
  return (uint32_t)f2h(x) | ((uint32_t)f2h(y) << 16);
}
// 1 / l of a record: an empty split (l = 0, m = -inf) stores zeros; a NaN l
// stays NaN.
__device__ __forceinline__ float record_inv(float l) { return l == 0.0f ? 0.0f : __builtin_amdgcn_rcpf(l); }
// 4 dims of a record's normalised output v * inv as fp16, one 8-byte store.
__device__ __forceinline__ void st_agent_h4(uint16_t* p, float4v v, float inv) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 w = {pack_f2h2(v[0] * inv, v[1] * inv), pack_f2h2(v[2] * inv, v[3] * inv)};
  asm volatile("global_store_dwordx2 %0, %1, off sc1" : : "v"(p), "v"(w) : "memory");
}
__device__ __forceinline__ void st_agent2(float* p, float x, float y) {
  typedef float float2v __attribute__((ext_vector_type(2)));
  const float2v v = {x, y};
  asm volatile("global_store_dwordx2 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

constexpr int kRedStride = 132;  // padded LDS row of one head's 128 accumulators
// Ticket counters live in a fixed 64 KiB area at the start of the workspace,
// so its record area starts at the same offset for every shape and a workspace
// shared by calls of different shapes never finds records where counters
// belong.  Counters sit 256 bytes apart while the units fit (the tickets of all
// units arrive within a few microseconds, and one shared cache line serialises
// them), closer beyond 256 units; beyond 16384 units the area grows.
constexpr size_t kCounterArea = 65536;
static inline int32_t counter_stride_of(int64_t units) {
  int32_t w = 64;
  while (w > 1 && (size_t)units * w * sizeof(uint32_t) > kCounterArea) w >>= 1;
  return w;
}

// Normalised fp16 output of 4 consecutive dims.
__device__ __forceinline__ void store_out4(uint16_t* orow, const float* x, float inv) {
  *reinterpret_cast<uint2*>(orow) = make_uint2((uint32_t)f2h(x[0] * inv) | ((uint32_t)f2h(x[1] * inv) << 16),
                                               (uint32_t)f2h(x[2] * inv) | ((uint32_t)f2h(x[3] * inv) << 16));
}

// Folds the 8 wave states of dims d0 .. d0+3 of head h, in wave order.  A
// state with m = -inf weighs 0, so an empty one adds 0 and one that carries
// NaN (all of its scores NaN) still makes the fold NaN.
template <class Shared>
__device__ __forceinline__ void fold_waves(const Shared& sh, int h, int d0, float& M, float& L, float* A) {
  constexpr int W = sizeof(sh.ml) / sizeof(sh.ml[0]);
  float m[W], l[W];
  float4v x[W];
#pragma unroll
  for (int u = 0; u < W; ++u) {
    const float2 ml = sh.ml[u][h];
    m[u] = ml.x;
    l[u] = ml.y;
    x[u] = *reinterpret_cast<const float4v*>(&sh.acc[u][h * kRedStride + d0]);
  }
#pragma unroll
  for (int u = 0; u < W; ++u) M = fmaxf(M, m[u]);
#pragma unroll
  for (int u = 0; u < W; ++u) {
    const float w = m[u] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m[u] - M);
    L += l[u] * w;
#pragma unroll
    for (int i = 0; i < 4; ++i) A[i] += x[u][i] * w;
  }
}

// Merges the partial folds of split groups 1 .. SG-1 of item `it` (LDS slot
// (g << ish) + it) into group 0's state, in group order.
// The fold state of a combining thread's 8 dims.
struct Acc8 {
  float4v lo, hi;
};

template <int SG>
__device__ __forceinline__ void merge_groups(const Acc8* red, const float2* redml, int it, int ish, float& Mc,
                                             float& Lc, Acc8& Ac) {
  float2 r[SG];
  Acc8 x[SG];
#pragma unroll
  for (int g2 = 1; g2 < SG; ++g2) {
    r[g2] = redml[(g2 << ish) + it];
    x[g2] = red[(g2 << ish) + it];
  }
  float Mx = Mc;
#pragma unroll
  for (int g2 = 1; g2 < SG; ++g2) Mx = fmaxf(Mx, r[g2].x);
  const float w0 = Mc == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(Mc - Mx);
  Lc *= w0;
  Ac.lo *= w0;
  Ac.hi *= w0;
#pragma unroll
  for (int g2 = 1; g2 < SG; ++g2) {
    const float w = r[g2].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(r[g2].x - Mx);
    Lc += r[g2].y * w;
    Ac.lo += x[g2].lo * w;
    Ac.hi += x[g2].hi * w;
  }
  Mc = Mx;
}

// Online fold of records 0 .. mine-1 (record r at pml + 2*SG*r, pac + r*rstride)
// in batches of B, all B + 1 loads of a batch in flight together: a record
// past `mine` rereads the last one and is then given weight 0, so the loads
// are unconditional.  A record holds its split's (m, l) and its normalised
// output o = acc / l in fp16, so it enters the fold as acc = o * l; a lane
// reads 8 dims (16 bytes) of o per record, which halves the load
// instructions of fp32 records at 4 dims per lane (the combining CU's load
// instructions bound the combine).  Records and states with m = -inf weigh 0
// (NaN they carry survives).
template <int B>
__device__ __forceinline__ void fold_records(const float* pml, const uint16_t* pac, int SG, int64_t rstride,
                                             int mine, float& Mc, float& Lc, Acc8& Ac) {
  // The 16 lanes of each lane group share (head, split group) and `mine`
  // (16 items per head, groups of 16 lanes all active or all idle), so one load
  // per batch fetches the B (m, l) pairs, lane k of the group holding record
  // k, and lane permutes within the group hand them to every lane.
  const int lane = threadIdx.x & 63;
  const int group_base = (lane & 48) * 4;  // byte address of lane 0 of this group
  for (int r0 = 0; r0 < mine; r0 += B) {
    float2 r[B];
    uint4 x[B];
    const float2 mlk = *reinterpret_cast<const float2*>(pml + 2 * SG * fold_record(r0, lane & (B - 1), mine));
#pragma unroll
    for (int u = 0; u < B; ++u) x[u] = *reinterpret_cast<const uint4*>(pac + fold_record(r0, u, mine) * rstride);
    if (r0 == 0) TP_STAMP(61);
#pragma unroll
    for (int u = 0; u < B; ++u) {
      r[u].x = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(group_base + 4 * u, __builtin_bit_cast(int, mlk.x)));
      r[u].y = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(group_base + 4 * u, __builtin_bit_cast(int, mlk.y)));
    }
    if (r0 == 0) TP_STAMP(62);
#pragma unroll
    for (int u = 0; u < B; ++u) {
      if (r0 + u >= mine) {
        r[u] = make_float2(-INFINITY, 0.0f);
        x[u] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
    float Mn = Mc;
#pragma unroll
    for (int u = 0; u < B; ++u) Mn = fmaxf(Mn, r[u].x);
    const float w0 = Mc == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(Mc - Mn);
    Lc *= w0;
    Ac.lo *= w0;
    Ac.hi *= w0;
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const float w = r[u].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(r[u].x - Mn);
      const float wl = r[u].y * w;
      const half2v o0 = __builtin_bit_cast(half2v, x[u].x);
      const half2v o1 = __builtin_bit_cast(half2v, x[u].y);
      const half2v o2 = __builtin_bit_cast(half2v, x[u].z);
      const half2v o3 = __builtin_bit_cast(half2v, x[u].w);
      Lc += wl;
      Ac.lo += float4v{(float)o0[0], (float)o0[1], (float)o1[0], (float)o1[1]} * wl;
      Ac.hi += float4v{(float)o2[0], (float)o2[1], (float)o3[0], (float)o3[1]} * wl;
    }
    Mc = Mn;
  }
}

// A decode workgroup's place in the 3-D grid (hkv, batch * head_blocks,
// n_splits).  x runs fastest, so consecutive workgroup ids go to different kv
// heads and, with round-robin dispatch over the 8 XCDs, every split of one kv
// head of a batch-1 step runs on the same XCD; the split and the kv head come
// straight from the block index (no division before the first page request).
struct DecodeSlot {
  int split, b, kv, hb;
  int64_t bkv;
};

__device__ __forceinline__ DecodeSlot decode_slot(const AttnArgs& a) {
  DecodeSlot d;
  d.kv = (int)blockIdx.x;
  d.split = (int)blockIdx.z;
  d.b = (int)fast_div(blockIdx.y, a.div_head_blocks);
  d.hb = (int)blockIdx.y - d.b * a.head_blocks;
  d.bkv = (int64_t)d.b * a.hkv + d.kv;
  return d;
}

template <int WAVES>
struct AttnShared {
  Lut lut;
  float2 ml[WAVES][16];
  alignas(16) float acc[WAVES][16 * kRedStride];
  int last;
};

// ---- end of a split: merge the waves, publish the record, combine ------------------
//
// Every wave holds an online-softmax state (m_run, l_run, acc) of its tokens:
// lane (head l16, lane group l4) holds dims 32*l4 + 8*i + j of head l16 in
// acc[j][i] and a partial l over its own scores.  The waves merge through LDS
// into one (m, l, acc[128]) per head; with one split acc / l is the output,
// otherwise (m, l) and acc / l in fp16 become the split's record and the last
// split of the unit to arrive combines all records.
//
// Cross-workgroup ordering: every wave's agent-scope record stores complete
// (s_waitcnt) before the workgroup barrier, then one thread draws the ticket
// with a relaxed agent-scope atomic; the workgroup that draws the last ticket
// issues an agent-scope acquire fence (invalidating its XCD's non-coherent
// cache lines) before the barrier after which it reads the records.
// End-phase variants of the measurement library (0 in the product).
constexpr int kFlRelease = 1;    // agent-scope release fence before the ticket
constexpr int kFlNoAcquire = 2;  // no acquire fence in the combining workgroup
constexpr int kFlTiers = 4;      // two-tier combine (launched only when tier_splits > 0)
constexpr int kFlBatch16 = 8;    // one-tier combine of exactly 16 splits (4-wave launches)

// One thread draws a ticket of a counter that `count` workgroups increment:
// relaxed agent-scope add; the workgroup that draws the last ticket issues an
// agent-scope acquire before it reads the records the others published.
template <int FL>
__device__ __forceinline__ bool draw_ticket(uint32_t* ctr, uint32_t count) {
  if constexpr ((FL & kFlRelease) != 0) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool last = prev == count - 1u;
  if constexpr ((FL & kFlNoAcquire) == 0) {
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  return last;
}

// A combining thread's item: (head hh, 8-dim chunk c8), nh * 16 items padded
// to a power of two 2^ish >= 32; thread (item, sg), sg < SG = 2^lsg = threads /
// 2^ish, folds records sg, sg + SG, ...
struct CombineItem {
  int it, sg, hh, c8, ish, lsg;
  bool item;
};

__host__ __device__ inline CombineItem combine_item(int tid, int nh, int waves) {
  CombineItem c;
  const int n_items = nh * 16;
  c.ish = n_items <= 32 ? 5 : (n_items <= 64 ? 6 : (n_items <= 128 ? 7 : 8));
  c.lsg = (waves == 8 ? 9 : 8) - c.ish;  // log2(threads) - ish; 4-wave launches have nh <= 8
  c.it = tid & ((1 << c.ish) - 1);
  c.sg = tid >> c.ish;
  c.item = c.it < n_items && tid < waves * 64;
  c.hh = c.it >> 4;
  c.c8 = c.it & 15;
  return c;
}

// Combines records first .. first+count-1 of a record area (S_area records per
// unit; (m, l) rows of Sp_area pairs per head): every thread folds its share
// online (running max, rescaled sums) with all loads of a batch of records in
// flight together (batches of 4 when no thread has more than 4 records, else
// 8); the SG partial folds then meet in LDS and are merged in sg order.  The
// threads with sg == 0 return the item's (M, L, A).
template <class Merge>
__device__ __forceinline__ void combine_records(Merge& sh, const CombineItem& ci, const float* part_ml,
                                                const uint16_t* part_acc, int64_t unit, int S_area, int Sp_area,
                                                int first, int count, float& Mc, float& Lc, Acc8& Ac) {
  constexpr int WAVES = sizeof(sh.ml) / sizeof(sh.ml[0]);
  // As many split groups as the threads allow: the record loads then spread
  // over every wave (fewer groups with more records each were slower).
  const int lsg = ci.lsg;
  const int SG = 1 << lsg;
  const bool active = ci.item;
  const int mine = active ? (count - ci.sg + SG - 1) >> lsg : 0;
  const uint16_t* pac = part_acc + record_acc(unit, S_area, first + ci.sg, ci.hh) + 8 * ci.c8;
  const float* pml = part_ml + record_ml(unit, ci.hh, Sp_area, first + ci.sg);
  const int64_t rstride = (int64_t)SG * kRecordAccStride;
  TP_STAMP(65);
  TP_STAMP(66);
  Mc = -INFINITY;
  Lc = 0.0f;
  Ac.lo = float4v{0.0f, 0.0f, 0.0f, 0.0f};
  Ac.hi = Ac.lo;
  if (((count + SG - 1) >> lsg) <= 4)
    fold_records<4>(pml, pac, SG, rstride, mine, Mc, Lc, Ac);
  else
    fold_records<8>(pml, pac, SG, rstride, mine, Mc, Lc, Ac);
  TP_STAMP(57);
  if (SG > 1) {
    const int tid = threadIdx.x;
    Acc8* red = reinterpret_cast<Acc8*>(&sh.acc[0][0]);
    float2* redml = reinterpret_cast<float2*>(red + (WAVES * 64));
    if (active) {
      red[tid] = Ac;
      redml[tid] = make_float2(Mc, Lc);
    }
    lds_barrier();
    TP_STAMP(63);
    if (ci.sg == 0 && ci.item) {
      if (lsg == 1)
        merge_groups<2>(red, redml, ci.it, ci.ish, Mc, Lc, Ac);
      else if (lsg == 2)
        merge_groups<4>(red, redml, ci.it, ci.ish, Mc, Lc, Ac);
      else if (lsg == 3)
        merge_groups<8>(red, redml, ci.it, ci.ish, Mc, Lc, Ac);
      else
        merge_groups<16>(red, redml, ci.it, ci.ish, Mc, Lc, Ac);
    }
  }
}

// One-tier combine by whole head rows, for up to kHeadCombineMax records:
// wave w combines heads w, w + WAVES, ... and lane l owns dims 2l and 2l + 1.
// The records come in batches of B (16 when there are at most 16, else 32),
// all B + 1 loads of a batch in flight together: lane j (mod B) reads record
// j's (m, l), and every lane reads the 4 bytes of its two dims of each
// record's fp16 output (a head's 256-byte row per record; a full batch's rows
// are consecutive, so its loads take immediate offsets from one base).  The
// batch maximum and the sum of the weights w_j = l_j 2^(m_j - M) are B-lane
// reductions by DPP within each 16-lane row and scalar reads of rows 0 and 1
// (no LDS round trips); the weights reach every lane through the wave's own
// 32 words of LDS (written, then read back as broadcast 16-byte reads by the
// same wave), and each lane folds its 2 x B products with mixed-precision FMAs
// from the fp16 outputs.
// No split groups and no merge between waves (the split-group combine of
// combine_records spent 0.42 µs of the 32k step's end phase in its LDS merge
// alone).  Records past `count` are read as the last one and enter with weight
// 0 and output 0; records with m = -inf weigh 0 (a NaN they carry survives, as
// in fold_records).
constexpr int kHeadCombineMax = 64;

// x from lane l of the wave's 16-lane row, for the DPP row control CTRL.
template <int CTRL>
__device__ __forceinline__ float row_dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
// op over lanes 0 .. B - 1 (B = 16 or 32) of the wave, returned in every lane:
// each 16-lane row reduces itself by DPP (quad swaps xor 1 and xor 2, then
// the half-row and row mirrors, after which every lane holds its row's
// result), and rows 0 and 1 are read back as scalars.
template <int B, class Op>
__device__ __forceinline__ float batch_reduce(float x, Op op) {
  static_assert(B == 16 || B == 32, "batches of 16 or 32 records");
  x = op(x, row_dpp<0xb1>(x));   // quad_perm [1, 0, 3, 2]
  x = op(x, row_dpp<0x4e>(x));   // quad_perm [2, 3, 0, 1]
  x = op(x, row_dpp<0x141>(x));  // row_half_mirror
  x = op(x, row_dpp<0x140>(x));  // row_mirror
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
  if constexpr (B == 16) return r0;
  return op(r0, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16)));
}

// One batch of fold_head_records: records r0 .. r0 + B - 1 of one head.  A
// full batch (kFull: all B records exist) reads record j at a fixed offset
// j * 256 bytes from the batch's base, so its B loads need no address
// arithmetic; the last, partial batch rereads the head's last record in place
// of those past `count`.
template <int B, bool kFull>
__device__ __forceinline__ void fold_head_batch(const float* pml, const uint16_t* pac, int r0, int count, int lane,
                                                float* wb, float& Mc, float& Lc, float& A0, float& A1) {
  const int rj = r0 + (lane & (B - 1));
  const float2 ml = *reinterpret_cast<const float2*>(pml + 2 * (kFull ? rj : min(rj, count - 1)));
  const uint16_t* pb = pac + (int64_t)r0 * kRecordAccStride;
  uint32_t o[B];
#pragma unroll
  for (int j = 0; j < B; ++j)
    o[j] = *reinterpret_cast<const uint32_t*>(pb + (int64_t)(kFull ? j : min(j, count - 1 - r0)) * kRecordAccStride);
  if (r0 == 0) TP_STAMP(61);
  const float m = kFull || rj < count ? ml.x : -INFINITY;
  const float Mn = fmaxf(Mc, batch_reduce<B>(m, [](float x, float y) { return fmaxf(x, y); }));
  const float w = m == -INFINITY ? 0.0f : ml.y * __builtin_amdgcn_exp2f(m - Mn);
  const float Ls = batch_reduce<B>(w, [](float x, float y) { return x + y; });
  const float s0 = Mc == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(Mc - Mn);
  Lc = Lc * s0 + Ls;
  A0 *= s0;
  A1 *= s0;
  if (lane < B) wb[lane] = w;
  if (r0 == 0) TP_STAMP(62);
#pragma unroll
  for (int k = 0; k < B / 4; ++k) {
    const float4v wk = *reinterpret_cast<const float4v*>(wb + 4 * k);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t x = kFull || r0 + 4 * k + i < count ? o[4 * k + i] : 0u;
      const half2v oj = __builtin_bit_cast(half2v, x);
      A0 = __builtin_fmaf((float)oj[0], wk[i], A0);
      A1 = __builtin_fmaf((float)oj[1], wk[i], A1);
    }
  }
  Mc = Mn;
}

template <int B>
__device__ __forceinline__ void fold_head_records(const float* pml, const uint16_t* pac, int count, int lane, float* wb,
                                                  float& Mc, float& Lc, float& A0, float& A1) {
  Mc = -INFINITY;
  Lc = 0.0f;
  A0 = 0.0f;
  A1 = 0.0f;
  for (int r0 = 0; r0 < count; r0 += B) {
    if (r0 + B <= count)
      fold_head_batch<B, true>(pml, pac, r0, count, lane, wb, Mc, Lc, A0, A1);
    else
      fold_head_batch<B, false>(pml, pac, r0, count, lane, wb, Mc, Lc, A0, A1);
  }
}

// Where combine_heads' wave finds its first head's records and output row:
// computed before the ticket is drawn, so a last workgroup issues its record
// loads without address arithmetic (or instruction fetches for it) after the
// ticket returns.
struct HeadRecords {
  const float* pml;     // record_ml(unit, wave, Sp, 0)
  const uint16_t* pac;  // record_acc(unit, S, 0, wave) + 2 * lane
  uint16_t* out;        // output row of head h0 + wave, dims 2 * lane
};

// The general head-row combine (any count, heads w, w + WAVES, ...), as a
// real call: its code then sits away from the straight path that follows the
// ticket, which the compiler lays out as the fall-through.
template <int WAVES>
__device__ __attribute__((noinline)) void combine_head_rows(float* wb, int wave, int lane, int nh, int S, int Sp,
                                                            int count, const float* pml, const uint16_t* pac,
                                                            uint16_t* out_rows) {
  for (int hh = wave; hh < nh; hh += WAVES) {
    float Mc, Lc, A0, A1;
    if (count <= 16)
      fold_head_records<16>(pml, pac, count, lane, wb, Mc, Lc, A0, A1);
    else
      fold_head_records<32>(pml, pac, count, lane, wb, Mc, Lc, A0, A1);
    TP_STAMP(57);
    const float inv = __builtin_amdgcn_rcpf(Lc);
    *reinterpret_cast<uint32_t*>(out_rows) = pack_f2h2(A0 * inv, A1 * inv);
    pml += (int64_t)WAVES * Sp * 2;  // record_ml of head hh + WAVES
    pac += (int64_t)WAVES * S * kRecordAccStride;
    out_rows += WAVES * kHeadDim;
  }
}

template <int WAVES, int FL, class Merge>
__device__ __forceinline__ void combine_heads(Merge& sh, int wave, int lane, int nh, int S, int Sp, int count,
                                              const HeadRecords& hr) {
  float* wb = reinterpret_cast<float*>(&sh.acc[0][0]) + wave * 32;  // this wave's 32 weights
  // One full batch per head: straight-line code from the ticket to the
  // record loads.  Launches of exactly 16 splits (kFlBatch16, 4-wave
  // workgroups: 4k tokens) take the 16-record batch in a kernel of their own;
  // a second straight path in one kernel measured slower for the other.
  constexpr int kB = (FL & kFlBatch16) != 0 ? 16 : 32;
  if constexpr (WAVES == 8) {
    // 8-wave launches have at most 8 heads per block below GQA 16: one head
    // per wave (a loop here measured slower at the headline shape).
    if (nh <= WAVES && count == kB) {
      if (wave < nh) {
        float Mc = -INFINITY, Lc = 0.0f, A0 = 0.0f, A1 = 0.0f;
        fold_head_batch<kB, true>(hr.pml, hr.pac, 0, count, lane, wb, Mc, Lc, A0, A1);
        TP_STAMP(57);
        const float inv = __builtin_amdgcn_rcpf(Lc);
        *reinterpret_cast<uint32_t*>(hr.out) = pack_f2h2(A0 * inv, A1 * inv);
      }
      return;
    }
  } else if (count == kB) {
    // 4-wave launches carry up to 8 heads: two per wave at GQA 8.
    const float* pml = hr.pml;
    const uint16_t* pac = hr.pac;
    uint16_t* out_rows = hr.out;
    for (int hh = wave; hh < nh; hh += WAVES) {
      float Mc = -INFINITY, Lc = 0.0f, A0 = 0.0f, A1 = 0.0f;
      fold_head_batch<kB, true>(pml, pac, 0, count, lane, wb, Mc, Lc, A0, A1);
      TP_STAMP(57);
      const float inv = __builtin_amdgcn_rcpf(Lc);
      *reinterpret_cast<uint32_t*>(out_rows) = pack_f2h2(A0 * inv, A1 * inv);
      pml += (int64_t)WAVES * Sp * 2;  // record_ml of head hh + WAVES
      pac += (int64_t)WAVES * S * kRecordAccStride;
      out_rows += WAVES * kHeadDim;
    }
    return;
  }
  combine_head_rows<WAVES>(wb, wave, lane, nh, S, Sp, count, hr.pml, hr.pac, hr.out);
}

template <int WAVES, int FL, class Merge>
__device__ __forceinline__ void finish_merged(Merge& sh, const AttnArgs& a, int tid, int b, int kv, int h0, int nh,
                                              int64_t bkv, int hb, int split);

template <int WAVES, int FL = 0, class Merge>
__device__ __forceinline__ void finish_unit(Merge& sh, const AttnArgs& a, int wave, int tid, float m_run, float l_run,
                                            const float4v* acc, int b, int kv, int h0, int nh, int64_t bkv, int hb,
                                            int split) {
  const int lane = tid & 63;
  const int l16 = lane & 15;
  const int l4 = lane >> 4;
  const bool member = wave < WAVES;  // waves past WAVES hold no state and only keep the barriers
  // Merge the waves through LDS.
  const float l_tot = sum_rows(l_run);
  if (member && l4 == 0) sh.ml[wave][l16] = make_float2(m_run, l_tot);
  // The lane holds dims 32*l4 + 8*i + j (acc[j][i]) of head l16: eight 16-byte
  // writes of 4 consecutive dims each; with the 132-float row stride the 8
  // lanes of each write phase cover all banks once.
  float* arow = &sh.acc[member ? wave : 0][l16 * kRedStride + 32 * l4];
  if (member && l16 < nh) {  // rows of heads past the block's own hold nothing the fold reads
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int i = q >> 1, j0 = 4 * (q & 1);
      *reinterpret_cast<float4v*>(arow + 4 * q) = float4v{acc[j0][i], acc[j0 + 1][i], acc[j0 + 2][i], acc[j0 + 3][i]};
    }
  }
  finish_merged<WAVES, FL>(sh, a, tid, b, kv, h0, nh, bkv, hb, split);
}

// The rest of the end phase once every wave's state (sh.ml[w][h], sh.acc[w]
// rows of the live heads) is in LDS.  FL: end-phase variant flags (above).
template <int WAVES, int FL, class Merge>
__device__ __forceinline__ void finish_merged(Merge& sh, const AttnArgs& a, int tid, int b, int kv, int h0, int nh,
                                              int64_t bkv, int hb, int split) {
  lds_barrier();

  // Fold the waves' records: thread t owns dims 4 (t % 32) .. +3 of head
  // t / 32 and folds the WAVES records in wave order (one 16-byte LDS read per
  // record; spreading 4 heads over all 512 threads at one dim each was slower).
  const int h = tid >> 5;
  const int d0 = (tid & 31) << 2;
  const bool live = h < nh;
  float M = -INFINITY, L = 0.0f;
  float A[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (live) fold_waves(sh, h, d0, M, L, A);
  if (a.n_splits == 1) {
    if (live)
      store_out4(a.out + ((int64_t)b * a.hq + (int64_t)kv * a.g + h0 + h) * kHeadDim + d0, A,
                 __builtin_amdgcn_rcpf(L));
    return;
  }
  const int64_t unit = bkv * a.head_blocks + hb;
  const int S = a.n_splits;
  const int Sp = (S + 1) & ~1;  // (m, l) row length in pairs
  if (live) {
    if (d0 == 0) st_agent2(a.part_ml + record_ml(unit, h, Sp, split), M, L);
    st_agent_h4(a.part_acc + record_acc(unit, S, split, h) + d0, float4v{A[0], A[1], A[2], A[3]}, record_inv(L));
  }
  TP_STAMP(53);
  wait_stores();
  __syncthreads();
  TP_STAMP(54);
  // One tier: the unit's ticket counts its S splits.  Two tiers: the ticket
  // of the split's group counts the group's splits, and the group's combiner
  // then draws the unit's ticket, which counts the groups.
  constexpr bool kTiers = (FL & kFlTiers) != 0;
  const int T = kTiers ? a.tier_splits : 0;
  const int grp = T > 0 ? split / T : 0;
  const int first = grp * T;
  const int count = T > 0 ? min(T, S - first) : S;
  uint32_t* unit_ctr = a.counters + unit * a.counter_slots * a.counter_stride;
  uint32_t* ctr = T > 0 ? unit_ctr + (1 + grp) * a.counter_stride : unit_ctr;
  HeadRecords hr;
  if constexpr (!kTiers) {
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    hr.pml = a.part_ml + record_ml(unit, wave, Sp, 0);
    hr.pac = a.part_acc + record_acc(unit, S, 0, wave) + 2 * lane;
    hr.out = a.out + ((int64_t)b * a.hq + (int64_t)kv * a.g + h0 + wave) * kHeadDim + 2 * lane;
    asm volatile("" : : "s"(hr.pml), "v"(hr.pac), "v"(hr.out));  // computed here, before the ticket
  }
  if (tid == 0) sh.last = draw_ticket<FL>(ctr, (uint32_t)count);
  __syncthreads();
  TP_STAMP(55);
  if (!sh.last) return;
  TP_STAMP(64);

  // Last workgroup of this (b, kv, head block), or of its split group:
  // combine the records.
  if constexpr (!kTiers) {
    if (__builtin_expect(count <= kHeadCombineMax, 1)) {
      combine_heads<WAVES, FL>(sh, __builtin_amdgcn_readfirstlane(tid >> 6), tid & 63, nh, S, Sp, count, hr);
      if (tid == 0) __hip_atomic_store(unit_ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      TP_STAMP(56);
      return;
    }
  }
  const CombineItem ci = combine_item(tid, nh, WAVES);
  float Mc, Lc;
  Acc8 Ac;
  combine_records(sh, ci, a.part_ml, a.part_acc, unit, S, Sp, first, count, Mc, Lc, Ac);
  if constexpr (kTiers) {
    // Publish the group's record, then the unit's ticket over the groups.
    const int G = a.tier_groups;
    const int Gp = (G + 1) & ~1;
    if (ci.sg == 0 && ci.item) {
      if (ci.c8 == 0) st_agent2(a.tier_ml + record_ml(unit, ci.hh, Gp, grp), Mc, Lc);
      const float inv = record_inv(Lc);
      uint16_t* trow = a.tier_acc + record_acc(unit, G, grp, ci.hh) + 8 * ci.c8;
      st_agent_h4(trow, Ac.lo, inv);
      st_agent_h4(trow + 4, Ac.hi, inv);
    }
    wait_stores();
    __syncthreads();
    if (tid == 0) {
      __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sh.last = draw_ticket<FL>(unit_ctr, (uint32_t)G);
    }
    __syncthreads();
    if (!sh.last) return;
    combine_records(sh, ci, a.tier_ml, a.tier_acc, unit, G, Gp, 0, G, Mc, Lc, Ac);
  }
  TP_STAMP(58);
  if (ci.sg == 0 && ci.item) {
    const float inv = __builtin_amdgcn_rcpf(Lc);
    uint16_t* orow = a.out + ((int64_t)b * a.hq + (int64_t)kv * a.g + h0 + ci.hh) * kHeadDim + 8 * ci.c8;
    *reinterpret_cast<uint4*>(orow) = make_uint4(pack_f2h2(Ac.lo[0] * inv, Ac.lo[1] * inv),
                                                 pack_f2h2(Ac.lo[2] * inv, Ac.lo[3] * inv),
                                                 pack_f2h2(Ac.hi[0] * inv, Ac.hi[1] * inv),
                                                 pack_f2h2(Ac.hi[2] * inv, Ac.hi[3] * inv));
  }
  if (tid == 0) __hip_atomic_store(unit_ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  TP_STAMP(56);
}

// ---- decode attention kernel ---------------------------------------------------

template <int KIND, int WAVES, int FL = 0, int QJL = kQjlOff, bool DV = false>
__global__ __launch_bounds__(WAVES * 64) void decode_attention_kernel(AttnArgs a) {
  // The fold maps the threads onto heads x 128 dims at 4 dims per thread (512
  // threads: 16 heads, 256 threads: 8), and the combine sizes its split groups
  // for the thread count.  The host launches 4 waves only for head blocks of
  // at most 8 query heads.
  static_assert(WAVES == 8 || WAVES == 4, "decode_attention_kernel takes 4 or 8 waves per workgroup");
  // Half-row token order (kKindDefaultHR): the host launches it only for head
  // blocks of at most 8 query heads.
  constexpr bool HR = KIND == kKindDefaultHR;
  __shared__ AttnShared<WAVES> sh;
  TP_STAMP(0);
  // Every argument the prologue reads arrives in one round of scalar loads:
  // left to itself the compiler loaded the page pointers only after waiting
  // for the grid fields, a second round trip to fresh argument memory before
  // the first page request.
  asm volatile("" ::"s"(a.q), "s"(a.radii), "s"(a.angle_l1), "s"(a.angle_deep), "s"(a.v_codes), "s"(a.v_scales),
               "s"(a.capacity), "s"(a.pages_per_split), "s"(a.live_end), "s"(a.head_blocks), "s"(a.hkv), "s"(a.g),
               "s"(a.hq), "s"(a.div_head_blocks.m), "s"(a.div_head_blocks.sh));
  TP_STAMP(59);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches
  const int l16 = lane & 15;
  const int l4 = lane >> 4;
  const DecodeSlot ds = decode_slot(a);
  const int split = ds.split, b = ds.b, kv = ds.kv, hb = ds.hb;
  const int64_t bkv = ds.bkv;
  const int h0 = hb * 16;
  const int nh = min(16, a.g - h0);

  // Compressed pages of this split that hold at least one unmasked token.
  const int p_begin = split * a.pages_per_split;
  const int p_end = min(p_begin + a.pages_per_split, a.live_end);

  // Q and the first page's loads go out before the table build and the
  // barrier, and nothing before the barrier uses them.
  half8v qb[4];
  load_q<HR>(a, b, kv, h0, nh, l16, l4, qb);
  TP_STAMP(60);
  int page = p_begin + wave;
  KRegs<KIND> kr;
  // V: the page store's codes, or the dense V planes' rows (DV).
  typename std::conditional<DV, DenseVRegs, VRegs>::type vr;
  if constexpr (KIND == kKindGeneric) {  // also the launch for a call without pages
    if (page < p_end) {
      load_k<KIND>(a, bkv * a.capacity + page, l16, l4, kr);
      if constexpr (DV)
        load_v<HR>(a, bkv * a.v_capacity + page, l16, l4, lane, vr);
      else
        load_v<HR>(a, bkv * a.capacity + page, l16, l4, lane, vr);
    }
  } else {
    // The specialised layouts always have pages (p_begin < n_pages).  A wave
    // without a page of its own issues the same loads with every lane on the
    // first bytes of the split's first page (one cache line per load) instead
    // of branching around them: a load under a branch would make the
    // compiler's wait counting treat Q as the newest load, so every QK would
    // wait for all loads in flight.
    int p_load, lane_e;
    first_page_load(page, p_begin, p_end, lane, p_load, lane_e);
    load_k<KIND>(a, bkv * a.capacity + p_load, lane_e & 15, lane_e >> 4, kr);
    if constexpr (DV)
      load_v<HR>(a, bkv * a.v_capacity + p_load, lane_e & 15, lane_e >> 4, lane_e, vr);
    else
      load_v<HR>(a, bkv * a.capacity + p_load, lane_e & 15, lane_e >> 4, lane_e, vr);
  }
  TP_STAMP(1);
  if (tid < 256) build_lut<KIND>(sh.lut, a, tid);
  TP_STAMP(3);
  __shared__ float qjl_sin[QJL != kQjlOff ? kQjlMaxBits + 1 : 1];
  __shared__ uint32_t qjl_qw[QJL == kQjlAny ? 16 * kQjlMaxWords : 1];
  uint64_t qsig = 0;
  float qnorm = 0.0f;
  if constexpr (QJL != kQjlOff) {
    build_qjl_sin(qjl_sin, tid, a.qjl_bits);
    qjl_query<HR, QJL>(a, b, kv, h0, nh, l16, qb, qsig, qnorm);
    if constexpr (QJL == kQjlAny) qjl_query_words(a, b, kv, h0, nh, tid, qjl_qw);
  }
  lds_barrier();
  TP_STAMP(2);

  const int sbase4 = 4 * (2 * v_token(0, l4, 0, HR) + (l16 >> 3));
  const uint32_t ssel = (l16 & 4) ? 0x07060302u : 0x05040100u;
  float m_run = -INFINITY;
  float l_run = 0.0f;
  float4v acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

  // Per page: QK on the resident K codes, then the next page's K loads go out,
  // softmax and PV on the resident V codes, then the next page's V loads.
  // The wave's last page is peeled off, so the loads inside the loop are
  // unconditional and every wait covers only the loads it needs: QK waits for
  // the page's K codes while its V codes may still be in flight.  A page with
  // a successor is fully valid (only the last live page can be partial).
  for (int it = 0; page + WAVES < p_end; page += WAVES, ++it) {
    float4v s[4];
    qk_regs<KIND>(a, sh.lut, kr, qb, l16, l4, s);
    if constexpr (QJL == kQjl64) qjl_correct<HR>(a, bkv * a.qjl_capacity + page, l4, qsig, qnorm, qjl_sin, s);
    if constexpr (QJL == kQjlAny)
      qjl_correct_any<HR>(a, bkv * a.qjl_capacity + page, l4, qjl_qw, HR ? (l16 & 7) : l16, qnorm, qjl_sin, s);
    if (it < 12) TP_STAMP(4 + 4 * it);
    load_k<KIND>(a, bkv * a.capacity + page + WAVES, l16, l4, kr);
    half8v pb[2];
    softmax_page<HR>(s, kPageTokens, a.scale_log2, l4, m_run, l_run, acc, pb);
    pv_regs<HR>(vr, sbase4, ssel, pb, acc);
    if constexpr (DV)
      load_v<HR>(a, bkv * a.v_capacity + page + WAVES, l16, l4, lane, vr);
    else
      load_v<HR>(a, bkv * a.capacity + page + WAVES, l16, l4, lane, vr);
    if (it < 12) TP_STAMP(5 + 4 * it);
  }
  if (page < p_end) {
    float4v s[4];
    qk_regs<KIND>(a, sh.lut, kr, qb, l16, l4, s);
    if constexpr (QJL == kQjl64) qjl_correct<HR>(a, bkv * a.qjl_capacity + page, l4, qsig, qnorm, qjl_sin, s);
    if constexpr (QJL == kQjlAny)
      qjl_correct_any<HR>(a, bkv * a.qjl_capacity + page, l4, qjl_qw, HR ? (l16 & 7) : l16, qnorm, qjl_sin, s);
    const int valid = (int)min((int64_t)kPageTokens, a.seq_len - (int64_t)page * kPageTokens);
    half8v pb[2];
    softmax_page<HR>(s, valid, a.scale_log2, l4, m_run, l_run, acc, pb);
    if constexpr (DV) {
      // Dense V rows of masked tokens get P = 0, but 0 * NaN is NaN in the
      // MFMA: rows at or past `valid` are zeroed, so whatever a caller's
      // buffer holds there adds nothing (the reference skips those tokens in
      // its V sum, tqpolar_online_attention.metal:10-196).
      if (valid < kPageTokens) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            if (v_token(ks, l4, e, HR) >= valid) vr.w[8 * ks + e] = u32x4{0u, 0u, 0u, 0u};
          }
        }
      }
    }
    pv_regs<HR>(vr, sbase4, ssel, pb, acc);
  }

  // The dense tail follows the last page; the last split's least loaded wave
  // takes it (no QJL correction on the tail: metal.py:310-316 pads it with 0).
  if (split == a.n_splits - 1 && a.tail_len > 0) {
    const int n_local = max(p_end - p_begin, 0);
    if (wave == n_local % WAVES) {
      const int64_t tok0 = (int64_t)a.n_pages * kPageTokens;
      const int valid = (int)min((int64_t)a.tail_len, a.seq_len - tok0);
      if (valid > 0) {
        TailRegs tr;
        load_tail<HR>(a, bkv, l16, l4, tr);
        __builtin_amdgcn_sched_barrier(0);  // all 32 loads out before the first MFMA waits
        float4v s[4];
        qk_tail<HR>(tr, qb, s);
        half8v pb[2];
        softmax_page<HR>(s, valid, a.scale_log2, l4, m_run, l_run, acc, pb);
        pv_tail(tr, pb, acc);
      }
    }
  }

  TP_STAMP(52);
  finish_unit<WAVES, FL>(sh, a, wave, tid, m_run, l_run, acc, b, kv, h0, nh, bkv, hb, split);
}


// ---- standalone fused QK -----------------------------------------------------------

// Scores of one page leave through LDS: each wave writes its [16 heads][64
// tokens] fp16 block (row stride 72 halves) and reads it back as 16-byte
// chunks, eight lanes per head row, so every global store instruction writes
// whole 128-byte rows instead of 8-byte pieces of 16 rows.  One page per
// wave, eight waves per workgroup (measured against four and two: 8 is the
// fastest, by 0.05 us on the default layout and 0.25 us on the fast one at
// 512 pages x 8 kv heads).
constexpr int kQkRow = 72;  // halves per staged head row
constexpr int kQkWaves = 8;

template <int KIND, int QJL = kQjlOff>
__global__ __launch_bounds__(kQkWaves * 64) void fused_qk_kernel(AttnArgs a) {
  __shared__ Lut lut;
  __shared__ float qjl_sin[QJL != kQjlOff ? kQjlMaxBits + 1 : 1];
  __shared__ uint32_t qjl_qw[QJL == kQjlAny ? 16 * kQjlMaxWords : 1];
  __shared__ uint4 stage[kQkWaves][16 * kQkRow / 8];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches
  const int l16 = lane & 15;
  const int l4 = lane >> 4;
  const int64_t bkv = blockIdx.y;
  const int hb = blockIdx.z;
  const int b = (int)(bkv / a.hkv);
  const int kv = (int)(bkv - (int64_t)b * a.hkv);
  const int h0 = hb * 16;
  const int nh = min(16, a.g - h0);
  half8v qb[4];
  load_q<false>(a, b, kv, h0, nh, l16, l4, qb);
  // The page's K loads go out before the table build and the barrier (a wave
  // past the last page reloads the last page and leaves after the barrier).
  const int page = blockIdx.x * kQkWaves + wave;
  KRegs<KIND> kr;
  load_k<KIND>(a, bkv * a.capacity + min(page, a.n_pages - 1), l16, l4, kr);
  if (tid < 256) build_lut<KIND>(lut, a, tid);
  uint64_t qsig = 0;
  float qnorm = 0.0f;
  if constexpr (QJL != kQjlOff) {
    build_qjl_sin(qjl_sin, tid, a.qjl_bits);
    qjl_query<false, QJL>(a, b, kv, h0, nh, l16, qb, qsig, qnorm);
    if constexpr (QJL == kQjlAny) qjl_query_words(a, b, kv, h0, nh, tid, qjl_qw);
  }
  __syncthreads();
  if (page >= a.n_pages) return;
  float4v s[4];
  qk_regs<KIND>(a, lut, kr, qb, l16, l4, s);
  if constexpr (QJL == kQjl64) qjl_correct<false>(a, bkv * a.qjl_capacity + page, l4, qsig, qnorm, qjl_sin, s);
  if constexpr (QJL == kQjlAny) qjl_correct_any<false>(a, bkv * a.qjl_capacity + page, l4, qjl_qw, l16, qnorm, qjl_sin, s);
  uint16_t* st = reinterpret_cast<uint16_t*>(&stage[wave][0]);
  if (l16 < nh) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const uint32_t w0 = (uint32_t)f2h(s[mt][0] * a.scale) | ((uint32_t)f2h(s[mt][1] * a.scale) << 16);
      const uint32_t w1 = (uint32_t)f2h(s[mt][2] * a.scale) | ((uint32_t)f2h(s[mt][3] * a.scale) << 16);
      *reinterpret_cast<uint2*>(st + l16 * kQkRow + 16 * mt + 4 * l4) = make_uint2(w0, w1);
    }
  }
  wave_lds_sync();
  const int64_t row0 = ((int64_t)b * a.hq + (int64_t)kv * a.g + h0) * ((int64_t)a.n_pages * kPageTokens) +
                       (int64_t)page * kPageTokens;
#pragma unroll
  for (int r0 = 0; r0 < 16; r0 += 8) {
    const int h = r0 + (lane >> 3);
    const int c = lane & 7;
    if (h < nh)
      *reinterpret_cast<uint4*>(a.scores + row0 + (int64_t)h * a.n_pages * kPageTokens + 8 * c) =
          *reinterpret_cast<const uint4*>(st + h * kQkRow + 8 * c);
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

// Two-tier combine: above kTierMinSplits splits per unit, the splits form
// groups of kTierSplits whose last workgroup combines the group, and the last
// group combines the groups, so no workgroup folds more than max(kTierSplits,
// groups) records.  Measured (default splits): one kv head of 4 / 8 query
// heads at 131k, 256 splits, 21.75 -> 15.9 / 28.2 -> 16.9 us; 128 splits at
// 32k (1 or 2 kv heads) -10 %; at 64 splits (4 kv heads, 131k) one tier is
// 0.7 us faster; groups of 16 beat 8 and 32.  Every counter of both tiers
// must fit the fixed counter area; a shape whose counters would not keeps one
// tier.
constexpr int32_t kTierMinSplits = 64;
constexpr int32_t kTierSplits = 16;

struct Tiers {
  int32_t splits;  // splits per group (0: one tier)
  int32_t groups;
};

static Tiers tiers_of(int64_t units, int32_t n_splits) {
  Tiers t{0, 0};
  if (n_splits <= kTierMinSplits) return t;
  const int32_t groups = (n_splits + kTierSplits - 1) / kTierSplits;
  if ((size_t)units * (1 + groups) * sizeof(uint32_t) > kCounterArea) return t;
  t.splits = kTierSplits;
  t.groups = groups;
  return t;
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
        (need_v && ((uintptr_t)pages->v_scales & 3u))) {
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

// The fused QK kernel of a layout kind and QJL form.
template <int QJL>
static void launch_fused_qk(const AttnArgs& a, int kind, dim3 grid, hipStream_t s) {
  switch (kind) {
    case kKindDefault: hipLaunchKernelGGL((fused_qk_kernel<kKindDefault, QJL>), grid, dim3(kQkWaves * 64), 0, s, a); break;
    case kKindFast: hipLaunchKernelGGL((fused_qk_kernel<kKindFast, QJL>), grid, dim3(kQkWaves * 64), 0, s, a); break;
    default: hipLaunchKernelGGL((fused_qk_kernel<kKindGeneric, QJL>), grid, dim3(kQkWaves * 64), 0, s, a); break;
  }
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
  const size_t units = (size_t)batch * hkv * head_blocks_of(hq, hkv);
  return std::max(kCounterArea, align256(units * sizeof(uint32_t)));
}

size_t tp_decode_workspace_bytes(int64_t batch, int32_t hq, int32_t hkv, int32_t n_pages,
                                 int32_t tail_len, int32_t pages_per_split) {
  (void)tail_len;
  if (batch < 1 || hq < 1 || hkv < 1) return 0;
  if (pages_per_split <= 0) pages_per_split = tp_default_pages_per_split(batch, hq, hkv, n_pages);
  const size_t units = (size_t)batch * hkv * head_blocks_of(hq, hkv);
  const size_t splits = (size_t)n_splits_of(n_pages, pages_per_split);
  const size_t groups = (size_t)tiers_of((int64_t)units, (int32_t)splits).groups;
  return tp_decode_counter_bytes(batch, hq, hkv) + align256(units * 16 * ((splits + 1) & ~(size_t)1) * 2 * sizeof(float)) +
         align256(units * splits * 16 * kHeadDim * sizeof(uint16_t)) +
         align256(units * 16 * ((groups + 1) & ~(size_t)1) * 2 * sizeof(float)) +
         align256(units * groups * 16 * kHeadDim * sizeof(uint16_t));
}

int32_t tp_fused_qk(const void* q, int64_t batch, int32_t hq, int32_t hkv,
                    const tp_page_layout* layout, const tp_pages* pages, int32_t n_pages, float scale,
                    void* scores, void* stream) {
  clear_error();
  AttnArgs a{};
  if (!fill_common(a, q, batch, hq, hkv, layout, pages, n_pages, false)) return TP_ERR_INVALID;
  if (n_pages == 0) return TP_OK;
  if (!scores || ((uintptr_t)scores & 15u)) {
    set_error("scores must be a non-NULL 16-byte aligned buffer");
    return TP_ERR_INVALID;
  }
  a.scores = static_cast<uint16_t*>(scores);
  a.scale = scale;
  const dim3 grid((unsigned)((n_pages + kQkWaves - 1) / kQkWaves), (unsigned)(batch * hkv), (unsigned)a.head_blocks);
  hipStream_t s = static_cast<hipStream_t>(stream);
  launch_fused_qk<kQjlOff>(a, layout_kind(layout), grid, s);
  return launch_status("tp_fused_qk");
}

// Validates a tp_qjl against the pages and fills the kernel arguments.
static bool fill_qjl(AttnArgs& a, const tp_qjl* qjl, int32_t n_pages) {
  if (!qjl) {
    set_error("qjl_payload and q_proj_signs are required when use_qjl=True");
    return false;
  }
  const int P = qjl->proj_dim;
  if (P < 8 || P > kQjlMaxBits || P % 8 != 0) {
    set_error("QJL proj_dim must be a multiple of 8 from 8 to %d sketch bits, got %d", kQjlMaxBits, P);
    return false;
  }
  // P = 64 reads 16-byte sketch pairs, 8-byte norm quads and 8-byte query
  // sketches; any other P reads sketch dwords, fp16 norms and query bytes.
  const bool p64 = P == kQjlBits;
  if (!qjl->q_signs || (p64 && ((uintptr_t)qjl->q_signs & 7u)) ||
      (n_pages > 0 && (!qjl->signs || !qjl->norms || ((uintptr_t)qjl->signs & (p64 ? 15u : 3u)) ||
                       ((uintptr_t)qjl->norms & (p64 ? 7u : 1u))))) {
    set_error(p64 ? "QJL buffers missing or misaligned (sketches 16-byte, norms and query sketches 8-byte aligned)"
                  : "QJL buffers missing or misaligned (sketches 4-byte, norms 2-byte aligned)");
    return false;
  }
  if (n_pages > 0 && qjl->capacity < n_pages) {
    set_error("QJL sketch capacity %lld is below n_pages=%d", (long long)qjl->capacity, n_pages);
    return false;
  }
  a.qjl_capacity = qjl->capacity;
  a.qjl_signs = static_cast<const uint64_t*>(qjl->signs);
  a.qjl_norms = static_cast<const uint16_t*>(qjl->norms);
  a.q_signs = static_cast<const uint64_t*>(qjl->q_signs);
  a.qjl_bits = P;
  return true;
}

int32_t tp_fused_qk_qjl(const void* q, int64_t batch, int32_t hq, int32_t hkv, const tp_page_layout* layout,
                        const tp_pages* pages, int32_t n_pages, const tp_qjl* qjl, float scale, void* scores,
                        void* stream) {
  clear_error();
  AttnArgs a{};
  if (!fill_common(a, q, batch, hq, hkv, layout, pages, n_pages, false)) return TP_ERR_INVALID;
  if (!fill_qjl(a, qjl, n_pages)) return TP_ERR_INVALID;
  if (n_pages == 0) return TP_OK;
  if (!scores || ((uintptr_t)scores & 15u)) {
    set_error("scores must be a non-NULL 16-byte aligned buffer");
    return TP_ERR_INVALID;
  }
  a.scores = static_cast<uint16_t*>(scores);
  a.scale = scale;
  const dim3 grid((unsigned)((n_pages + kQkWaves - 1) / kQkWaves), (unsigned)(batch * hkv), (unsigned)a.head_blocks);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a.qjl_bits == kQjlBits)
    launch_fused_qk<kQjl64>(a, layout_kind(layout), grid, s);
  else
    launch_fused_qk<kQjlAny>(a, layout_kind(layout), grid, s);
  return launch_status("tp_fused_qk_qjl");
}

#ifdef TP_TIMELINE
// The measurement library's decode-kernel variants (tp_attention_measure.inc).
static int32_t g_measure_variant = 0;
static int32_t launch_measure_variant(const AttnArgs& a, dim3 grid, int kind, hipStream_t s);
#endif

}  // extern "C"

// tp_decode_attention and, with qjl, tp_decode_attention_qjl.
// The decode kernel of a layout kind, with the two-tier combine compiled in
// only for launches that use it.
// Plain (no QJL, quantised V) 4-wave launches of exactly 16 splits take the
// kernel whose combine is specialised for one batch of 16 records (kFlBatch16;
// paired: 4k 8.06 -> 7.90 us).
template <int KIND, int W, int QJL, bool DV = false>
static void launch_decode_w(const AttnArgs& a, dim3 grid, hipStream_t s) {
  const dim3 block(W * 64);
  if (a.tier_splits > 0) {
    hipLaunchKernelGGL((decode_attention_kernel<KIND, W, kFlTiers, QJL, DV>), grid, block, 0, s, a);
    return;
  }
  if constexpr (W == 4 && QJL == kQjlOff && !DV) {
    if (a.n_splits == 16) {
      hipLaunchKernelGGL((decode_attention_kernel<KIND, 4, kFlBatch16, kQjlOff, false>), grid, block, 0, s, a);
      return;
    }
  }
  hipLaunchKernelGGL((decode_attention_kernel<KIND, W, 0, QJL, DV>), grid, block, 0, s, a);
}

// A split of at most 4 pages leaves waves 4-7 of an 8-wave workgroup without
// a page (they still issue one cache line per page load and join every
// barrier); splits of 5-8 pages give each of 4 waves two pages instead of one
// page per wave.  Such launches take 4-wave workgroups when every head block
// has at most 8 query heads (the 4-wave fold and combine cover 8 heads):
// measured 15.28 -> 14.85 us for one kv head at 131k (8-page splits, two-tier
// combine), 13.12 -> 12.61 at 16k and 11.98 -> 11.41 at 12k (8 kv heads, 8-
// and 6-page splits), 13.10 -> 12.20 for batch 2 at 8k; longer splits stay on
// 8 waves (at 32k, 4-wave workgroups with 8-page splits took 20.68 us against
// 18.40 for the default 16-page splits on 8 waves).
static bool four_waves(const AttnArgs& a) { return a.g <= 8 && a.pages_per_split <= 8; }

// The decode kernel's kind for a layout kind: default-layout pages take the
// half-row token order when every head block has at most 8 query heads (its
// QK columns hold 8 heads x 2 halves).  Paired against the row order (same
// process, same caches, two sessions): 8 kv heads x 4 query heads at 4k 8.51 ->
// 8.32 and 8.63 -> 8.45 us; one kv head x 4 at 131k 14.41 -> 14.16; 8 x 8 at
// 32k 18.40 -> 18.30; 8 x 4 at 8k, 32k and 131k within 0.05 us either way.
// The 8-wave kernel's registers fall from 245 to 219 VGPRs.
static int decode_kind(int kind, const AttnArgs& a) { return kind == kKindDefault && a.g <= 8 ? kKindDefaultHR : kind; }

template <int KIND, int QJL>
static void launch_decode(const AttnArgs& a, dim3 grid, hipStream_t s) {
  if (four_waves(a))
    launch_decode_w<KIND, 4, QJL>(a, grid, s);
  else
    launch_decode_w<KIND, kDecodeWaves, QJL>(a, grid, s);
}

// The decode kernel of a decode kind (decode_kind) and QJL form.
template <int QJL>
static void launch_decode_kind(const AttnArgs& a, int kind, dim3 grid, hipStream_t s) {
  switch (kind) {
    case kKindDefaultHR: launch_decode<kKindDefaultHR, QJL>(a, grid, s); break;
    case kKindDefault: launch_decode<kKindDefault, QJL>(a, grid, s); break;
    case kKindFast: launch_decode<kKindFast, QJL>(a, grid, s); break;
    default: launch_decode<kKindGeneric, QJL>(a, grid, s); break;
  }
}

// Dense V (the reference's dense_v_debug storage) takes the same workgroup
// size rule as the quantised V pages.
template <int QJL>
static void launch_decode_dense_v(const AttnArgs& a, int kind, dim3 grid, hipStream_t s) {
  const bool w4 = four_waves(a);
  switch (decode_kind(kind, a)) {
    case kKindDefaultHR:
      if (w4)
        launch_decode_w<kKindDefaultHR, 4, QJL, true>(a, grid, s);
      else
        launch_decode_w<kKindDefaultHR, kDecodeWaves, QJL, true>(a, grid, s);
      break;
    case kKindDefault:
      if (w4)
        launch_decode_w<kKindDefault, 4, QJL, true>(a, grid, s);
      else
        launch_decode_w<kKindDefault, kDecodeWaves, QJL, true>(a, grid, s);
      break;
    case kKindFast:
      if (w4)
        launch_decode_w<kKindFast, 4, QJL, true>(a, grid, s);
      else
        launch_decode_w<kKindFast, kDecodeWaves, QJL, true>(a, grid, s);
      break;
    default:
      if (w4)
        launch_decode_w<kKindGeneric, 4, QJL, true>(a, grid, s);
      else
        launch_decode_w<kKindGeneric, kDecodeWaves, QJL, true>(a, grid, s);
      break;
  }
}

static int32_t decode_attention_impl(const void* q, int64_t batch, int32_t hq, int32_t hkv,
                                     const tp_page_layout* layout, const tp_pages* pages, int32_t n_pages,
                                     const tp_qjl* qjl, const void* tail_k, const void* tail_v, int32_t tail_len,
                                     int64_t tail_stride, int64_t actual_seq_len, float scale,
                                     int32_t pages_per_split, void* workspace, size_t workspace_bytes, void* out,
                                     void* stream, bool use_qjl, const void* v_dense = nullptr,
                                     int64_t v_capacity = 0) {
  clear_error();
  AttnArgs a{};
  if (!fill_common(a, q, batch, hq, hkv, layout, pages, n_pages, v_dense == nullptr)) return TP_ERR_INVALID;
  if (use_qjl && !fill_qjl(a, qjl, n_pages)) return TP_ERR_INVALID;
  if (v_dense) {
    if (((uintptr_t)v_dense & 15u) || v_capacity < n_pages) {
      set_error("dense V must be 16-byte aligned with v_capacity >= n_pages (got %lld < %d)", (long long)v_capacity,
                n_pages);
      return TP_ERR_INVALID;
    }
    a.v_codes = nullptr;
    a.v_scales = nullptr;
    a.v_dense = static_cast<const uint16_t*>(v_dense);
    a.v_capacity = v_capacity;
  }
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
  // The reference masks tokens at or past actual_seq_len and accepts a length
  // beyond the stored tokens (tqpolar_online_attention.metal:474; metal.py:318),
  // so a longer length attends every stored token.  A length below 1 would
  // mask everything (the reference's softmax then returns NaN): rejected.
  const int64_t total = (int64_t)n_pages * kPageTokens + tail_len;
  if (actual_seq_len < 1) {
    set_error("actual_seq_len=%lld must be at least 1", (long long)actual_seq_len);
    return TP_ERR_INVALID;
  }
  if (actual_seq_len > total) actual_seq_len = total;
  if (pages_per_split <= 0) pages_per_split = tp_default_pages_per_split(batch, hq, hkv, n_pages);
  const int32_t n_splits = n_splits_of(n_pages, pages_per_split);
  // The grid is (hkv, batch * head_blocks, n_splits); y and z are at most 65535.
  const int64_t n_rows = (int64_t)batch * a.head_blocks;
  if (n_splits > 65535 || n_rows > 65535) {
    set_error("grid (%d, %lld, %d) exceeds the grid limit of 65535 in y and z%s", hkv, (long long)n_rows,
              n_splits, n_splits > 65535 ? "; raise pages_per_split" : "");
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
  a.live_end = (int32_t)std::min<int64_t>(n_pages, (actual_seq_len + kPageTokens - 1) / kPageTokens);
  a.div_head_blocks = make_fastdiv((uint32_t)a.head_blocks);
  if (n_splits > 1) {
    const size_t need = tp_decode_workspace_bytes(batch, hq, hkv, n_pages, tail_len, pages_per_split);
    if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255u)) {
      set_error("workspace of %zu bytes (256-byte aligned) required, got %zu", need, workspace_bytes);
      return TP_ERR_WORKSPACE;
    }
    const size_t units = (size_t)batch * hkv * a.head_blocks;
    const Tiers tiers = tiers_of((int64_t)units, n_splits);
    a.tier_splits = tiers.splits;
    a.tier_groups = tiers.groups;
    a.counter_slots = 1 + tiers.groups;
    char* ws = static_cast<char*>(workspace);
    a.counters = reinterpret_cast<uint32_t*>(ws);
    a.counter_stride = counter_stride_of((int64_t)units * a.counter_slots);
    ws += tp_decode_counter_bytes(batch, hq, hkv);
    a.part_ml = reinterpret_cast<float*>(ws);
    ws += align256(units * 16 * (((size_t)n_splits + 1) & ~(size_t)1) * 2 * sizeof(float));
    a.part_acc = reinterpret_cast<uint16_t*>(ws);
    ws += align256(units * (size_t)n_splits * 16 * kHeadDim * sizeof(uint16_t));
    a.tier_ml = reinterpret_cast<float*>(ws);
    ws += align256(units * 16 * (((size_t)tiers.groups + 1) & ~(size_t)1) * 2 * sizeof(float));
    a.tier_acc = reinterpret_cast<uint16_t*>(ws);
  }
  const dim3 grid((unsigned)hkv, (unsigned)n_rows, (unsigned)n_splits);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (v_dense) {
    const int kind = layout_kind(layout);
    if (!use_qjl)
      launch_decode_dense_v<kQjlOff>(a, kind, grid, s);
    else if (a.qjl_bits == kQjlBits)
      launch_decode_dense_v<kQjl64>(a, kind, grid, s);
    else
      launch_decode_dense_v<kQjlAny>(a, kind, grid, s);
    return launch_status("tp_decode_attention_dense_v");
  }
  if (use_qjl) {
    const int kind = n_pages > 0 ? decode_kind(layout_kind(layout), a) : (int)kKindGeneric;
    if (a.qjl_bits == kQjlBits)
      launch_decode_kind<kQjl64>(a, kind, grid, s);
    else
      launch_decode_kind<kQjlAny>(a, kind, grid, s);
    return launch_status("tp_decode_attention_qjl");
  }
#ifdef TP_TIMELINE
  if (g_measure_variant != 0) {
    // The measurement variants combine in one tier (any split count).
    a.tier_splits = 0;
    a.tier_groups = 0;
    return launch_measure_variant(a, grid, n_pages > 0 ? layout_kind(layout) : -1, s);
  }
#endif
  launch_decode_kind<kQjlOff>(a, n_pages > 0 ? decode_kind(layout_kind(layout), a) : (int)kKindGeneric, grid, s);
  return launch_status("tp_decode_attention");
}

extern "C" {

int32_t tp_decode_attention(const void* q, int64_t batch, int32_t hq, int32_t hkv,
                            const tp_page_layout* layout, const tp_pages* pages, int32_t n_pages,
                            const void* tail_k, const void* tail_v, int32_t tail_len,
                            int64_t tail_stride, int64_t actual_seq_len, float scale,
                            int32_t pages_per_split, void* workspace, size_t workspace_bytes,
                            void* out, void* stream) {
  return decode_attention_impl(q, batch, hq, hkv, layout, pages, n_pages, nullptr, tail_k, tail_v, tail_len,
                               tail_stride, actual_seq_len, scale, pages_per_split, workspace, workspace_bytes, out,
                               stream, false);
}

int32_t tp_decode_attention_qjl(const void* q, int64_t batch, int32_t hq, int32_t hkv,
                                const tp_page_layout* layout, const tp_pages* pages, int32_t n_pages,
                                const tp_qjl* qjl, const void* tail_k, const void* tail_v, int32_t tail_len,
                                int64_t tail_stride, int64_t actual_seq_len, float scale,
                                int32_t pages_per_split, void* workspace, size_t workspace_bytes,
                                void* out, void* stream) {
  return decode_attention_impl(q, batch, hq, hkv, layout, pages, n_pages, qjl, tail_k, tail_v, tail_len,
                               tail_stride, actual_seq_len, scale, pages_per_split, workspace, workspace_bytes, out,
                               stream, true);
}

int32_t tp_decode_attention_dense_v(const void* q, int64_t batch, int32_t hq, int32_t hkv,
                                    const tp_page_layout* layout, const tp_pages* pages, int32_t n_pages,
                                    const tp_qjl* qjl, const void* v_dense, int64_t v_capacity,
                                    int64_t actual_seq_len, float scale, int32_t pages_per_split, void* workspace,
                                    size_t workspace_bytes, void* out, void* stream) {
  if (n_pages < 1 || !v_dense) {
    clear_error();
    set_error("tp_decode_attention_dense_v needs pages and their dense V");
    return TP_ERR_INVALID;
  }
  return decode_attention_impl(q, batch, hq, hkv, layout, pages, n_pages, qjl, nullptr, nullptr, 0, 0,
                               actual_seq_len, scale, pages_per_split, workspace, workspace_bytes, out, stream,
                               qjl != nullptr, v_dense, v_capacity);
}

}  // extern "C"

// ---- host-side bounds check of the decode kernels' memory accesses ----------------------
//
// tp_selftest_decode_bounds enumerates, for every workgroup, wave and lane of
// one launch, the byte range of every global load and store of
// decode_attention_kernel (or fused_qk_kernel) from the address functions
// the kernels themselves use (k_radii_base ... record_acc, first_page_load,
// combine_item, fold_record), and counts the ranges outside their buffers.
// Buffers take the smallest sizes the C ABI admits for the shape: page fields
// of `capacity` slots per (batch, kv head), the dense tail ending right after
// the last row's tail_len tokens, the workspace of tp_decode_workspace_bytes.
// Loads through bounded raw buffer resources (q, the dense tail) are checked
// by their resource's range.  No GPU work.

namespace {

struct BoundsLog {
  unsigned long long bad = 0;
  unsigned long long checked = 0;
  char first[512] = {0};
  void check(const char* what, int64_t off, int64_t bytes, int64_t size, int lin, int wave, int lane) {
    ++checked;
    if (off >= 0 && off + bytes <= size) return;
    if (!bad)
      snprintf(first, sizeof(first), "%s: bytes [%lld, %lld) outside a %lld-byte buffer (workgroup %d, wave %d, lane %d)",
               what, (long long)off, (long long)(off + bytes), (long long)size, lin, wave, lane);
    ++bad;
  }
};

}  // namespace

extern "C" unsigned long long tp_selftest_decode_bounds(const tp_bounds_case* c, char* msg, int32_t msg_len) {
  BoundsLog log;
  if (msg && msg_len > 0) msg[0] = 0;
  int l1_row = 0, deep_row = 0;
  if (!c || !check_layout(&c->layout, &l1_row, &deep_row) || c->batch < 1 || c->hq < 1 || c->hkv < 1 ||
      c->hq % c->hkv || c->n_pages < 1 || c->capacity < c->n_pages || c->seq_len < 1) {
    if (msg && msg_len > 0) snprintf(msg, msg_len, "bad case");
    return ~0ull;
  }
  const int kind = layout_kind(&c->layout);
  const int64_t BH = c->batch * c->hkv;
  const int g = c->hq / c->hkv;
  AttnArgs ka{};
  ka.g = g;
  const int dkind = decode_kind(kind, ka);  // the decode kernel's kind (the fused QK kernel takes `kind`)
  const bool hr = dkind == kKindDefaultHR;
  const int head_blocks = head_blocks_of(c->hq, c->hkv);
  const int n_pages = c->n_pages;
  const int64_t cap = c->capacity;
  const bool int8r = c->layout.int8_radii != 0;
  const int pps = c->pages_per_split > 0 ? c->pages_per_split
                                         : tp_default_pages_per_split(c->batch, c->hq, c->hkv, n_pages);
  const int S = n_splits_of(n_pages, pps);
  const int64_t units = BH * head_blocks;
  const int64_t total = (int64_t)n_pages * kPageTokens + c->tail_len;
  const int64_t seq = std::min(c->seq_len, total);
  // Buffer sizes in bytes.
  const int64_t sz_q = c->batch * c->hq * kHeadDim * 2;
  const int64_t sz_out = sz_q;
  const int64_t sz_radii = BH * cap * kPageTokens * kPairs * (int8r ? 1 : 2);
  const int64_t sz_rs = BH * cap * 2;
  const int64_t sz_l1 = BH * cap * kPageTokens * l1_row;
  const int64_t sz_deep = BH * cap * kPageTokens * deep_row;
  const int64_t sz_vc = BH * cap * kPageTokens * kHeadDim;
  const int64_t sz_vs = BH * cap * kPageTokens * kVGroups * 2;
  const int64_t sz_dv = BH * c->v_capacity * kPageTokens * kHeadDim * 2;
  const int64_t sz_tail = c->tail_len > 0 ? ((BH - 1) * c->tail_stride + c->tail_len) * kHeadDim * 2 : 0;
  const int qjl_p = c->qjl_bits > 0 ? c->qjl_bits : kQjlBits;  // sketch bits
  const int qjl_nb = qjl_p / 8;                                  // sketch bytes per token and query head
  const int64_t sz_sig = BH * c->qjl_capacity * kPageTokens * qjl_nb;
  const int64_t sz_nrm = BH * c->qjl_capacity * kPageTokens * 2;
  const int64_t sz_qs = c->batch * c->hq * qjl_nb;

  // One lane's loads of page `page` (lane addresses of lane_e), as the kernels issue them.
  auto page_loads = [&](int lin, int wave, int lane, int64_t bkv, int page, int lane_e) {
    const int64_t slot = bkv * cap + page;
    const int l16 = lane_e & 15, l4 = lane_e >> 4;
    if (dkind == kKindDefaultHR) {
      for (int g8 = 0; g8 < 8; ++g8) {
        log.check("radii", hr_radii_base(slot, l16, l4) + hr_radii_row(g8), 16, sz_radii, lin, wave, lane);
        log.check(hr_code_from_l1(l16) ? "angle_l1" : "angle_deep", hr_code_base(slot, l16, l4) + hr_code_row(g8), 4,
                  hr_code_from_l1(l16) ? sz_l1 : sz_deep, lin, wave, lane);
      }
    } else if (dkind == kKindDefault) {
      for (int mt = 0; mt < 4; ++mt) {
        const int t = 16 * mt + l16;
        log.check("radii", k_radii_base(slot, l4) + k_radii_row(t), 32, sz_radii, lin, wave, lane);
        log.check(k_code_from_l1(l4) ? "angle_l1" : "angle_deep", k_code_base(slot, l4) + k_code_row(t), 8,
                  k_code_from_l1(l4) ? sz_l1 : sz_deep, lin, wave, lane);
      }
    } else if (kind == kKindFast) {
      for (int mt = 0; mt < 4; ++mt) {
        const int t = 16 * mt + l16;
        log.check("radii", fast_base(slot, l4) + fast_row(t), 16, sz_radii, lin, wave, lane);
        log.check("angle_deep", fast_base(slot, l4) + fast_row(t), 16, sz_deep, lin, wave, lane);
      }
      log.check("radii_scales", fast_scale(slot), 2, sz_rs, lin, wave, lane);
    }
    if (c->dense_v) {
      for (int ks = 0; ks < 2; ++ks)
        for (int e = 0; e < 8; ++e)
          log.check("dense V", dense_v_base(bkv * c->v_capacity + page, l16) + dense_v_row(ks, l4, e, hr), 16, sz_dv, lin,
                    wave, lane);
    } else {
      for (int ks = 0; ks < 2; ++ks)
        for (int e = 0; e < 8; ++e)
          log.check("v_codes", v_code_base(slot, l16) + v_code_row(ks, l4, e, hr), 8, sz_vc, lin, wave, lane);
      const int64_t sb = v_scale_base(slot);
      log.check("v_scales", sb + 4 * lane_e, 4, sz_vs, lin, wave, lane);
      log.check("v_scales", sb + 4 * (lane_e + 64) + (c->mutate == 1 ? 512 : 0), 4, sz_vs, lin, wave, lane);
    }
  };
  // The generic layout's codes, gathered during the math of a page it owns.
  auto generic_loads = [&](int lin, int wave, int lane, int64_t bkv, int page) {
    const int64_t slot = bkv * cap + page;
    const int l16 = lane & 15, l4 = lane >> 4;
    const int split_half = c->layout.split_dim / 2;
    if (int8r) log.check("radii_scales", slot * 2, 2, sz_rs, lin, wave, lane);
    for (int mt = 0; mt < 4; ++mt) {
      const int64_t row = slot * kPageTokens + 16 * mt + l16;
      for (int kk = 0; kk < 4; ++kk)
        for (int i = 0; i < 4; ++i) {
          const int p = 16 * l4 + 4 * kk + i;
          log.check("radii", (row * kPairs + p) * (int8r ? 1 : 2), int8r ? 1 : 2, sz_radii, lin, wave, lane);
          if (p < split_half)
            log.check("angle_l1", row * l1_row + (p * c->layout.l1_bits) / 8, 1, sz_l1, lin, wave, lane);
          else
            log.check("angle_deep", row * deep_row + ((p - split_half) * c->layout.deep_bits) / 8, 1, sz_deep, lin, wave,
                      lane);
        }
    }
  };

  if (c->kernel == 1) {  // fused_qk_kernel: one page per wave, the last page reloaded past n_pages
    const int gx = (n_pages + kQkWaves - 1) / kQkWaves;
    for (int64_t bkv = 0; bkv < BH; ++bkv)
      for (int hb = 0; hb < head_blocks; ++hb)
        for (int bx = 0; bx < gx; ++bx)
          for (int wave = 0; wave < kQkWaves; ++wave)
            for (int lane = 0; lane < 64; ++lane) {
              const int page = bx * kQkWaves + wave;
              const int b = (int)(bkv / c->hkv), kv = (int)(bkv % c->hkv), h0 = hb * 16, nh = std::min(16, g - h0);
              const int lin = (int)((bkv * head_blocks + hb) * gx + bx);
              log.check("q (buffer range)", ((int64_t)b * c->hq + (int64_t)kv * g + h0) * kHeadDim * 2,
                        (int64_t)nh * kHeadDim * 2, sz_q, lin, wave, lane);
              if (kind != kKindGeneric) {
                const int64_t slot_page = std::min(page, n_pages - 1);
                const int l16 = lane & 15, l4 = lane >> 4;
                const int64_t slot = bkv * cap + slot_page;
                for (int mt = 0; mt < 4; ++mt) {
                  const int t = 16 * mt + l16;
                  if (kind == kKindDefault) {
                    log.check("radii", k_radii_base(slot, l4) + k_radii_row(t), 32, sz_radii, lin, wave, lane);
                    log.check("angle codes", k_code_base(slot, l4) + k_code_row(t), 8,
                              k_code_from_l1(l4) ? sz_l1 : sz_deep, lin, wave, lane);
                  } else {
                    log.check("radii", fast_base(slot, l4) + fast_row(t), 16, sz_radii, lin, wave, lane);
                    log.check("angle_deep", fast_base(slot, l4) + fast_row(t), 16, sz_deep, lin, wave, lane);
                  }
                }
              } else if (page < n_pages) {
                generic_loads(lin, wave, lane, bkv, page);
              }
              if (page < n_pages) {
                const int64_t sz_scores = c->batch * c->hq * (int64_t)n_pages * kPageTokens * 2;
                for (int r0 = 0; r0 < 16; r0 += 8) {
                  const int h = r0 + (lane >> 3), cc = lane & 7;
                  if (h < nh)
                    log.check("scores",
                              ((((int64_t)b * c->hq + (int64_t)kv * g + h0) * n_pages * kPageTokens +
                                (int64_t)page * kPageTokens) + (int64_t)h * n_pages * kPageTokens + 8 * cc) * 2,
                              16, sz_scores, lin, wave, lane);
                }
              }
            }
  } else {  // decode_attention_kernel
    AttnArgs a{};
    a.g = g;
    a.pages_per_split = pps;
    const int waves = four_waves(a) ? 4 : kDecodeWaves;
    const Tiers tiers = S > 1 ? tiers_of(units, S) : Tiers{0, 0};
    const int slots = 1 + tiers.groups;
    const int32_t cstride = counter_stride_of(units * slots);
    const int64_t sz_ws = S > 1 ? (int64_t)tp_decode_workspace_bytes(c->batch, c->hq, c->hkv, n_pages, c->tail_len, pps) : 0;
    const int64_t cbytes = (int64_t)tp_decode_counter_bytes(c->batch, c->hq, c->hkv);
    const int Sp = (S + 1) & ~1;
    const int64_t ml_off = cbytes;
    const int64_t acc_off = ml_off + (int64_t)align256(units * 16 * Sp * 2 * sizeof(float));
    const int64_t tml_off = acc_off + (int64_t)align256(units * S * 16 * kHeadDim * 2);
    const int G = tiers.groups;
    const int Gp = (G + 1) & ~1;
    const int64_t tacc_off = tml_off + (int64_t)align256(units * 16 * Gp * 2 * sizeof(float));
    const int64_t live_pages = (seq + kPageTokens - 1) / kPageTokens;
    // The combine of records first .. first+count-1 of an area, by every thread of one workgroup.
    auto combine_loads = [&](int lin, int64_t unit, int nh, int64_t mlb, int64_t acb, int S_area, int Sp_area,
                             int first, int count) {
      for (int tid = 0; tid < waves * 64; ++tid) {
        const CombineItem ci = combine_item(tid, nh, waves);
        const int SG = 1 << ci.lsg;
        const int mine = ci.item ? (count - ci.sg + SG - 1) >> ci.lsg : 0;
        const int B = ((count + SG - 1) >> ci.lsg) <= 4 ? 4 : 8;
        const int lane = tid & 63;
        for (int r0 = 0; r0 < mine; r0 += B) {
          log.check("records (m, l)",
                    mlb + (record_ml(unit, ci.hh, Sp_area, first + ci.sg) + 2 * SG * fold_record(r0, lane & (B - 1), mine)) * 4,
                    8, sz_ws, lin, tid >> 6, lane);
          for (int u = 0; u < B; ++u)
            log.check("records o",
                      acb + (record_acc(unit, S_area, first + ci.sg, ci.hh) + 8 * ci.c8 +
                             (int64_t)fold_record(r0, u, mine) * SG * kRecordAccStride) * 2,
                      16, sz_ws, lin, tid >> 6, lane);
        }
      }
    };
    for (int64_t lin = 0; lin < (int64_t)S * units; ++lin) {
      const int split = (int)(lin / units);
      const int64_t unit = lin % units;
      const int64_t bkv = unit / head_blocks;
      const int hb = (int)(unit % head_blocks);
      const int b = (int)(bkv / c->hkv), kv = (int)(bkv % c->hkv);
      const int h0 = hb * 16, nh = std::min(16, g - h0);
      const int p_begin = split * pps;
      const int p_end = (int)std::min<int64_t>(std::min(p_begin + pps, n_pages), live_pages);
      const int L = (int)lin;
      for (int wave = 0; wave < waves; ++wave)
        for (int lane = 0; lane < 64; ++lane) {
          const int l16 = lane & 15;
          log.check("q (buffer range)", ((int64_t)b * c->hq + (int64_t)kv * g + h0) * kHeadDim * 2,
                    (int64_t)nh * kHeadDim * 2, sz_q, L, wave, lane);
          int page = p_begin + wave;
          if (kind == kKindGeneric) {
            for (; page < p_end; page += waves) {
              generic_loads(L, wave, lane, bkv, page);
              page_loads(L, wave, lane, bkv, page, lane);
            }
          } else {
            int p_load, lane_e;
            first_page_load(page, p_begin, p_end, lane, p_load, lane_e);
            if (c->mutate == 2 && page >= p_end) p_load = p_begin + pps;  // the no-page load moved one split on
            page_loads(L, wave, lane, bkv, p_load, lane_e);
            for (; page + waves < p_end; page += waves) page_loads(L, wave, lane, bkv, page + waves, lane);
          }
          if (c->qjl) {
            for (int pg = p_begin + wave; pg < p_end; pg += waves) {
              const int64_t qslot = bkv * c->qjl_capacity + pg;
              const int l4 = lane >> 4;
              for (int mt = 0; mt < 4; ++mt) {
                if (qjl_p != kQjlBits) {  // qjl_correct_any: the dwords covering each token's sketch
                  for (int i = 0; i < 4; ++i) {
                    const int t = score_token(mt, i, l4, hr);
                    const int64_t o = qjl_any_row(qslot, t, qjl_nb);
                    const int sh = (int)(o & 3);
                    log.check("qjl signs", o - sh, 4 * qjl_any_dwords(sh, qjl_nb), sz_sig, L, wave, lane);
                    log.check("qjl norms", (qslot * kPageTokens + t) * 2, 2, sz_nrm, L, wave, lane);
                  }
                } else if (hr) {
                  for (int j = 0; j < 2; ++j) {
                    log.check("qjl signs", qjl_sign_base(qslot, l4, true) + 128 * mt + 64 * j, 16, sz_sig, L, wave, lane);
                    log.check("qjl norms", qjl_norm_base(qslot, l4, true) + 32 * mt + 16 * j, 4, sz_nrm, L, wave, lane);
                  }
                } else {
                  log.check("qjl signs", qjl_sign_base(qslot, l4) + 128 * mt, 32, sz_sig, L, wave, lane);
                  log.check("qjl norms", qjl_norm_base(qslot, l4) + 32 * mt, 8, sz_nrm, L, wave, lane);
                }
              }
            }
            if (qjl_p == kQjlBits) {
              log.check("q signs", ((int64_t)b * c->hq + (int64_t)kv * g + h0 + std::min(l16, nh - 1)) * 8, 8, sz_qs,
                        L, wave, lane);
            } else {  // qjl_query_words: thread t < 16 * kQjlMaxWords reads bytes 4w .. of head t / kQjlMaxWords
              const int tid = wave * 64 + lane;
              const int h = tid / kQjlMaxWords, w = tid % kQjlMaxWords;
              if (tid < 16 * kQjlMaxWords && h < nh)
                for (int j = 0; j < 4; ++j)
                  if (4 * w + j < qjl_nb)
                    log.check("q signs", ((int64_t)b * c->hq + (int64_t)kv * g + h0 + h) * qjl_nb + 4 * w + j, 1,
                              sz_qs, L, wave, lane);
            }
          }
          if (split == S - 1 && c->tail_len > 0 && wave == std::max(p_end - p_begin, 0) % waves &&
              std::min<int64_t>(c->tail_len, seq - (int64_t)n_pages * kPageTokens) > 0)
            log.check("tail (buffer range)", bkv * c->tail_stride * kHeadDim * 2, (int64_t)c->tail_len * kHeadDim * 2,
                      sz_tail, L, wave, lane);
        }
      // The fold's record (or, with one split, output) stores: thread t, head t/32, dims 4(t%32)..+3.
      for (int tid = 0; tid < waves * 64; ++tid) {
        const int h = tid >> 5, d0 = (tid & 31) << 2;
        if (h >= nh) continue;
        if (S == 1) {
          log.check("out", (((int64_t)b * c->hq + (int64_t)kv * g + h0 + h) * kHeadDim + d0) * 2, 8, sz_out, L, tid >> 6,
                    tid & 63);
          continue;
        }
        if (d0 == 0) log.check("record (m, l)", ml_off + record_ml(unit, h, Sp, split) * 4, 8, sz_ws, L, tid >> 6, tid & 63);
        log.check("record o", acc_off + (record_acc(unit, S, split, h) + d0) * 2, 8, sz_ws, L, tid >> 6, tid & 63);
      }
      if (S > 1) {
        const int T = tiers.splits;
        const int grp = T > 0 ? split / T : 0;
        const int64_t ctr = unit * slots * cstride;
        log.check("ticket", (ctr + (T > 0 ? (1 + grp) * cstride : 0)) * 4, 4, cbytes, L, 0, 0);
        const bool group_last = T > 0 ? split == std::min(S, (grp + 1) * T) - 1 : split == S - 1;
        if (group_last) {  // any workgroup may combine; its loads are the same, so check once per group
          const int first = grp * T;
          const int count = T > 0 ? std::min(T, S - first) : S;
          if (T == 0 && count <= kHeadCombineMax) {
            // combine_heads: wave w takes heads w, w + waves, ...; lane l dims 2l, 2l + 1; batches of B records.
            for (int hh = 0; hh < nh; ++hh)
              for (int lane = 0; lane < 64; ++lane) {
                const int wave = hh % waves;
                const int B = count <= 16 ? 16 : 32;
                for (int r0 = 0; r0 < count; r0 += B) {
                  const int rj = std::min(r0 + (lane & (B - 1)), count - 1);
                  log.check("records (m, l)", ml_off + (record_ml(unit, hh, Sp, 0) + 2 * rj) * 4, 8, sz_ws, L, wave,
                            lane);
                  for (int j = 0; j < B; ++j)
                    log.check("records o",
                              acc_off + (record_acc(unit, S, 0, hh) + 2 * lane +
                                         (int64_t)std::min(r0 + j, count - 1) * kRecordAccStride) * 2,
                              4, sz_ws, L, wave, lane);
                }
                log.check("out", (((int64_t)b * c->hq + (int64_t)kv * g + h0 + hh) * kHeadDim + 2 * lane) * 2, 4,
                          sz_out, L, wave, lane);
              }
            continue;
          }
          combine_loads(L, unit, nh, ml_off, acc_off, S, Sp, first, count);
          if (T > 0) {
            for (int tid = 0; tid < waves * 64; ++tid) {
              const CombineItem ci = combine_item(tid, nh, waves);
              if (ci.sg != 0 || !ci.item) continue;
              if (ci.c8 == 0)
                log.check("group record (m, l)", tml_off + record_ml(unit, ci.hh, Gp, grp) * 4, 8, sz_ws, L, tid >> 6,
                          tid & 63);
              log.check("group record o", tacc_off + (record_acc(unit, G, grp, ci.hh) + 8 * ci.c8) * 2, 16, sz_ws, L,
                        tid >> 6, tid & 63);
            }
            log.check("unit ticket", ctr * 4, 4, cbytes, L, 0, 0);
            if (grp == G - 1) combine_loads(L, unit, nh, tml_off, tacc_off, G, Gp, 0, G);
          }
          for (int tid = 0; tid < waves * 64; ++tid) {
            const CombineItem ci = combine_item(tid, nh, waves);
            if (ci.sg == 0 && ci.item)
              log.check("out", (((int64_t)b * c->hq + (int64_t)kv * g + h0 + ci.hh) * kHeadDim + 8 * ci.c8) * 2, 16,
                        sz_out, L, tid >> 6, tid & 63);
          }
        }
      }
    }
  }
  if (msg && msg_len > 0) snprintf(msg, msg_len, "%s", log.first);
  return log.bad;
}

// ---- entry point that allocates nothing -----------------------------------------
//
// tp_decode_attention_noalloc keeps its split-K records and ticket counters in
// `scratch`, a file-scope device array (kScratchBytes per GPU, held for the
// life of the process), instead of a caller-provided workspace.  Host code
// never passes the array's name to a kernel or a copy: the name is a host-side
// stand-in.  Its device address is taken once per device with
// hipGetSymbolAddress, with that device current, and kept per device.

namespace tp {

constexpr size_t kScratchBytes = TP_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device

__global__ __launch_bounds__(256) void clear_words_kernel(uint32_t* p, uint32_t n) {
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < n; i += gridDim.x * 256u) p[i] = 0u;
}

// Device address of `scratch` on the device of `stream`.  The first call on a
// device looks it up and clears the ticket-counter area with a fill kernel on
// `stream` (a kernel, not a memset node, so the call can sit inside a captured
// graph); every decode launch leaves the counters zero again.
static int32_t scratch_of(hipStream_t stream, size_t counter_bytes, void** out) {
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("tp_decode_attention_noalloc: cannot resolve the stream's device (%s)", hipGetErrorString(e));
    return TP_ERR_HIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) {
      set_error("tp_decode_attention_noalloc: hipGetDevice failed");
      return TP_ERR_HIP;
    }
    if (cur != dev && hipSetDevice(dev) != hipSuccess) {
      set_error("tp_decode_attention_noalloc: hipSetDevice(%d) failed", dev);
      return TP_ERR_HIP;
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess && p) {
      const uint32_t words = (uint32_t)(counter_bytes / sizeof(uint32_t));
      hipLaunchKernelGGL(clear_words_kernel, dim3((words + 255) / 256 < 64 ? (words + 255) / 256 : 64), dim3(256), 0,
                         stream, static_cast<uint32_t*>(p), words);
      e = hipGetLastError();
    }
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || !p) {
      set_error("tp_decode_attention_noalloc: scratch set-up failed: %s", hipGetErrorString(e));
      return TP_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TP_OK;
}

}  // namespace tp

extern "C" int32_t tp_decode_attention_noalloc(const void* q, int64_t batch, int32_t hq, int32_t hkv,
                                               const tp_page_layout* layout, const tp_pages* pages,
                                               int32_t n_pages, const void* tail_k, const void* tail_v,
                                               int32_t tail_len, int64_t tail_stride, int64_t actual_seq_len,
                                               float scale, int32_t pages_per_split, void* out, void* stream) {
  clear_error();
  if (pages_per_split <= 0) pages_per_split = tp_default_pages_per_split(batch, hq, hkv, n_pages);
  const bool split = n_pages > 0 && n_splits_of(n_pages, pages_per_split) > 1;
  void* ws = nullptr;
  size_t ws_bytes = 0;
  if (split && batch >= 1 && hq >= 1 && hkv >= 1) {
    const size_t need = tp_decode_workspace_bytes(batch, hq, hkv, n_pages, tail_len, pages_per_split);
    if (need > kScratchBytes) {
      set_error("tp_decode_attention_noalloc: this call needs %zu bytes of split-K scratch, the library's static "
                "scratch holds %zu; raise pages_per_split or call tp_decode_attention with a workspace",
                need, kScratchBytes);
      return TP_ERR_WORKSPACE;
    }
    const int32_t st = scratch_of(static_cast<hipStream_t>(stream), tp_decode_counter_bytes(batch, hq, hkv), &ws);
    if (st != TP_OK) return st;
    ws_bytes = kScratchBytes;
  }
  return tp_decode_attention(q, batch, hq, hkv, layout, pages, n_pages, tail_k, tail_v, tail_len, tail_stride,
                             actual_seq_len, scale, pages_per_split, ws, ws_bytes, out, stream);
}

extern "C" unsigned long long tp_selftest_fastdiv(uint32_t d_max, unsigned long long* checks) {
  unsigned long long bad = 0, n_checked = 0;
  const uint64_t top = 1ull << 31;
  for (uint32_t d = 1; d <= d_max && d != 0; ++d) {
    const FastDiv f = make_fastdiv(d);
    auto check = [&](uint64_t n) {
      if (n >= top) return;
      ++n_checked;
      if (fast_div((uint32_t)n, f) != (uint32_t)n / d) ++bad;
    };
    for (uint64_t k = 0; k < top; k += top / 257 + d) {
      const uint64_t base = k / d * d;
      check(base);
      check(base + 1);
      if (base) check(base - 1);
    }
    for (uint64_t n = top - std::min<uint64_t>(top, 3ull * d); n < top; ++n) check(n);
    for (uint64_t n = 0; n < 3ull * d + 5; ++n) check(n);
  }
  if (checks) *checks = n_checked;
  return bad;
}

#ifdef TP_TIMELINE
#include "tp_attention_measure.inc"
#endif
