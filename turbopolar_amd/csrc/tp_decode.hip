// tp_decode.hip -- decompress pages back to dense fp16 K and V.
//
// Restates PolarQuantDecoder.decode_block (rfsn_v11/quant/polar/decoder.py:7-67)
// and GroupedVQuantizer.dequantize_block (rfsn_v11/quant/v_quant/encoder.py:32-38)
// with the reference's fp32 arithmetic: angle = f32(code)/f32(levels-1) *
// f32(2*pi) - f32(pi); r = f32(radius) or exp(f32(code) * f32(scale));
// k = f16(r * cos(angle)), f16(r * sin(angle)); v = f16(f32(code) * f32(scale)).
//
// One 256-thread workgroup per page; thread (t = tid/4, q = tid%4) writes key
// pairs [16q, 16q+16) and value group q of token t (64 contiguous bytes each).
// The page's code rows are staged in LDS, and the fp32 cos / sin of every code
// angle (and, for int8 log radii, exp(code * scale) of every code) are built
// once per workgroup into LDS tables, so a pair costs two lookups and two fp32
// multiplies; the table entries are the same fp32 values the per-pair
// expressions give, so the output is unchanged.
#include "tp_common.h"

namespace tp {

struct DecodeArgs {
  const void* radii;
  const uint16_t* radii_scales;
  const uint8_t* angle_l1;
  const uint8_t* angle_deep;
  const int8_t* v_codes;
  const uint16_t* v_scales;
  int64_t capacity;
  int64_t page_begin;
  int32_t n_pages;
  int32_t int8_radii;
  int32_t l1_bits;
  int32_t deep_bits;
  int32_t split_half;
  int32_t l1_row;
  int32_t deep_row;
  uint16_t* k_out;
  uint16_t* v_out;
  int64_t out_tokens;  // tokens per (batch, head) row of k_out / v_out
  int64_t out_offset;  // token of that row where page page_begin lands
  // Gather launches (tp_decode_pages_gather): output page j is stored page
  // page_index[j], clamped to [0, n_stored), instead of page_begin + j.
  const int32_t* page_index;
  int32_t n_stored;
};

// The stored page that output page `page` of a launch decodes.
template <bool GATHER>
__device__ __forceinline__ int64_t source_page(const DecodeArgs& a, int page) {
  if constexpr (GATHER) return (int64_t)min(max(a.page_index[page], 0), a.n_stored - 1);
  return a.page_begin + page;
}

template <bool GATHER>
__global__ __launch_bounds__(256) void decode_pages_kernel(DecodeArgs a) {
  __shared__ float2 s_cs_l1[256];
  __shared__ float2 s_cs_deep[256];
  __shared__ float s_exp[256];
  __shared__ uint32_t s_l1[kPageTokens * 64 / 4];
  __shared__ uint32_t s_deep[kPageTokens * 64 / 4];
  const int page = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int tid = threadIdx.x;
  const int t = tid >> 2;
  const int qq = tid & 3;
  const int64_t slot = bh * a.capacity + source_page<GATHER>(a, page);
  const int64_t row = slot * kPageTokens + t;
  const int64_t out_off = (bh * a.out_tokens + a.out_offset + (int64_t)page * kPageTokens + t) * kHeadDim + 32 * qq;

  if (a.k_out) {
    // Tables: (cos, sin) of each l1 / deep code angle (decoder.py:37-55) and
    // exp(code * scale) of each int8 log-radius code (decoder.py:57-62).
    if (tid < (1 << a.l1_bits) && a.split_half > 0) {
      const float th = code_angle((uint32_t)tid, a.l1_bits);
      s_cs_l1[tid] = make_float2(cosf(th), sinf(th));
    }
    if (tid < (1 << a.deep_bits)) {
      const float th = code_angle((uint32_t)tid, a.deep_bits);
      s_cs_deep[tid] = make_float2(cosf(th), sinf(th));
    }
    if (a.int8_radii) s_exp[tid] = expf((float)(tid - 128) * h2f(a.radii_scales[slot]));
    // The page's code rows: 64 rows of l1_row / deep_row bytes each, contiguous.
    const uint32_t* l1src = reinterpret_cast<const uint32_t*>(a.angle_l1 + slot * kPageTokens * a.l1_row);
    for (int i = tid; i < 16 * a.l1_row; i += 256) s_l1[i] = l1src[i];
    const uint32_t* deepsrc = reinterpret_cast<const uint32_t*>(a.angle_deep + slot * kPageTokens * a.deep_row);
    for (int i = tid; i < 16 * a.deep_row; i += 256) s_deep[i] = deepsrc[i];
    // Radii of the thread's 16 pairs: 32 bytes (fp16) or 16 bytes (int8 codes).
    uint4 rv[2];
    if (a.int8_radii) {
      rv[0] = *reinterpret_cast<const uint4*>(static_cast<const int8_t*>(a.radii) + row * kPairs + 16 * qq);
      rv[1] = make_uint4(0u, 0u, 0u, 0u);
    } else {
      const uint4* rp = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.radii) + row * kPairs + 16 * qq);
      rv[0] = rp[0];
      rv[1] = rp[1];
    }
    __syncthreads();
    const uint8_t* l1row = reinterpret_cast<const uint8_t*>(s_l1) + t * a.l1_row;
    const uint8_t* deeprow = reinterpret_cast<const uint8_t*>(s_deep) + t * a.deep_row;
    const uint32_t rw[8] = {rv[0].x, rv[0].y, rv[0].z, rv[0].w, rv[1].x, rv[1].y, rv[1].z, rv[1].w};
    uint32_t w[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int p = 16 * qq + j;
      float r;
      if (a.int8_radii) {
        r = s_exp[((rw[j >> 2] >> (8 * (j & 3))) + 128u) & 0xffu];
      } else {
        r = h2f((uint16_t)(rw[j >> 1] >> (16 * (j & 1))));
      }
      const float2 cs = p < a.split_half ? s_cs_l1[packed_code(l1row, p, a.l1_bits)]
                                         : s_cs_deep[packed_code(deeprow, p - a.split_half, a.deep_bits)];
      w[j] = (uint32_t)f2h(r * cs.x) | ((uint32_t)f2h(r * cs.y) << 16);
    }
    uint4* dst = reinterpret_cast<uint4*>(a.k_out + out_off);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
  }

  if (a.v_out) {
    const float s = h2f(a.v_scales[row * kVGroups + qq]);
    const uint4* src = reinterpret_cast<const uint4*>(a.v_codes + row * kHeadDim + 32 * qq);
    const uint4 c0 = src[0];
    const uint4 c1 = src[1];
    const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    uint32_t w[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int e0 = 2 * i, e1 = 2 * i + 1;
      const float v0 = (float)(int8_t)((cw[e0 >> 2] >> (8 * (e0 & 3))) & 0xffu) * s;
      const float v1 = (float)(int8_t)((cw[e1 >> 2] >> (8 * (e1 & 3))) & 0xffu) * s;
      w[i] = (uint32_t)f2h(v0) | ((uint32_t)f2h(v1) << 16);
    }
    uint4* dst = reinterpret_cast<uint4*>(a.v_out + out_off);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
  }
}

// ---- specialised layouts ------------------------------------------------------
//
// The default layout (fp16 radii, 4-bit l1 and deep codes, split 64) and the
// fast layout (int8 log radii with an fp16 page scale, 8-bit deep codes,
// split 0) get their own kernel, one page per workgroup.  Thread T decodes
// the 8-dim chunk c = T % 16 (pairs 4c .. 4c+3, V group c / 4) of tokens
// T / 16 + 16 k, k = 0..3, so every load and store instruction of a wave
// covers consecutive bytes (a wave's 16-byte output stores fill 1 KiB runs).
// All loads are issued first; the (cos, sin) table (16 or 256 entries) and,
// for the fast layout, the page's exp table are built in LDS while they are in
// flight, and V is decoded and stored before the barrier that guards the
// tables.  V is dequantised as fp16 pairs, f16(code * scale) with one
// rounding of the exact product, as the f32 expression rounds it.  Outputs
// are the generic kernel's, bit for bit.
enum DecodeKind { kDecDefault = 0, kDecFast = 1 };

__device__ __forceinline__ uint32_t i8pair_to_h2(uint32_t w, int first) {
  // Bytes `first` and `first + 1` of w (int8) as an exact fp16 pair.
  const f16 lo = (f16)(int)(int8_t)(w >> (8 * first));
  const f16 hi = (f16)(int)(int8_t)(w >> (8 * first + 8));
  return (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}

// WANT_K / WANT_V: which of k_out / v_out the launch writes.  They are
// template parameters, not branches on the pointers: a register set under a
// branch made the compiler wait for the K loads at its join, so the V loads
// went out one memory round trip late.
template <int KIND, bool WANT_K, bool WANT_V, bool GATHER = false>
__global__ __launch_bounds__(256) void decode_pages_spec_kernel(DecodeArgs a) {
  constexpr bool kFast = KIND == kDecFast;
  constexpr int kCodes = kFast ? 256 : 16;
  constexpr int kTok = 4;  // tokens per thread
  __shared__ float2 s_cs[kCodes];
  __shared__ float s_exp[kFast ? 256 : 1];
  const int tid = threadIdx.x;
  const int c = tid & 15;    // 8-dim chunk
  const int t0 = tid >> 4;   // first token; the others are t0 + 16 k
  const int64_t bh = blockIdx.y;
  const int page = blockIdx.x;
  const int64_t slot = bh * a.capacity + source_page<GATHER>(a, page);
  const int64_t row0 = slot * kPageTokens;
  const int64_t out0 = bh * a.out_tokens + a.out_offset + (int64_t)page * kPageTokens;
  constexpr bool want_k = WANT_K;
  constexpr bool want_v = WANT_V;

  // All loads first.
  uint32_t rw[kTok][kFast ? 1 : 2];  // radii of pairs 4c..4c+3
  uint32_t cw[kTok];                 // their angle codes (low 16 bits for 4-bit codes)
  uint16_t ls16 = 0;
  if constexpr (want_k) {
#pragma unroll
    for (int k = 0; k < kTok; ++k) {
      const int64_t row = row0 + t0 + 16 * k;
      if constexpr (kFast) {
        rw[k][0] = *reinterpret_cast<const uint32_t*>(static_cast<const int8_t*>(a.radii) + row * kPairs + 4 * c);
        cw[k] = *reinterpret_cast<const uint32_t*>(a.angle_deep + row * kPairs + 4 * c);
      } else {
        const uint2 r = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.radii) + row * kPairs + 4 * c);
        rw[k][0] = r.x, rw[k][1] = r.y;
        cw[k] = *reinterpret_cast<const uint16_t*>((c < 8 ? a.angle_l1 : a.angle_deep) + row * 16 + 2 * (c & 7));
      }
    }
    if constexpr (kFast) ls16 = a.radii_scales[slot];
  }
  uint2 vc[kTok];
  uint16_t vs16[kTok];
  if constexpr (want_v) {
#pragma unroll
    for (int k = 0; k < kTok; ++k) {
      const int64_t row = row0 + t0 + 16 * k;
      vc[k] = *reinterpret_cast<const uint2*>(a.v_codes + row * kHeadDim + 8 * c);
      vs16[k] = a.v_scales[row * kVGroups + (c >> 2)];
    }
  }

  // Tables (decoder.py:37-62) while the loads are in flight.
  if (want_k && tid < kCodes) {
    const float th = code_angle((uint32_t)tid, kFast ? 8 : 4);
    s_cs[tid] = make_float2(cosf(th), sinf(th));
  }

  // V (v_quant/encoder.py:32-38).
  if constexpr (want_v) {
#pragma unroll
    for (int k = 0; k < kTok; ++k) {
      const half2v sp = __builtin_bit_cast(half2v, (uint32_t)vs16[k] | ((uint32_t)vs16[k] << 16));
      uint32_t w[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const half2v h = __builtin_bit_cast(half2v, i8pair_to_h2(q < 2 ? vc[k].x : vc[k].y, 2 * (q & 1)));
        w[q] = __builtin_bit_cast(uint32_t, h * sp);
      }
      *reinterpret_cast<uint4*>(a.v_out + (out0 + t0 + 16 * k) * kHeadDim + 8 * c) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
  if constexpr (!want_k) return;
  if constexpr (kFast) s_exp[tid] = expf((float)(tid - 128) * h2f(ls16));
  __syncthreads();

  // K (decoder.py:57-67).
#pragma unroll
  for (int k = 0; k < kTok; ++k) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float r;
      uint32_t code;
      if constexpr (kFast) {
        r = s_exp[((rw[k][0] >> (8 * j)) + 128u) & 0xffu];
        code = (cw[k] >> (8 * j)) & 0xffu;
      } else {
        r = h2f((uint16_t)(rw[k][j >> 1] >> (16 * (j & 1))));
        code = (cw[k] >> (4 * j)) & 0xfu;
      }
      const float2 cs = s_cs[code];
      w[j] = (uint32_t)f2h(r * cs.x) | ((uint32_t)f2h(r * cs.y) << 16);
    }
    *reinterpret_cast<uint4*>(a.k_out + (out0 + t0 + 16 * k) * kHeadDim + 8 * c) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

}  // namespace tp

using namespace tp;

template <int KIND, bool GATHER>
static void launch_spec(const DecodeArgs& a, dim3 grid, hipStream_t s) {
  if (a.k_out && a.v_out)
    hipLaunchKernelGGL((decode_pages_spec_kernel<KIND, true, true, GATHER>), grid, dim3(256), 0, s, a);
  else if (a.k_out)
    hipLaunchKernelGGL((decode_pages_spec_kernel<KIND, true, false, GATHER>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((decode_pages_spec_kernel<KIND, false, true, GATHER>), grid, dim3(256), 0, s, a);
}

// Pages [page_begin, page_begin + n_pages) (page_index NULL), or the stored
// pages page_index[0 .. n_pages) of the first n_stored (a device array), of
// every (batch, head) row into output tokens [out_offset, out_offset + 64
// n_pages) of rows of out_tokens tokens.
static int32_t decode_pages_impl(const tp_page_layout* layout, const tp_pages* pages, int64_t bh,
                                 int64_t page_begin, int32_t n_pages, const int32_t* page_index, int32_t n_stored,
                                 void* k_out, void* v_out, int64_t out_tokens, int64_t out_offset, void* stream) {
  clear_error();
  int l1_row = 0, deep_row = 0;
  if (!check_layout(layout, &l1_row, &deep_row)) return TP_ERR_UNSUPPORTED;
  if (!pages || bh < 1 || bh > 65535 || n_pages < 0 || page_begin < 0 ||
      (page_index ? (n_stored < 1 || n_stored > pages->capacity || ((uintptr_t)page_index & 3u))
                  : page_begin + n_pages > pages->capacity)) {
    set_error("bad page range");
    return TP_ERR_INVALID;
  }
  if (out_offset < 0 || out_offset + (int64_t)n_pages * kPageTokens > out_tokens) {
    set_error("pages [%lld, %lld) of output rows of %lld tokens", (long long)out_offset,
              (long long)(out_offset + (int64_t)n_pages * kPageTokens), (long long)out_tokens);
    return TP_ERR_INVALID;
  }
  if (n_pages == 0 || (!k_out && !v_out)) return TP_OK;
  if (k_out && (!pages->radii || (l1_row > 0 && !pages->angle_l1) ||
                (deep_row > 0 && !pages->angle_deep) ||
                (layout->int8_radii && !pages->radii_scales) || ((uintptr_t)k_out & 15u) ||
                ((uintptr_t)pages->radii & 15u) || ((uintptr_t)pages->angle_l1 & 3u) ||
                ((uintptr_t)pages->angle_deep & 3u))) {
    set_error("key page buffers missing or misaligned (radii 16-byte, codes 4-byte), or k_out misaligned");
    return TP_ERR_INVALID;
  }
  if (v_out && (!pages->v_codes || !pages->v_scales || ((uintptr_t)v_out & 15u) ||
                ((uintptr_t)pages->v_codes & 15u))) {
    set_error("value page buffers missing or v_out misaligned");
    return TP_ERR_INVALID;
  }
  DecodeArgs a;
  a.radii = pages->radii;
  a.radii_scales = static_cast<const uint16_t*>(pages->radii_scales);
  a.angle_l1 = pages->angle_l1;
  a.angle_deep = pages->angle_deep;
  a.v_codes = pages->v_codes;
  a.v_scales = static_cast<const uint16_t*>(pages->v_scales);
  a.capacity = pages->capacity;
  a.page_begin = page_begin;
  a.n_pages = n_pages;
  a.int8_radii = layout->int8_radii;
  a.l1_bits = layout->l1_bits;
  a.deep_bits = layout->deep_bits;
  a.split_half = layout->split_dim / 2;
  a.l1_row = l1_row;
  a.deep_row = deep_row;
  a.k_out = static_cast<uint16_t*>(k_out);
  a.v_out = static_cast<uint16_t*>(v_out);
  a.out_tokens = out_tokens;
  a.out_offset = out_offset;
  a.page_index = page_index;
  a.n_stored = n_stored;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool is_default = !layout->int8_radii && layout->l1_bits == 4 && layout->deep_bits == 4 && layout->split_dim == 64;
  const bool is_fast = layout->int8_radii && layout->deep_bits == 8 && layout->split_dim == 0;
  const bool aligned = (!k_out || (is_default ? ((uintptr_t)pages->angle_l1 & 1u) == 0 && ((uintptr_t)pages->angle_deep & 1u) == 0
                                              : ((uintptr_t)pages->angle_deep & 3u) == 0 &&
                                                    ((uintptr_t)pages->radii & 3u) == 0)) &&
                       (!v_out || ((uintptr_t)pages->v_codes & 7u) == 0);
  const dim3 grid((unsigned)n_pages, (unsigned)bh);
  if ((is_default || is_fast) && aligned) {
    if (page_index) {
      if (is_default)
        launch_spec<kDecDefault, true>(a, grid, s);
      else
        launch_spec<kDecFast, true>(a, grid, s);
    } else {
      if (is_default)
        launch_spec<kDecDefault, false>(a, grid, s);
      else
        launch_spec<kDecFast, false>(a, grid, s);
    }
  } else if (page_index) {
    hipLaunchKernelGGL(decode_pages_kernel<true>, grid, dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL(decode_pages_kernel<false>, grid, dim3(256), 0, s, a);
  }
  return launch_status("tp_decode_pages");
}

extern "C" int32_t tp_decode_pages_into(const tp_page_layout* layout, const tp_pages* pages, int64_t bh,
                                        int64_t page_begin, int32_t n_pages, void* k_out, void* v_out,
                                        int64_t out_tokens, int64_t out_offset, void* stream) {
  return decode_pages_impl(layout, pages, bh, page_begin, n_pages, nullptr, 0, k_out, v_out, out_tokens, out_offset,
                           stream);
}

extern "C" int32_t tp_decode_pages_gather(const tp_page_layout* layout, const tp_pages* pages, int64_t bh,
                                          int32_t n_stored, const int32_t* page_index, int32_t n_index, void* k_out,
                                          void* v_out, void* stream) {
  if (!page_index && n_index > 0) {
    clear_error();
    set_error("tp_decode_pages_gather needs a page index array");
    return TP_ERR_INVALID;
  }
  if (n_index == 0) {
    clear_error();
    return TP_OK;
  }
  return decode_pages_impl(layout, pages, bh, 0, n_index, page_index, n_stored, k_out, v_out,
                           (int64_t)(n_index > 0 ? n_index : 0) * kPageTokens, 0, stream);
}

extern "C" int32_t tp_decode_pages(const tp_page_layout* layout, const tp_pages* pages, int64_t bh,
                                   int64_t page_begin, int32_t n_pages, void* k_out, void* v_out,
                                   void* stream) {
  return tp_decode_pages_into(layout, pages, bh, page_begin, n_pages, k_out, v_out,
                              (int64_t)(n_pages > 0 ? n_pages : 0) * kPageTokens, 0, stream);
}
