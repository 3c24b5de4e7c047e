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

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

template <bool kF32>
__global__ __launch_bounds__(256) void encode_pages_kernel(EncodeArgs a) {
  __shared__ uint8_t s_codes[kPageTokens * kPairs];
  __shared__ float s_max[4];

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
      float lr[16];
      uint32_t lfix = 0;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint16_t rb = r16[j] > kF16RadiusFloor ? r16[j] : kF16RadiusFloor;
        bool exact;
        lr[j] = h2f(log_f16_fast(h2f(rb), &exact));
        lfix |= exact ? 0u : (1u << j);
      }
      while (lfix) {
        const int j = __builtin_ctz(lfix);
        lfix &= lfix - 1u;
        uint16_t rb = 0;
#pragma unroll
        for (int k2 = 0; k2 < 16; ++k2) rb = k2 == j ? r16[k2] : rb;
        rb = rb > kF16RadiusFloor ? rb : kF16RadiusFloor;
        const float exact_lr = h2f(log_f16_slow(h2f(rb)));
#pragma unroll
        for (int k2 = 0; k2 < 16; ++k2) lr[k2] = k2 == j ? exact_lr : lr[k2];
      }
      float mx = 0.0f;
#pragma unroll
      for (int j = 0; j < 16; ++j) mx = fmaxf(mx, fabsf(lr[j]));
      mx = wave_max(mx);
      if ((tid & 63) == 0) s_max[tid >> 6] = mx;
      __syncthreads();
      mx = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
      const float ls = mx == 0.0f ? 1e-6f : mx;
      const uint16_t ls16 = f2h(ls / 127.0f);
      const float lsf = h2f(ls16);
      uint32_t packed[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t c = (uint32_t)(to_int8_rne(lr[j] / lsf) & 0xff);
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
    for (int i = 0; i < 32; ++i) m = fmaxf(m, fabsf(raw_val(vraw, i)));
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
  if (in_dtype == 1)
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
