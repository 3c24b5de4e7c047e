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
};

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
  const int64_t slot = bh * a.capacity + a.page_begin + page;
  const int64_t row = slot * kPageTokens + t;
  const int64_t out_off = ((bh * a.n_pages + page) * kPageTokens + t) * kHeadDim + 32 * qq;

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

}  // namespace tp

using namespace tp;

extern "C" int32_t tp_decode_pages(const tp_page_layout* layout, const tp_pages* pages, int64_t bh,
                                   int64_t page_begin, int32_t n_pages, void* k_out, void* v_out,
                                   void* stream) {
  clear_error();
  int l1_row = 0, deep_row = 0;
  if (!check_layout(layout, &l1_row, &deep_row)) return TP_ERR_UNSUPPORTED;
  if (!pages || bh < 1 || bh > 65535 || n_pages < 0 || page_begin < 0 ||
      page_begin + n_pages > pages->capacity) {
    set_error("bad page range");
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
  hipLaunchKernelGGL(decode_pages_kernel, dim3((unsigned)n_pages, (unsigned)bh), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status("tp_decode_pages");
}
