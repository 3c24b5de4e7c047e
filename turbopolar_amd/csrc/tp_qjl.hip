// tp_qjl.hip -- QJL residual sign sketches and the sketch score estimate.
//
// QJLResidualEncoder.compute_residual_sketch (rfsn_v11/quant/qjl/encoder.py:
// 30-44): proj = E @ W (W [dim][P] fp32, unit columns), bit p of a token's
// sketch = proj[p] >= 0, packed little-endian (bit i of byte j is projection
// 8j + i), and the residual norm f16(sqrt(sum E^2)).  One wave per row: lane
// p computes projection p (64 at a time) from the row and W staged in LDS, and
// one ballot yields 64 sketch bits.
//
// qjl_dot_estimate (rfsn_v11/quant/qjl/score_estimate.py:6-54): correction =
// |E| |q| sin(pi/2 * (P - 2 hamming) / P), the Hamming distance between the
// query's and the token's sketches, for every (query head, token); the query
// head reads the sketches of kv head h / g.  fp32 throughout.

#include "tp_common.h"

namespace tp {

constexpr int kQjlMaxDim = 256;
constexpr int kQjlMaxProj = 256;

template <bool F32IN>
__global__ __launch_bounds__(256) void qjl_sketch_kernel(const void* e, int64_t rows, int32_t dim, const float* w,
                                                         int32_t proj, uint8_t* packed, uint16_t* norms) {
  extern __shared__ float sm[];  // W [dim][proj], then one row of E per wave
  float* sw = sm;
  float* srow = sm + dim * proj + (threadIdx.x >> 6) * dim;
  for (int i = threadIdx.x; i < dim * proj; i += 256) sw[i] = w[i];
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int64_t waves = (int64_t)gridDim.x * 4;
  for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < rows; row += waves) {
    float ss = 0.0f;
    for (int d = lane; d < dim; d += 64) {
      const float x = F32IN ? static_cast<const float*>(e)[row * dim + d]
                            : h2f(static_cast<const uint16_t*>(e)[row * dim + d]);
      srow[d] = x;
      ss = __builtin_fmaf(x, x, ss);
    }
    wave_lds_sync();  // the row is in LDS for every lane of the wave
    for (int p0 = 0; p0 < proj; p0 += 64) {
      const int p = p0 + lane;
      float acc = 0.0f;
      if (p < proj) {
        for (int d = 0; d < dim; ++d) acc = __builtin_fmaf(srow[d], sw[d * proj + p], acc);
      }
      const uint64_t bits = __builtin_amdgcn_ballot_w64(p < proj && acc >= 0.0f);
      const int nbytes = min(8, (proj - p0) >> 3);
      if (lane < nbytes) packed[row * (proj >> 3) + (p0 >> 3) + lane] = (uint8_t)(bits >> (8 * lane));
    }
    if (norms) {
      for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
      if (lane == 0) norms[row] = f2h(sqrtf(ss));
    }
    wave_lds_sync();  // every lane is done with the row before the next overwrites it
  }
}

// sin(pi/2 * m / P) for the integer m = P - 2 hamming.
__device__ __forceinline__ float qjl_cos_est(int hamming, int proj) {
  return sinf(1.57079632679489662f * (float)(proj - 2 * hamming) / (float)proj);
}

__global__ __launch_bounds__(256) void qjl_estimate_kernel(const uint16_t* q, int32_t hq, int32_t g, int32_t dim,
                                                           const uint8_t* k_packed, const uint16_t* norms,
                                                           int64_t tokens, const uint8_t* q_packed, int32_t proj,
                                                           int64_t total, float* out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int64_t bhq = i / tokens;
  const int64_t t = i - bhq * tokens;
  const int64_t b = bhq / hq;
  const int64_t h = bhq - b * hq;
  const int64_t bkv = b * (hq / g) + h / g;
  float qq = 0.0f;
  for (int d = 0; d < dim; ++d) {
    const float x = h2f(q[bhq * dim + d]);
    qq = __builtin_fmaf(x, x, qq);
  }
  const int nb = proj >> 3;
  const uint8_t* ks = k_packed + (bkv * tokens + t) * nb;
  const uint8_t* qs = q_packed + bhq * nb;
  int ham = 0;
  for (int j = 0; j < nb; ++j) ham += __builtin_popcount((uint32_t)(ks[j] ^ qs[j]));
  out[i] = h2f(norms[bkv * tokens + t]) * sqrtf(qq) * qjl_cos_est(ham, proj);
}

}  // namespace tp

using namespace tp;

extern "C" {

int32_t tp_qjl_sketch(const void* e, int32_t in_dtype, int64_t rows, int32_t dim, const float* w, int32_t proj_dim,
                      uint8_t* packed, uint16_t* norms, void* stream) {
  clear_error();
  if (in_dtype != 0 && in_dtype != 1) {
    set_error("in_dtype must be 0 (float16) or 1 (float32), got %d", in_dtype);
    return TP_ERR_INVALID;
  }
  if (!e || !w || !packed || rows < 1 || dim < 1 || dim > kQjlMaxDim || proj_dim < 8 || proj_dim > kQjlMaxProj ||
      proj_dim % 8) {
    set_error("bad arguments: rows=%lld dim=%d proj_dim=%d (dim <= %d, proj_dim a multiple of 8 up to %d)",
              (long long)rows, dim, proj_dim, kQjlMaxDim, kQjlMaxProj);
    return TP_ERR_INVALID;
  }
  const size_t lds = ((size_t)dim * proj_dim + 4 * (size_t)dim) * sizeof(float);
  if (lds > 160 * 1024) {
    set_error("dim x proj_dim too large for one workgroup's LDS");
    return TP_ERR_INVALID;
  }
  const unsigned blocks = (unsigned)std::min<int64_t>((rows + 3) / 4, 2048);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (in_dtype)
    hipLaunchKernelGGL(qjl_sketch_kernel<true>, dim3(blocks), dim3(256), lds, s, e, rows, dim, w, proj_dim, packed,
                       norms);
  else
    hipLaunchKernelGGL(qjl_sketch_kernel<false>, dim3(blocks), dim3(256), lds, s, e, rows, dim, w, proj_dim, packed,
                       norms);
  return launch_status("tp_qjl_sketch");
}

int32_t tp_qjl_dot_estimate(const void* q, int64_t batch, int32_t hq, int32_t hkv, int32_t dim, const void* k_packed,
                            const void* norms, int64_t tokens, const void* q_packed, int32_t proj_dim, float* out,
                            void* stream) {
  clear_error();
  if (!q || !k_packed || !norms || !q_packed || !out || batch < 1 || hq < 1 || hkv < 1 || hq % hkv || dim < 1 ||
      tokens < 1 || proj_dim < 8 || proj_dim % 8) {
    set_error("bad arguments: batch=%lld hq=%d hkv=%d dim=%d tokens=%lld proj_dim=%d", (long long)batch, hq, hkv, dim,
              (long long)tokens, proj_dim);
    return TP_ERR_INVALID;
  }
  const int64_t total = batch * hq * tokens;
  if ((total + 255) / 256 > INT32_MAX) {
    set_error("batch * hq * tokens too large for one launch");
    return TP_ERR_INVALID;
  }
  hipLaunchKernelGGL(qjl_estimate_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(q), hq, hq / hkv, dim,
                     static_cast<const uint8_t*>(k_packed), static_cast<const uint16_t*>(norms), tokens,
                     static_cast<const uint8_t*>(q_packed), proj_dim, total, out);
  return launch_status("tp_qjl_dot_estimate");
}

}  // extern "C"
