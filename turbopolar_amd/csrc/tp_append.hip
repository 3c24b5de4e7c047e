// tp_append.hip -- the per-append staging step of TurboPolarKVCacheRuntime.
//
// The reference validates every append with mx.isfinite(...).all() (one host
// synchronisation per input, turbo_polar_cache.py:69) and then concatenates
// the new tokens onto its dense tail (:114-115).  Here one launch does both:
// it scans every element of k and v for non-finite values and copies a token
// range of them into the caller's preallocated dense tail; the host then reads
// one 4-byte verdict.  Nothing else in the runtime's state changes, so a
// rejected append leaves the cache as it was (only tail slots past the valid
// length were written).
#include "tp_common.h"

namespace tp {

struct AppendArgs {
  const void* k;
  const void* v;
  void* tail_k;
  void* tail_v;
  int64_t bh;
  int64_t in_tokens;
  int64_t copy_begin;
  int64_t n_copy;
  int64_t tail_tokens;  // token capacity of one (b, h) row of the tail
  int64_t tail_pos;
  uint32_t* flag;
  uint32_t epoch;
  int32_t check;
};

__device__ __forceinline__ bool all_finite(uint4 w, bool f32) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  bool ok = true;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (f32) {
      ok = ok && ((ws[i] & 0x7f800000u) != 0x7f800000u);
    } else {
      ok = ok && ((ws[i] & 0x7c00u) != 0x7c00u) && ((ws[i] & 0x7c000000u) != 0x7c000000u);
    }
  }
  return ok;
}

// One thread per 16-byte chunk of k (and the same chunk of v).
template <bool kF32>
__global__ __launch_bounds__(256) void append_stage_kernel(AppendArgs a) {
  constexpr int kElems = kF32 ? 4 : 8;           // elements per 16-byte chunk
  constexpr int kChunks = kHeadDim / kElems;     // chunks per token row
  const int64_t n = a.bh * a.in_tokens * kChunks;
  bool bad = false;
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < n; c += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = c / kChunks;             // (bh, token)
    const int part = (int)(c - row * kChunks);
    const int64_t bh = row / a.in_tokens;
    const int64_t tok = row - bh * a.in_tokens;
    const uint4 kw = reinterpret_cast<const uint4*>(a.k)[c];
    const uint4 vw = reinterpret_cast<const uint4*>(a.v)[c];
    if (a.check) bad = bad || !all_finite(kw, kF32) || !all_finite(vw, kF32);
    const int64_t rel = tok - a.copy_begin;
    if (rel >= 0 && rel < a.n_copy) {
      const int64_t dst = (bh * a.tail_tokens + a.tail_pos + rel) * kChunks + part;
      reinterpret_cast<uint4*>(a.tail_k)[dst] = kw;
      reinterpret_cast<uint4*>(a.tail_v)[dst] = vw;
    }
  }
  if (a.check == 2 && gridDim.x == 1) {
    // One workgroup: it reports completion itself, epoch (all finite) or
    // epoch + 1, once every thread's copies are issued and its verdict known;
    // the host polls the pinned word instead of synchronising the stream.
    const bool any_bad = __syncthreads_or(bad);
    if (threadIdx.x == 0)
      __hip_atomic_store(a.flag, any_bad ? a.epoch + 1u : a.epoch, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  } else if (bad) {  // every writer stores the same value
    if (a.check >= 2)
      __hip_atomic_store(a.flag, a.epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);  // pinned host flag
    else
      *a.flag = a.epoch;
  }
}

}  // namespace tp

using namespace tp;

extern "C" {

int32_t tp_append_stage(const void* k, const void* v, int32_t in_dtype, int64_t bh, int64_t in_tokens,
                        int64_t copy_begin, int64_t n_copy, void* tail_k, void* tail_v, int64_t tail_tokens,
                        int64_t tail_pos, int32_t check, uint32_t* flag, uint32_t epoch, void* stream) {
  clear_error();
  if (in_dtype != 0 && in_dtype != 1) {
    set_error("in_dtype must be 0 (fp16) or 1 (fp32), got %d", in_dtype);
    return TP_ERR_INVALID;
  }
  if (!k || !v || bh < 1 || in_tokens < 1) {
    set_error("bad input: k=%p v=%p bh=%lld tokens=%lld", k, v, (long long)bh, (long long)in_tokens);
    return TP_ERR_INVALID;
  }
  if (copy_begin < 0 || n_copy < 0 || copy_begin + n_copy > in_tokens || tail_pos < 0 ||
      tail_pos + n_copy > tail_tokens || (n_copy > 0 && (!tail_k || !tail_v))) {
    set_error("bad copy range: begin=%lld n=%lld of %lld tokens into tail position %lld of %lld",
              (long long)copy_begin, (long long)n_copy, (long long)in_tokens, (long long)tail_pos,
              (long long)tail_tokens);
    return TP_ERR_INVALID;
  }
  if (check < 0 || check > 3 || (check && !flag) || (check >= 2 && (epoch & 1u))) {
    set_error("check must be 0, 1 (device flag), 2 (pinned host flag, even epoch) or 3 (deferred, pinned host "
              "flag, even epoch), with a flag when checking");
    return TP_ERR_INVALID;
  }
  const uintptr_t al = (uintptr_t)k | (uintptr_t)v | (uintptr_t)tail_k | (uintptr_t)tail_v;
  if (al & 15u) {
    set_error("k, v and the tail buffers must be 16-byte aligned");
    return TP_ERR_INVALID;
  }
  AppendArgs a;
  a.k = k;
  a.v = v;
  a.tail_k = tail_k;
  a.tail_v = tail_v;
  a.bh = bh;
  a.in_tokens = in_tokens;
  a.copy_begin = copy_begin;
  a.n_copy = n_copy;
  a.tail_tokens = tail_tokens;
  a.tail_pos = tail_pos;
  a.flag = flag;
  a.epoch = epoch;
  a.check = check;
  const int64_t chunks = bh * in_tokens * (in_dtype ? kHeadDim / 4 : kHeadDim / 8);
  const unsigned blocks = (unsigned)std::min<int64_t>((chunks + 255) / 256, 1024);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (in_dtype)
    hipLaunchKernelGGL(append_stage_kernel<true>, dim3(blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(append_stage_kernel<false>, dim3(blocks), dim3(256), 0, s, a);
  int32_t st = launch_status("tp_append_stage");
  if (st != TP_OK || !check || check == 3) return st;
  if (check == 2) {  // the kernel writes the pinned host flag directly, no copy
    volatile uint32_t* vf = reinterpret_cast<volatile uint32_t*>(flag);
    uint32_t verdict = 0;
    bool done = false;
    if (blocks == 1) {
      // Poll for the workgroup's completion word (bounded; a launch that has
      // not reported by then is waited for the ordinary way).
      for (int spin = 0; spin < (1 << 22) && !done; ++spin) {
        verdict = *vf;
        done = verdict == epoch || verdict == epoch + 1u;
      }
    }
    if (!done) {
      if (hipStreamSynchronize(s) != hipSuccess) {
        set_error("tp_append_stage: synchronising the stream failed");
        return TP_ERR_HIP;
      }
      verdict = *vf;
    }
    if (verdict == epoch + 1u) {
      set_error("append() inputs must contain finite values");
      return TP_ERR_NONFINITE;
    }
    return TP_OK;
  }
  uint32_t verdict = 0;
  if (hipMemcpyAsync(&verdict, flag, sizeof(verdict), hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess) {
    set_error("tp_append_stage: reading the verdict failed");
    return TP_ERR_HIP;
  }
  if (verdict == epoch) {
    set_error("append() inputs must contain finite values");
    return TP_ERR_NONFINITE;
  }
  return TP_OK;
}

}  // extern "C"
