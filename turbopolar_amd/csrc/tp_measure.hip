// tp_measure.hip -- the streaming-read ceiling of the decode step's page bytes.
//
// Linked into the measurement library only (libturbopolar_hip_timeline.so),
// never into the product library.  tp_measure_stream_read reads up to eight
// device buffers once, whole, with the decode kernel's load form (16-byte
// non-temporal loads, one lane-contiguous KiB per wave instruction) and does
// nothing with the bytes but fold them into a register.  Timed over the page
// fields of a cache, it is the fastest that this many bytes can leave HBM
// through a kernel of the given grid: the decode kernel's roofline fraction
// read against it separates what the page format costs from what the kernel
// costs.

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxSegments = 8;

struct Segments {
  const u32x4* ptr[kMaxSegments];
  int64_t n16[kMaxSegments];  // 16-byte units in each buffer
  int64_t chunk_begin[kMaxSegments + 1];  // first claimable chunk of each buffer (dynamic kernel)
  int count;
};

// Grid-stride over each buffer; a thread issues U loads before it folds
// them, so every wave keeps U KiB in flight.  The fold result is stored only
// if it equals a fixed 128-bit value (the store exists so that the loads are
// live; sink holds one word per workgroup).
template <int U>
__global__ __launch_bounds__(1024) void stream_read_kernel(Segments s, uint32_t* sink) {
  u32x4 acc = {0u, 0u, 0u, 0u};
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * U;
  for (int k = 0; k < s.count; ++k) {
    const u32x4* p = s.ptr[k];
    const int64_t n = s.n16[k];
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x * U + threadIdx.x; i < n; i += stride) {
      u32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t j = i + (int64_t)u * blockDim.x;
        v[u] = j < n ? __builtin_nontemporal_load(p + j) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < U; ++u) acc ^= v[u];
    }
  }
  if (acc.x == 0x9E3779B9u && acc.y == 0x7F4A7C15u && acc.z == 0xF39CC060u && acc.w == 0x5CEDC834u)
    sink[blockIdx.x] = acc.x ^ acc.y;
}

// The same reads handed out dynamically: a wave claims chunks of 64 x U
// 16-byte units (U KiB, one lane-contiguous KiB per load instruction) from a
// 64-bit counter with one atomic, and claims its next chunk right after
// issuing the current chunk's loads, so the claim's round trip overlaps them.
// Claim values count from `base`; every wave leaves after its first claim past
// the last chunk, so a launch takes exactly chunks + waves claims and the next
// launch's base is known on the host without clearing the counter.
template <int U>
__global__ __launch_bounds__(1024) void stream_read_dynamic_kernel(Segments s, uint64_t* counter, uint64_t base,
                                                                   uint32_t* sink) {
  const int lane = threadIdx.x & 63;
  const int64_t total = s.chunk_begin[s.count];
  u32x4 acc = {0u, 0u, 0u, 0u};
  uint64_t got = 0;
  if (lane == 0) got = __hip_atomic_fetch_add(counter, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  int64_t c = (int64_t)(__builtin_amdgcn_readfirstlane((uint32_t)(got - base)));
  while (c < total) {
    int k = 0;
    while (k + 1 < s.count && c >= s.chunk_begin[k + 1]) ++k;
    const u32x4* p = s.ptr[k];
    const int64_t n = s.n16[k];
    const int64_t off = (c - s.chunk_begin[k]) * 64 * U + lane;
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = off + (int64_t)u * 64;
      v[u] = j < n ? __builtin_nontemporal_load(p + j) : u32x4{0u, 0u, 0u, 0u};
    }
    got = 0;
    if (lane == 0) got = __hip_atomic_fetch_add(counter, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int64_t next = (int64_t)__builtin_amdgcn_readfirstlane((uint32_t)(got - base));
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u];
    c = next;
  }
  if (acc.x == 0x9E3779B9u && acc.y == 0x7F4A7C15u && acc.z == 0xF39CC060u && acc.w == 0x5CEDC834u)
    sink[blockIdx.x] = acc.x ^ acc.y;
}

}  // namespace

// Reads buffers[0..count) (byte sizes sizes[], each a multiple of 16 and
// 16-byte aligned) with grid x threads workgroups, unroll 4, 8 or 16.  sink:
// at least grid words of device memory.  Returns 0, or -1 for arguments outside
// these limits (nothing is launched then).
extern "C" int32_t tp_measure_stream_read(const void* const* buffers, const int64_t* sizes, int32_t count,
                                          int32_t grid, int32_t threads, int32_t unroll, uint32_t* sink,
                                          hipStream_t stream) {
  if (count < 1 || count > kMaxSegments || grid < 1 || grid > (1 << 20) || sink == nullptr) return -1;
  if (threads != 256 && threads != 512 && threads != 1024) return -1;
  Segments s = {};
  s.count = count;
  for (int k = 0; k < count; ++k) {
    if (buffers[k] == nullptr || sizes[k] < 0 || sizes[k] % 16 || reinterpret_cast<uintptr_t>(buffers[k]) % 16)
      return -1;
    s.ptr[k] = static_cast<const u32x4*>(buffers[k]);
    s.n16[k] = sizes[k] / 16;
  }
  if (unroll == 4)
    hipLaunchKernelGGL(stream_read_kernel<4>, dim3(grid), dim3(threads), 0, stream, s, sink);
  else if (unroll == 8)
    hipLaunchKernelGGL(stream_read_kernel<8>, dim3(grid), dim3(threads), 0, stream, s, sink);
  else if (unroll == 16)
    hipLaunchKernelGGL(stream_read_kernel<16>, dim3(grid), dim3(threads), 0, stream, s, sink);
  else
    return -1;
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// tp_measure_stream_read with the chunks claimed dynamically by every wave
// (stream_read_dynamic_kernel).  counter: one 64-bit device word, zero before
// the first launch and never cleared after; base: 0 for the first launch, then
// the *next_base the previous launch returned (launches on one stream).
// Returns 0, or -1 for arguments outside the limits of tp_measure_stream_read.
extern "C" int32_t tp_measure_stream_read_dynamic(const void* const* buffers, const int64_t* sizes, int32_t count,
                                                  int32_t grid, int32_t threads, int32_t unroll, uint64_t* counter,
                                                  uint64_t base, uint64_t* next_base, uint32_t* sink,
                                                  hipStream_t stream) {
  if (count < 1 || count > kMaxSegments || grid < 1 || grid > (1 << 20) || sink == nullptr || counter == nullptr ||
      next_base == nullptr)
    return -1;
  if (threads != 256 && threads != 512 && threads != 1024) return -1;
  if (unroll != 4 && unroll != 8 && unroll != 16) return -1;
  Segments s = {};
  s.count = count;
  s.chunk_begin[0] = 0;
  for (int k = 0; k < count; ++k) {
    if (buffers[k] == nullptr || sizes[k] < 0 || sizes[k] % 16 || reinterpret_cast<uintptr_t>(buffers[k]) % 16)
      return -1;
    s.ptr[k] = static_cast<const u32x4*>(buffers[k]);
    s.n16[k] = sizes[k] / 16;
    s.chunk_begin[k + 1] = s.chunk_begin[k] + (s.n16[k] + 64 * unroll - 1) / (64 * unroll);
  }
  const int64_t waves = (int64_t)grid * (threads / 64);
  // claim offsets travel as 32-bit values within a launch
  if (s.chunk_begin[count] + waves >= (int64_t)INT32_MAX) return -1;
  if (unroll == 4)
    hipLaunchKernelGGL(stream_read_dynamic_kernel<4>, dim3(grid), dim3(threads), 0, stream, s, counter, base, sink);
  else if (unroll == 8)
    hipLaunchKernelGGL(stream_read_dynamic_kernel<8>, dim3(grid), dim3(threads), 0, stream, s, counter, base, sink);
  else
    hipLaunchKernelGGL(stream_read_dynamic_kernel<16>, dim3(grid), dim3(threads), 0, stream, s, counter, base, sink);
  *next_base = base + (uint64_t)(s.chunk_begin[count] + waves);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
