// Measurement probes for bench.py: the HBM floor that the attention and append
// rooflines are read against.  Not part of the C-ABI of libkaplumba_tq.so (no
// counterpart in the reference); built as libkaplumba_probe.so.
//
//   tqp_stream_read  reads `bytes` (a multiple of 16) once with 16-byte
//                    nontemporal loads, grid-stride, `unroll` loads in flight
//                    per thread; nothing is written unless a checksum happens
//                    to hit a magic value (keeps the loads live).
//   tqp_copy         copies `bytes` with 16-byte nontemporal loads and stores.
// Both return 0 or the HIP error code of the launch.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kThreads = 256;
constexpr uint32_t kMagic = 0x9e3779b9u;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int U>
__global__ __launch_bounds__(kThreads) void stream_read_kernel(const u32x4* __restrict__ src, int64_t n,
                                                               uint32_t* __restrict__ sink) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (U - 1) * stride < n; i += U * stride) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (; i < n; i += stride) {
    const u32x4 v = __builtin_nontemporal_load(src + i);
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  if (acc == kMagic) sink[blockIdx.x] = acc;
}

template <int U>
__global__ __launch_bounds__(kThreads) void copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                        int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  for (; i + (U - 1) * stride < n; i += U * stride) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < U; ++u) __builtin_nontemporal_store(v[u], dst + i + u * stride);
  }
  for (; i < n; i += stride) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

}  // namespace

extern "C" int tqp_stream_read(const void* src, int64_t bytes, void* sink, int blocks, int unroll,
                               void* stream) {
  if (!src || !sink || bytes <= 0 || bytes % 16 || blocks <= 0) return static_cast<int>(hipErrorInvalidValue);
  const auto* s = static_cast<const u32x4*>(src);
  auto* k = static_cast<uint32_t*>(sink);
  const int64_t n = bytes / 16;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (unroll) {
    case 2: hipLaunchKernelGGL(stream_read_kernel<2>, dim3(blocks), dim3(kThreads), 0, st, s, n, k); break;
    case 4: hipLaunchKernelGGL(stream_read_kernel<4>, dim3(blocks), dim3(kThreads), 0, st, s, n, k); break;
    case 8: hipLaunchKernelGGL(stream_read_kernel<8>, dim3(blocks), dim3(kThreads), 0, st, s, n, k); break;
    default: return static_cast<int>(hipErrorInvalidValue);
  }
  return static_cast<int>(hipGetLastError());
}

extern "C" int tqp_copy(const void* src, void* dst, int64_t bytes, int blocks, void* stream) {
  if (!src || !dst || bytes <= 0 || bytes % 16 || blocks <= 0) return static_cast<int>(hipErrorInvalidValue);
  hipLaunchKernelGGL(copy_kernel<4>, dim3(blocks), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), bytes / 16);
  return static_cast<int>(hipGetLastError());
}
