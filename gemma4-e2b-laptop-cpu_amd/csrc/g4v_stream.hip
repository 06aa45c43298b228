// g4v_stream.hip -- device memory bandwidth probe: the method of the reference's host probe
// (bench/stream_bw.cpp:10-19: one buffer far larger than the last-level cache, streamed whole a
// number of passes with wide loads, bandwidth = passes x bytes / wall time) on the GPU, plus a
// copy pass of known bytes that calibrates the FETCH_SIZE / WRITE_SIZE counters.
#include "g4v_internal.h"

namespace g4v {

typedef unsigned int su4 __attribute__((ext_vector_type(4)));
// streaming (non-temporal) 16-byte accesses: the probe's data is used once
__device__ __forceinline__ uint4 ld_nt(const uint4* p) {
  const su4 t = __builtin_nontemporal_load(reinterpret_cast<const su4*>(p));
  return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ void st_nt(uint4* p, uint4 v) {
  const su4 t = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(t, reinterpret_cast<su4*>(p));
}

// read pass: every 16-byte word once per pass, folded into one word per thread (kept live by a
// store only the host-invisible sink receives)
__global__ __launch_bounds__(256) void k_stream_read(const uint4* __restrict__ src, size_t n, uint4* __restrict__ sink) {
  uint4 acc = make_uint4(0, 0, 0, 0);
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n; i += 4 * stride) {  // four loads in flight per thread
    const uint4 a = ld_nt(src + i), b = ld_nt(src + i + stride), c = ld_nt(src + i + 2 * stride),
                d = ld_nt(src + i + 3 * stride);
    acc.x ^= a.x ^ b.x ^ c.x ^ d.x;
    acc.y ^= a.y ^ b.y ^ c.y ^ d.y;
    acc.z ^= a.z ^ b.z ^ c.z ^ d.z;
    acc.w ^= a.w ^ b.w ^ c.w ^ d.w;
  }
  for (; i < n; i += stride) {
    const uint4 a = src[i];
    acc.x ^= a.x;
    acc.y ^= a.y;
    acc.z ^= a.z;
    acc.w ^= a.w;
  }
  sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

__global__ __launch_bounds__(256) void k_stream_copy(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) st_nt(dst + i, ld_nt(src + i));
}

__global__ void k_stream_fill(uint4* __restrict__ dst, size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    dst[i] = make_uint4((uint32_t)i, (uint32_t)(i >> 32) ^ 0x9E3779B9u, (uint32_t)i * 3u, 7u);
}

// 2048 blocks of 256 threads, four loads in flight per thread: the fastest of the shapes tried
// (2048 to 32768 blocks, four or eight loads, plain or non-temporal: 4.7 to 5.85 TB/s)
int stream_grid() { return 2048; }

void launch_stream(int mode, const uint4* src, uint4* dst, size_t n16, hipStream_t st) {
  const int grid = stream_grid();
  if (mode == 2)
    hipLaunchKernelGGL(k_stream_fill, dim3(grid), dim3(256), 0, st, dst, n16);
  else if (mode == 1)
    hipLaunchKernelGGL(k_stream_copy, dim3(grid), dim3(256), 0, st, src, dst, n16);
  else
    hipLaunchKernelGGL(k_stream_read, dim3(grid), dim3(256), 0, st, src, n16, dst);
}

}  // namespace g4v
