// measure.hip -- the achievable HBM read bandwidth on this device, measured
// in the same run as the roofline kernels (bench.py): a plain streaming read
// of a device buffer, 16-byte loads, eight in flight per thread, grid-stride
// over the buffer.  Nothing is written except, never in practice, one word
// per block that keeps the loads from being optimised away.
#include "common.hpp"

namespace kh {

constexpr int kRdThreads = 256;
constexpr int kRdUnroll = 8;

__global__ __launch_bounds__(kRdThreads) void stream_read_kernel(const uint4* __restrict__ src, int64_t n16,
                                                                  uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  const int64_t step = (int64_t)gridDim.x * kRdThreads * kRdUnroll;
  for (int64_t base = (int64_t)blockIdx.x * kRdThreads * kRdUnroll + threadIdx.x; base < n16; base += step) {
    uint4 v[kRdUnroll];
#pragma unroll
    for (int u = 0; u < kRdUnroll; ++u) v[u] = src[min(base + (int64_t)u * kRdThreads, n16 - 1)];
#pragma unroll
    for (int u = 0; u < kRdUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

}  // namespace kh

using namespace kh;

extern "C" int kh_stream_read(const void* src_dev, int64_t bytes, uint32_t* sink_dev, int blocks,
                              void* stream) {
  KH_CHECK_ARG(src_dev && sink_dev, "null argument");
  KH_CHECK_ARG(bytes >= 16 && bytes % 16 == 0, "bytes %lld must be a positive multiple of 16",
               (long long)bytes);
  KH_CHECK_ARG(blocks >= 1 && blocks <= (1 << 20), "blocks %d not in [1, 2^20]", blocks);
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(kRdThreads), 0, as_stream(stream),
                     static_cast<const uint4*>(src_dev), bytes / 16, sink_dev);
  KH_LAUNCHED();
  return KH_OK;
}
