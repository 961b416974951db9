// Read-only streaming kernel: how fast one launch can read a buffer.
//
// The W4A16 GEMV at M = 1 reads its packed codes once and does little else,
// so its ceiling is what a launch that only reads the same bytes achieves.
// This kernel reads a buffer with 16-byte non-temporal loads in a grid-stride
// loop, U loads in flight per thread, and keeps the data alive by comparing
// each thread's XOR of everything it read with a fixed value (the flag is
// written only on that, practically never, match).  The benchmark times it
// over several grid sizes and unroll depths at each GEMV's byte count.
#include "common.hpp"

namespace gptq {
namespace {

constexpr uint32_t kSentinel = 0x9E3779B9u;

template <int U>
__global__ __launch_bounds__(256) void stream_read_k(const u32x4* __restrict__ p, int64_t n16,
                                                     uint32_t* __restrict__ flag) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (; i + (U - 1) * stride < n16; i += U * stride) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u];
  }
  for (; i < n16; i += stride) acc ^= __builtin_nontemporal_load(p + i);
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == kSentinel) flag[0] = 1u;
}

}  // namespace
}  // namespace gptq

using namespace gptq;

extern "C" int gptq_stream_read(const void* buf, size_t bytes, int blocks, int unroll, uint32_t* flag,
                                gptq_stream_t stream) {
  clear_error();
  GPTQ_REQUIRE(buf && flag, GPTQ_ERR_ARG, "stream_read: null pointer");
  GPTQ_REQUIRE(bytes % 16 == 0 && reinterpret_cast<uintptr_t>(buf) % 16 == 0, GPTQ_ERR_ARG,
               "stream_read: buffer and size must be multiples of 16 bytes");
  GPTQ_REQUIRE(blocks >= 1 && blocks <= (1 << 20), GPTQ_ERR_ARG, "stream_read: blocks %d out of range", blocks);
  const int64_t n16 = static_cast<int64_t>(bytes / 16);
  const u32x4* p = static_cast<const u32x4*>(buf);
  hipStream_t st = as_hip(stream);
  switch (unroll) {
    case 1: hipLaunchKernelGGL(stream_read_k<1>, dim3(blocks), dim3(256), 0, st, p, n16, flag); break;
    case 2: hipLaunchKernelGGL(stream_read_k<2>, dim3(blocks), dim3(256), 0, st, p, n16, flag); break;
    case 4: hipLaunchKernelGGL(stream_read_k<4>, dim3(blocks), dim3(256), 0, st, p, n16, flag); break;
    case 8: hipLaunchKernelGGL(stream_read_k<8>, dim3(blocks), dim3(256), 0, st, p, n16, flag); break;
    default: GPTQ_REQUIRE(false, GPTQ_ERR_ARG, "stream_read: unroll %d is not 1, 2, 4 or 8", unroll);
  }
  return check_launch("stream_read");
}
