// Shared helpers of libgptq_hip.so: status/last-error plumbing, element
// conversions and the MFMA vector types used by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <type_traits>

#include "plan.hpp"

namespace gptq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// f(std::integral_constant<int, i>) for i = I .. N - 1: an unrolled loop whose
// index is a compile-time constant in the body (register arrays, LDS buffers)
template <int I, int N, class F>
__device__ __forceinline__ void sfor(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    sfor<I + 1, N>(f);
  }
}

// -------------------------------------------------------------- errors ----
// (set_error, clear_error and GPTQ_REQUIRE come from status.hpp)
inline hipStream_t as_hip(gptq_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Checks the launch just enqueued.
int check_launch(const char* what);

// ----------------------------------------------------- element access ----
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  _Float16 h;
  __builtin_memcpy(&h, &b, 2);
  return static_cast<float>(h);
}
// Round-to-nearest-even float -> bf16 bits (inputs here are finite).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u) return static_cast<uint16_t>((u >> 16) | ((u & 0xffff) ? 0x40 : 0));
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = static_cast<_Float16>(f);
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

// Element i of an fp32 / fp16 / bf16 array, in two parts so that a caller can
// issue the load early and convert where the value is used: elem_word loads
// the aligned 32-bit word that holds the element (a 16-bit element is its low
// or high half, `hi`; that word lies inside the allocation, whose base is
// 256-byte aligned and whose size is a multiple of 4) with plain pointer
// arithmetic from p, so the load stays a global (not flat) load; elem_value
// converts.  Both are branch-free: a branch on the dtype around the load, a
// flat load, or a conversion right after the load each made the compiler wait
// for the load before issuing the next ones.
__device__ __forceinline__ uint32_t elem_word(const void* p, int64_t i, int dtype, bool& hi) {
  const char* b = static_cast<const char*>(p);
  const int64_t off = dtype == GPTQ_F32 ? 4 * i : 2 * i;
  const int mis = static_cast<int>((reinterpret_cast<uintptr_t>(b) + static_cast<uintptr_t>(off)) & 3u);
  hi = (mis & 2) != 0;
  return *reinterpret_cast<const uint32_t*>(b + (off - mis));
}
__device__ __forceinline__ float elem_value(uint32_t w, bool hi, int dtype) {
  const uint16_t h = static_cast<uint16_t>(hi ? (w >> 16) : w);
  const float v16 = dtype == GPTQ_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
  return dtype == GPTQ_F32 ? __builtin_bit_cast(float, w) : v16;
}
__device__ __forceinline__ float load_elem(const void* p, int64_t i, int dtype) {
  bool hi;
  const uint32_t w = elem_word(p, i, dtype, hi);
  return elem_value(w, hi, dtype);
}
__device__ __forceinline__ void store_elem(void* p, int64_t i, int dtype, float v) {
  if (dtype == GPTQ_F32) {
    static_cast<float*>(p)[i] = v;
  } else {
    static_cast<uint16_t*>(p)[i] = dtype == GPTQ_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
  }
}

// (valid_dtype and dtype_size come from plan.hpp)
__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Orders one wave's LDS accesses for the compiler: lanes exchange data
// through LDS, stored by some lanes and read by others, which a single
// thread's view of memory does not order (wave-scope release and acquire
// around a wave barrier; the hardware runs a wave's LDS accesses in order).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ------------------------------------------------------ packed codes ----
// The 32 codes of a chunk (BITS consecutive 32-bit words of an LSB-first bit
// stream) as 16 pairs: codes 2p, 2p + 1 in the low / high 16 bits.
template <int BITS, int PP>
__device__ __forceinline__ uint32_t chunk_pair(const uint32_t (&w)[BITS]) {
  if constexpr (BITS == 4) {
    const uint32_t v = (w[PP / 4] >> (8 * (PP % 4))) & 0xFFu;
    return (v & 0xFu) | ((v >> 4) << 16);
  } else if constexpr (BITS == 2) {
    const uint32_t v = (w[PP / 8] >> (4 * (PP % 8))) & 0xFu;
    return (v & 0x3u) | ((v >> 2) << 16);
  } else if constexpr (BITS == 8) {
    const uint32_t v = w[PP / 2] >> (16 * (PP % 2));
    return (v & 0xFFu) | ((v & 0xFF00u) << 8);
  } else {
    constexpr int b0 = 6 * PP, d = b0 / 32, o = b0 % 32;
    uint64_t v = w[d];
    if constexpr (d + 1 < 3) v |= static_cast<uint64_t>(w[d + 1]) << 32;
    v >>= o;
    return static_cast<uint32_t>(v & 7u) | (static_cast<uint32_t>((v >> 3) & 7u) << 16);
  }
}

}  // namespace gptq
