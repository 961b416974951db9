// Packing formats, dequantisation and the elementwise tensor quantiser.
//
// Native layout: row n of the (N x K) codes is an LSB-first bit stream of
// `bits`-bit fields, pitch = ceil(K * bits / 8) bytes.  Packing writes one
// 32-bit word per thread (aligned pitches) so a wave stores 256 contiguous
// bytes; unpacking reads the one or two bytes that hold a code.
#include "common.hpp"

#include <utility>

namespace gptq {
namespace {

__host__ __device__ inline int64_t pitch_of(int64_t K, int bits) { return (K * bits + 7) / 8; }

__device__ __forceinline__ uint32_t code_at(const uint8_t* __restrict__ row, int64_t pitch, int64_t k, int bits) {
  if (bits == 0) return row[k];
  const int64_t bit = k * bits;
  const int64_t byte = bit >> 3;
  uint32_t v = row[byte];
  if (byte + 1 < pitch) v |= static_cast<uint32_t>(row[byte + 1]) << 8;
  return (v >> (bit & 7)) & ((1u << bits) - 1u);
}

// one 32-bit output word per thread (pitch % 4 == 0)
__global__ void pack_words(const uint8_t* __restrict__ codes, int64_t N, int64_t K, int bits,
                           uint32_t* __restrict__ out, int64_t wpr) {
  const int64_t total = N * wpr;
  const uint32_t mask = (1u << bits) - 1u;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = idx / wpr, w = idx - (idx / wpr) * wpr;
    const int64_t b0 = w * 32;
    const int64_t k_lo = b0 / bits;
    const int64_t k_hi = std::min<int64_t>(K - 1, (b0 + 31) / bits);
    uint32_t word = 0;
    const uint8_t* row = codes + n * K;
    for (int64_t k = k_lo; k <= k_hi; ++k) {
      const uint32_t c = row[k] & mask;
      const int64_t off = k * bits - b0;
      word |= off >= 0 ? (c << off) : (c >> (-off));
    }
    out[idx] = word;
  }
}

// one output byte per thread (any pitch)
__global__ void pack_bytes(const uint8_t* __restrict__ codes, int64_t N, int64_t K, int bits,
                           uint8_t* __restrict__ out, int64_t pitch) {
  const int64_t total = N * pitch;
  const uint32_t mask = (1u << bits) - 1u;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = idx / pitch, b = idx - (idx / pitch) * pitch;
    const int64_t b0 = b * 8;
    const int64_t k_lo = b0 / bits;
    const int64_t k_hi = std::min<int64_t>(K - 1, (b0 + 7) / bits);
    uint32_t v = 0;
    const uint8_t* row = codes + n * K;
    for (int64_t k = k_lo; k <= k_hi; ++k) {
      const uint32_t c = row[k] & mask;
      const int64_t off = k * bits - b0;
      v |= off >= 0 ? (c << off) : (c >> (-off));
    }
    out[idx] = static_cast<uint8_t>(v & 0xffu);
  }
}

__global__ void unpack_k(const uint8_t* __restrict__ packed, int64_t N, int64_t K, int bits,
                         uint8_t* __restrict__ codes, int64_t pitch) {
  const int64_t total = N * K;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = idx / K, k = idx - (idx / K) * K;
    codes[idx] = static_cast<uint8_t>(code_at(packed + n * pitch, pitch, k, bits));
  }
}

// GPTQ.pack_weights layout from (N x K) codes: out is (K x N/epb)
__global__ void pack_ref_layout_k(const uint8_t* __restrict__ codes, int64_t N, int64_t K, int bits,
                                  uint8_t* __restrict__ out) {
  const int epb = bits == 4 ? 2 : (bits == 2 ? 4 : 1);
  const int64_t cols = N / epb;
  const int64_t total = K * cols;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t k = idx / cols, i = idx - (idx / cols) * cols;
    uint32_t v;
    if (bits == 4) {
      v = 16u * codes[(2 * i) * K + k] + codes[(2 * i + 1) * K + k];
    } else if (bits == 2) {
      v = 64u * codes[(4 * i) * K + k] + 16u * codes[(4 * i + 1) * K + k] + 4u * codes[(4 * i + 2) * K + k] +
          codes[(4 * i + 3) * K + k];
    } else {
      v = codes[i * K + k];
    }
    out[idx] = static_cast<uint8_t>(v & 0xffu);
  }
}

#pragma clang fp contract(off)
// (q - z) * s in fp32 (no FMA), stored as fp32 or rounded to fp16 / bf16
__global__ void dequant_k(const uint8_t* __restrict__ packed, int bits, const void* __restrict__ scales,
                          const void* __restrict__ zeros, int sz_dtype, const int32_t* __restrict__ g_idx, int gs,
                          int64_t ngroups, int64_t N, int64_t K, void* __restrict__ out, int out_dtype,
                          int64_t pitch) {
  const int64_t total = N * K;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = idx / K, k = idx - (idx / K) * K;
    // out-of-range group indices are clamped so that no read leaves the arrays
    const int64_t g = g_idx ? std::min<int64_t>(std::max<int64_t>(g_idx[k], 0), ngroups - 1) : k / gs;
    const float q = static_cast<float>(code_at(packed + n * pitch, pitch, k, bits));
    const float z = load_elem(zeros, n * ngroups + g, sz_dtype);
    const float s = load_elem(scales, n * ngroups + g, sz_dtype);
    const float d = q - z;
    store_elem(out, idx, out_dtype, d * s);
  }
}

template <int BITS, int PP>
__device__ __forceinline__ void dequant_pair(const uint32_t (&w)[BITS], float z, float s, float (&v)[32]) {
  const uint32_t cp = chunk_pair<BITS, PP>(w);
  const float d0 = static_cast<float>(cp & 0xFFFFu) - z, d1 = static_cast<float>(cp >> 16) - z;
  v[2 * PP] = d0 * s;
  v[2 * PP + 1] = d1 * s;
}
template <int BITS, int... PP>
__device__ __forceinline__ void dequant_pairs(const uint32_t (&w)[BITS], float z, float s, float (&v)[32],
                                              std::integer_sequence<int, PP...>) {
  (dequant_pair<BITS, PP>(w, z, s, v), ...);
}

// The same for K % 32 == 0 and groups of a multiple of 32 columns: one thread
// per 32-code chunk (one group), one 4 * BITS-byte load and 64 (128 for fp32)
// contiguous bytes stored; consecutive threads take consecutive chunks.
template <int BITS>
__global__ __launch_bounds__(256) void dequant_chunks_k(const uint8_t* __restrict__ packed,
                                                        const void* __restrict__ scales,
                                                        const void* __restrict__ zeros, int sz_dtype, int gs,
                                                        int64_t ngroups, int64_t N, int64_t nch, int64_t pitch,
                                                        void* __restrict__ out, int out_dtype) {
  const int64_t total = N * nch;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = idx / nch, c = idx - n * nch;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(packed + n * pitch + c * 4 * BITS);
    uint32_t w[BITS];
    if constexpr (BITS == 4) {
      const uint4 v = *reinterpret_cast<const uint4*>(src);
      w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (BITS == 8) {
      const uint4 v0 = reinterpret_cast<const uint4*>(src)[0], v1 = reinterpret_cast<const uint4*>(src)[1];
      w[0] = v0.x; w[1] = v0.y; w[2] = v0.z; w[3] = v0.w; w[4] = v1.x; w[5] = v1.y; w[6] = v1.z; w[7] = v1.w;
    } else if constexpr (BITS == 2) {
      const uint2 v = *reinterpret_cast<const uint2*>(src);
      w[0] = v.x; w[1] = v.y;
    } else {
      w[0] = src[0]; w[1] = src[1]; w[2] = src[2];
    }
    const int64_t g = (c * 32) / gs;
    const float z = load_elem(zeros, n * ngroups + g, sz_dtype);
    const float s = load_elem(scales, n * ngroups + g, sz_dtype);
    float v[32];
    dequant_pairs<BITS>(w, z, s, v, std::make_integer_sequence<int, 16>{});
    if (out_dtype == GPTQ_F32) {
      uint4* dst = reinterpret_cast<uint4*>(static_cast<float*>(out) + idx * 32);
#pragma unroll
      for (int q = 0; q < 8; ++q)
        dst[q] = uint4{__float_as_uint(v[4 * q]), __float_as_uint(v[4 * q + 1]), __float_as_uint(v[4 * q + 2]),
                       __float_as_uint(v[4 * q + 3])};
    } else {
      const bool bf = out_dtype == GPTQ_BF16;
      uint32_t h[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const uint32_t lo = bf ? f32_to_bf16_bits(v[2 * q]) : f32_to_f16_bits(v[2 * q]);
        const uint32_t hi = bf ? f32_to_bf16_bits(v[2 * q + 1]) : f32_to_f16_bits(v[2 * q + 1]);
        h[q] = lo | (hi << 16);
      }
      uint4* dst = reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + idx * 32);
#pragma unroll
      for (int q = 0; q < 4; ++q) dst[q] = uint4{h[4 * q], h[4 * q + 1], h[4 * q + 2], h[4 * q + 3]};
    }
  }
}

// -------------------------------------------------- flat tensor quantiser --
// one wave per group: s = (max - min) / maxq, z = -min / s (unrounded)
__global__ __launch_bounds__(256) void tensor_params_k(const void* __restrict__ x, int dtype, int64_t n, int gs,
                                                       int maxq, float* __restrict__ scales,
                                                       float* __restrict__ zeros, int64_t ngroups) {
  const int64_t g = blockIdx.x * 4LL + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (g >= ngroups) return;
  const int64_t a = g * gs, b = std::min<int64_t>(a + gs, n);
  float mn = INFINITY, mx = -INFINITY;
  for (int64_t i = a + lane; i < b; i += 64) {
    const float v = load_elem(x, i, dtype);
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    mn = fminf(mn, __shfl_xor(mn, o, 64));
    mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  }
  if (lane == 0) {
    const float s = (mx - mn) / static_cast<float>(maxq);
    scales[g] = s;
    zeros[g] = -mn / s;
  }
}

__global__ void tensor_quant_k(const void* __restrict__ x, int dtype, int64_t n, int gs, int maxq,
                               const float* __restrict__ scales, const float* __restrict__ zeros,
                               int8_t* __restrict__ q) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t g = i / gs;
    const float v = roundf(load_elem(x, i, dtype) / scales[g] + zeros[g]);
    const float c = fminf(fmaxf(v, 0.0f), static_cast<float>(maxq));
    q[i] = static_cast<int8_t>(static_cast<uint8_t>(static_cast<int>(c)));
  }
}

__global__ void tensor_dequant_k(const int8_t* __restrict__ q, int64_t n, int gs, const float* __restrict__ scales,
                                 const float* __restrict__ zeros, float* __restrict__ out) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t g = i / gs;
    const float d = static_cast<float>(q[i]) - zeros[g];
    out[i] = d * scales[g];
  }
}
#pragma clang fp contract(on)

unsigned blocks_for(int64_t n) { return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(cdiv(n, 256), 65536))); }

bool valid_bits(int b) { return b == 2 || b == 3 || b == 4 || b == 8; }

}  // namespace
}  // namespace gptq

using namespace gptq;

extern "C" int gptq_pack(const uint8_t* codes, int64_t N, int64_t K, int bits, uint8_t* packed,
                         gptq_stream_t stream) {
  clear_error();
  GPTQ_REQUIRE(codes && packed, GPTQ_ERR_ARG, "pack: null pointer");
  GPTQ_REQUIRE(valid_bits(bits), GPTQ_ERR_ARG, "pack: bits must be 2, 3, 4 or 8 (got %d)", bits);
  GPTQ_REQUIRE(N > 0 && K > 0, GPTQ_ERR_SHAPE, "pack: bad shape");
  const int64_t pitch = pitch_of(K, bits);
  hipStream_t st = as_hip(stream);
  if (pitch % 4 == 0 && reinterpret_cast<uintptr_t>(packed) % 4 == 0) {
    const int64_t wpr = pitch / 4;
    hipLaunchKernelGGL(pack_words, dim3(blocks_for(N * wpr)), dim3(256), 0, st, codes, N, K, bits,
                       reinterpret_cast<uint32_t*>(packed), wpr);
  } else {
    hipLaunchKernelGGL(pack_bytes, dim3(blocks_for(N * pitch)), dim3(256), 0, st, codes, N, K, bits, packed, pitch);
  }
  return check_launch("pack");
}

extern "C" int gptq_unpack(const uint8_t* packed, int64_t N, int64_t K, int bits, uint8_t* codes,
                           gptq_stream_t stream) {
  clear_error();
  GPTQ_REQUIRE(codes && packed, GPTQ_ERR_ARG, "unpack: null pointer");
  GPTQ_REQUIRE(valid_bits(bits), GPTQ_ERR_ARG, "unpack: bits must be 2, 3, 4 or 8 (got %d)", bits);
  GPTQ_REQUIRE(N > 0 && K > 0, GPTQ_ERR_SHAPE, "unpack: bad shape");
  hipLaunchKernelGGL(unpack_k, dim3(blocks_for(N * K)), dim3(256), 0, as_hip(stream), packed, N, K, bits, codes,
                     pitch_of(K, bits));
  return check_launch("unpack");
}

extern "C" int gptq_pack_reference_layout(const uint8_t* codes, int64_t N, int64_t K, int bits, uint8_t* out,
                                          gptq_stream_t stream) {
  clear_error();
  GPTQ_REQUIRE(codes && out, GPTQ_ERR_ARG, "pack_reference_layout: null pointer");
  GPTQ_REQUIRE(valid_bits(bits), GPTQ_ERR_ARG, "pack_reference_layout: bits=%d", bits);
  const int epb = bits == 4 ? 2 : (bits == 2 ? 4 : 1);
  GPTQ_REQUIRE(N > 0 && K > 0 && N % epb == 0, GPTQ_ERR_SHAPE,
               "pack_reference_layout: N=%lld must be a multiple of %d (core/gptq.py:237,248)", (long long)N, epb);
  hipLaunchKernelGGL(pack_ref_layout_k, dim3(blocks_for(K * (N / epb))), dim3(256), 0, as_hip(stream), codes, N, K,
                     bits, out);
  return check_launch("pack_reference_layout");
}

extern "C" int gptq_dequant_to(const uint8_t* packed, int bits, const void* scales, const void* zeros, int sz_dtype,
                               const int32_t* g_idx, int group_size, int64_t ngroups, int64_t N, int64_t K, void* out,
                               int out_dtype, gptq_stream_t stream) {
  clear_error();
  GPTQ_REQUIRE(packed && scales && zeros && out, GPTQ_ERR_ARG, "dequant: null pointer");
  GPTQ_REQUIRE(bits == 0 || valid_bits(bits), GPTQ_ERR_ARG, "dequant: bits=%d", bits);
  GPTQ_REQUIRE(valid_dtype(sz_dtype) && valid_dtype(out_dtype), GPTQ_ERR_DTYPE, "dequant: bad scale or output dtype");
  GPTQ_REQUIRE(N > 0 && K > 0 && ngroups > 0 && (g_idx || group_size > 0), GPTQ_ERR_SHAPE, "dequant: bad shape");
  GPTQ_REQUIRE(g_idx || cdiv(K, group_size) <= ngroups, GPTQ_ERR_SHAPE, "dequant: %lld groups < ceil(K/g)",
               (long long)ngroups);
  const int64_t pitch = bits == 0 ? K : pitch_of(K, bits);
  hipStream_t st = as_hip(stream);
  const bool aligned = (reinterpret_cast<uintptr_t>(packed) % 16) == 0 && (reinterpret_cast<uintptr_t>(out) % 16) == 0;
  if (!g_idx && bits != 0 && K % 32 == 0 && group_size % 32 == 0 && aligned) {
    const int64_t nch = K / 32;
    const unsigned blocks = static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(cdiv(N * nch, 256), 16384)));
    switch (bits) {
      case 4: hipLaunchKernelGGL(dequant_chunks_k<4>, dim3(blocks), dim3(256), 0, st, packed, scales, zeros, sz_dtype,
                                 group_size, ngroups, N, nch, pitch, out, out_dtype); break;
      case 3: hipLaunchKernelGGL(dequant_chunks_k<3>, dim3(blocks), dim3(256), 0, st, packed, scales, zeros, sz_dtype,
                                 group_size, ngroups, N, nch, pitch, out, out_dtype); break;
      case 2: hipLaunchKernelGGL(dequant_chunks_k<2>, dim3(blocks), dim3(256), 0, st, packed, scales, zeros, sz_dtype,
                                 group_size, ngroups, N, nch, pitch, out, out_dtype); break;
      default: hipLaunchKernelGGL(dequant_chunks_k<8>, dim3(blocks), dim3(256), 0, st, packed, scales, zeros,
                                  sz_dtype, group_size, ngroups, N, nch, pitch, out, out_dtype); break;
    }
    return check_launch("dequant");
  }
  hipLaunchKernelGGL(dequant_k, dim3(blocks_for(N * K)), dim3(256), 0, st, packed, bits, scales, zeros, sz_dtype, g_idx,
                     group_size, ngroups, N, K, out, out_dtype, pitch);
  return check_launch("dequant");
}

extern "C" int gptq_dequant(const uint8_t* packed, int bits, const void* scales, const void* zeros, int sz_dtype,
                            const int32_t* g_idx, int group_size, int64_t ngroups, int64_t N, int64_t K, float* out,
                            gptq_stream_t stream) {
  return gptq_dequant_to(packed, bits, scales, zeros, sz_dtype, g_idx, group_size, ngroups, N, K, out, GPTQ_F32,
                         stream);
}

extern "C" int gptq_quantize_tensor(const void* x, int dtype, int64_t n, int bits, int group_size, int flags,
                                    int8_t* q, float* scales, float* zeros, gptq_stream_t stream) {
  clear_error();
  GPTQ_REQUIRE(x && q && scales && zeros, GPTQ_ERR_ARG, "quantize_tensor: null pointer");
  GPTQ_REQUIRE(valid_dtype(dtype), GPTQ_ERR_DTYPE, "quantize_tensor: bad dtype");
  GPTQ_REQUIRE(bits >= 1 && bits <= 8 && group_size > 0 && n > 0, GPTQ_ERR_ARG, "quantize_tensor: bad args");
  const int maxq = (1 << bits) - 1;
  const int64_t ng = cdiv(n, group_size);
  hipStream_t st = as_hip(stream);
  if (!(flags & GPTQ_TENSOR_PARAMS_GIVEN)) {
    hipLaunchKernelGGL(tensor_params_k, dim3(static_cast<unsigned>(cdiv(ng, 4))), dim3(256), 0, st, x, dtype, n,
                       group_size, maxq, scales, zeros, ng);
    int rc = check_launch("tensor_params");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(tensor_quant_k, dim3(blocks_for(n)), dim3(256), 0, st, x, dtype, n, group_size, maxq, scales,
                     zeros, q);
  return check_launch("tensor_quant");
}

extern "C" int gptq_dequantize_tensor(const int8_t* q, int64_t n, int group_size, const float* scales,
                                      const float* zeros, float* out, gptq_stream_t stream) {
  clear_error();
  GPTQ_REQUIRE(q && scales && zeros && out, GPTQ_ERR_ARG, "dequantize_tensor: null pointer");
  GPTQ_REQUIRE(group_size > 0 && n > 0, GPTQ_ERR_ARG, "dequantize_tensor: bad args");
  hipLaunchKernelGGL(tensor_dequant_k, dim3(blocks_for(n)), dim3(256), 0, as_hip(stream), q, n, group_size, scales,
                     zeros, out);
  return check_launch("dequantize_tensor");
}
