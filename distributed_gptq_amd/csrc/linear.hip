// Dequant-matmul y = x @ dequant(W)^T (+ bias) on gfx950: the gptq::linear op.
//
// Weight rows are the native LSB-first bit streams (pitch ceil(K*bits/8)),
// scales/zeros (N x ngroups), group of column k = k / group_size (or g_idx).
// sum_k x_k (q_k - z) s is evaluated per chunk as s * (sum_k x_k q_k -
// z * sum_k x_k) with exact small-integer codes in fp16/bf16 and fp32
// accumulation, so a code costs one packed decode step and half a v_dot2.
//
//  * gemv_m1_k (M = 1): persistent workgroups; each lane loads the x values of
//    its 32-code chunks once, permutes them into the order the packed words
//    decode into fp16/bf16 pairs (one shift and one and-or per pair) and keeps
//    them in registers across all rows it visits; no LDS, no barrier.
//  * gemv_k (M <= 4): 4 waves per workgroup share x staged in LDS; a wave
//    walks 4 weight rows at a time, lane l taking 128-bit chunks l, l+64, ...
//    of each row (a wave load covers 1 KiB of contiguous codes).  Within a
//    chunk, codes are paired the way the packed word yields them cheaply
//    ((0,4),(1,5).. for 4-bit), and x is stored in LDS in that order.
//  * dq_split_k / dq_tile_k (M > 4, K % 128 == 0, group size % 32 == 0):
//    codes are dequantised to the activation type ((q - z) exact, one
//    rounding of the product with s; for fp16 with integer zeros in [0, 1023]
//    a packed magic-exponent form), written to LDS and fed to
//    v_mfma_f32_16x16x32_{f16,bf16} (dq_split_k: the waves of a workgroup
//    split K over 128-column blocks and reduce through LDS; dq_tile_k:
//    128-row weight tiles x 64/128 activation rows, double-buffered LDS).
//  * dq_rx_k (16 < M <= 384): the codes are decoded in registers straight
//    into the MFMA operands; X is staged in LDS by loader waves.  Layers of
//    fewer than 192 x 128 rows split K over workgroups when the caller gives
//    a workspace for the fp32 partial sums (splitk_reduce_k adds them in
//    split order).
//  * dq_mfma_k (other M > 4 layouts): 16 weight rows x 16 activation rows per
//    MFMA step with zero points folded per group, 4 waves splitting K.
//  * linear_generic: any layout (fp32 x, g_idx, ragged K): one wave per
//    output, fp32.
#include "common.hpp"

#include <mutex>

namespace gptq {
namespace {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int BITS> struct Fmt;
template <> struct Fmt<4> { static constexpr int CB = 32, NW = 4; };
template <> struct Fmt<2> { static constexpr int CB = 64, NW = 4; };
template <> struct Fmt<8> { static constexpr int CB = 16, NW = 4; };
template <> struct Fmt<3> { static constexpr int CB = 128, NW = 12; };

// chunk-local code index held by LDS slot s (pairs of slots = decoded pairs)
template <int BITS>
__device__ __forceinline__ int slot_code(int s) {
  if constexpr (BITS == 4) {
    const int d = s >> 3, j = s & 7;
    return 8 * d + (j >> 1) + 4 * (j & 1);
  } else if constexpr (BITS == 2) {
    const int d = s >> 4, j = s & 15;
    return 16 * d + (j >> 1) + 8 * (j & 1);
  } else {
    return s;
  }
}

// codes of pair p of a chunk as two 16-bit integers (lo, hi)
template <int BITS, int P>
__device__ __forceinline__ uint32_t decode_pair(const uint32_t* dw) {
  if constexpr (BITS == 4) {
    constexpr int d = P / 4, i = P % 4;
    return (dw[d] >> (4 * i)) & 0x000F000Fu;
  } else if constexpr (BITS == 2) {
    constexpr int d = P / 8, i = P % 8;
    return (dw[d] >> (2 * i)) & 0x00030003u;
  } else if constexpr (BITS == 8) {
    constexpr int d = P / 2, i = P % 2;
    const uint32_t w = dw[d] >> (16 * i);
    return (w & 0xFFu) | ((w & 0xFF00u) << 8);
  } else {
    constexpr int b0 = 6 * P;  // bit offset of code 2P
    constexpr int d = b0 / 32, o = b0 % 32;
    uint64_t v = dw[d];
    if constexpr (d + 1 < Fmt<3>::NW) v |= static_cast<uint64_t>(dw[d + 1]) << 32;
    v >>= o;
    return static_cast<uint32_t>(v & 7u) | (static_cast<uint32_t>((v >> 3) & 7u) << 16);
  }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// bf16 codes carry a magic offset of 128 (0x4300 | code is 128 + code for
// code < 128); 8-bit codes do not fit under it and are converted exactly.
template <int BITS, bool BF16>
struct Magic {
  static constexpr bool kBF16Offset = BF16 && BITS != 8;
  static constexpr float kOffset = kBF16Offset ? 128.0f : 0.0f;
};

// two small integers (lo, hi halves of c) -> the pair of bf16 values, exact
__device__ __forceinline__ uint32_t bf16_pair_exact(uint32_t c) {
  const uint32_t lo = __float_as_uint(static_cast<float>(c & 0xffffu));
  const uint32_t hi = __float_as_uint(static_cast<float>(c >> 16));
  return (lo >> 16) | (hi & 0xffff0000u);
}

// dot of the chunk's decoded codes with x pairs; returns sum x*(code + off)
// where off = Magic::kOffset (fp16: the 1024 magic is subtracted exactly with
// a packed fp16 op; bf16: the 128 magic is left in and corrected by the
// caller through the x sums).
template <int BITS, bool BF16, int P>
__device__ __forceinline__ float chunk_dot_pair(const uint32_t* dw, uint32_t xpair, float acc) {
  const uint32_t c = decode_pair<BITS, P>(dw);
  if constexpr (!BF16) {
    const uint32_t t = c | 0x64006400u;                 // 1024 + code, fp16
    f16x2 h = __builtin_bit_cast(f16x2, t) - f16x2{1024.0f16, 1024.0f16};
    return __builtin_amdgcn_fdot2(h, __builtin_bit_cast(f16x2, xpair), acc, false);
  } else {
    const uint32_t t = Magic<BITS, BF16>::kBF16Offset ? (c | 0x43004300u) : bf16_pair_exact(c);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, t), __builtin_bit_cast(bf16x2, xpair), acc,
                                           false);
  }
}

template <int BITS, bool BF16, int... Ps>
__device__ __forceinline__ float chunk_dot(const uint32_t* dw, const uint32_t* xp, std::integer_sequence<int, Ps...>) {
  float acc = 0.0f;
  ((acc = chunk_dot_pair<BITS, BF16, Ps>(dw, xp[Ps], acc)), ...);
  return acc;
}

struct LinArgs {
  const uint16_t* x;
  int64_t M;
  const uint8_t* packed;
  int64_t pitch;
  const void* scales;
  const void* zeros;
  int sz_dtype;
  int gs;
  int64_t ngroups;
  const void* bias;
  int bias_dtype;
  int64_t N, K;
  uint16_t* y;
  int y_dtype;
  float* part = nullptr;      // split-K partial sums (fp32 [S][M][N]) or null
  size_t part_bytes = 0;      // bytes available at part
};

constexpr int kRB = 4;  // weight rows per wave pass

template <int BITS, bool BF16, int MV>
__global__ __launch_bounds__(256) void gemv_k(LinArgs a) {
  using F = Fmt<BITS>;
  constexpr int CB = F::CB;
  constexpr int NP = CB / 2;  // pairs per chunk
  extern __shared__ uint32_t lds[];
  const int64_t K = a.K;
  const int64_t nch = K / CB;
  uint16_t* xs = reinterpret_cast<uint16_t*>(lds);          // MV x K (slot order)
  float* xsum = reinterpret_cast<float*>(lds + MV * K / 2);  // MV x nch
  const int tid = threadIdx.x;
  for (int64_t i = tid; i < MV * K; i += 256) {
    const int64_t m = i / K, s = i - (i / K) * K;
    const int64_t c = s / CB;
    const int cs = static_cast<int>(s - c * CB);
    xs[i] = a.x[m * K + c * CB + slot_code<BITS>(cs)];
  }
  __syncthreads();
  for (int64_t i = tid; i < MV * nch; i += 256) {
    const int64_t m = i / nch, c = i - (i / nch) * nch;
    float s = 0.0f;
    for (int e = 0; e < CB; ++e) {
      const uint16_t b = xs[m * K + c * CB + e];
      s += BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
    }
    xsum[i] = s;
  }
  __syncthreads();

  const int lane = tid & 63;
  const int64_t nwaves = static_cast<int64_t>(gridDim.x) * 4;
  const int64_t nbatches = cdiv(a.N, kRB);
  for (int64_t rb = blockIdx.x * 4LL + (tid >> 6); rb < nbatches; rb += nwaves) {
    const int64_t n0 = rb * kRB;
    float acc[kRB][MV];
#pragma unroll
    for (int r = 0; r < kRB; ++r)
#pragma unroll
      for (int m = 0; m < MV; ++m) acc[r][m] = 0.0f;
#pragma unroll 2
    for (int64_t c = lane; c < nch; c += 64) {
      uint32_t dw[kRB][F::NW];
#pragma unroll
      for (int r = 0; r < kRB; ++r) {
        const int64_t n = std::min<int64_t>(n0 + r, a.N - 1);
        const u32x4* src = reinterpret_cast<const u32x4*>(a.packed + n * a.pitch + c * (CB * BITS / 8));
#pragma unroll
        for (int v = 0; v < F::NW / 4; ++v) {
          const u32x4 t = __builtin_nontemporal_load(src + v);
          dw[r][4 * v] = t[0]; dw[r][4 * v + 1] = t[1]; dw[r][4 * v + 2] = t[2]; dw[r][4 * v + 3] = t[3];
        }
      }
      const int64_t g = static_cast<int>(c * CB) / a.gs;  // 32-bit division (K < 2^31)
      float sc[kRB], zc[kRB];
#pragma unroll
      for (int r = 0; r < kRB; ++r) {
        const int64_t n = std::min<int64_t>(n0 + r, a.N - 1);
        sc[r] = load_elem(a.scales, n * a.ngroups + g, a.sz_dtype);
        zc[r] = load_elem(a.zeros, n * a.ngroups + g, a.sz_dtype);
        zc[r] += Magic<BITS, BF16>::kOffset;
      }
#pragma unroll
      for (int m = 0; m < MV; ++m) {
        uint32_t xp[NP];
        const u32x4* xv = reinterpret_cast<const u32x4*>(xs + m * K + c * CB);
#pragma unroll
        for (int v = 0; v < NP / 4; ++v) {
          const u32x4 t = xv[v];
          xp[4 * v] = t[0]; xp[4 * v + 1] = t[1]; xp[4 * v + 2] = t[2]; xp[4 * v + 3] = t[3];
        }
        const float xsm = xsum[m * nch + c];
#pragma unroll
        for (int r = 0; r < kRB; ++r) {
          const float d = chunk_dot<BITS, BF16>(dw[r], xp, std::make_integer_sequence<int, NP>{});
          acc[r][m] += sc[r] * (d - zc[r] * xsm);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < kRB; ++r)
#pragma unroll
      for (int m = 0; m < MV; ++m) acc[r][m] = wave_sum(acc[r][m]);
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < kRB; ++r) {
        const int64_t n = n0 + r;
        if (n >= a.N) continue;
        const float b = a.bias ? load_elem(a.bias, n, a.bias_dtype) : 0.0f;
#pragma unroll
        for (int m = 0; m < MV; ++m) store_elem(a.y, m * a.N + n, a.y_dtype, acc[r][m] + b);
      }
    }
  }
}

// ------------------------------------------------------------ M = 1 GEMV --
// 32-code chunks for every width (BITS dwords per chunk).  Pair p of a chunk
// holds the codes (pair_a(p), pair_b(p)): the two codes one and-or lifts out
// of a packed dword into the low and high halves, under the fp16 magic
// exponent 0x6400 (value 1024 + code) or the bf16 one 0x4300 (128 + code).
// With fp16, a mask need not sit at bit 0: (w & 0x00F000F0) | 0x64006400 is
// 1024 + 16 * code, exact, so 4-bit pairs need one shift per dword and 2-bit
// pairs one per dword too; pairs then fall into "classes" by the power of
// two m_c their codes carry, each with its own accumulator, and
//   sum_k x_k (q_k - z) = sum_c acc_c / m_c - sum_c (off / m_c + z) X_c
// where X_c sums the x values of class c.  The x pairs are stored in the
// same order as the pairs, so each costs one and-or and one v_dot2.
template <int BITS>
__host__ __device__ constexpr int pair_a(int p) {
  return BITS == 4 ? 8 * (p / 4) + p % 4 : BITS == 2 ? 16 * (p / 8) + p % 8 : BITS == 8 ? 4 * (p / 2) + p % 2 : p;
}
template <int BITS>
__host__ __device__ constexpr int pair_b(int p) {
  return pair_a<BITS>(p) + (BITS == 4 ? 4 : BITS == 2 ? 8 : BITS == 8 ? 2 : 16);
}

// 3-bit codes with fp16 activations pair code k with code k + 8 (k in 0..7,
// 16..23): 24 bits apart, so both sit at the same offset (3k mod 8) inside
// their bytes.  One byte permute gathers the two 16-bit windows that hold
// them, one and-or masks them under the magic exponent (1024 + 2^s * code,
// exact for s <= 7), and the pair's class is its bit offset s.
__host__ __device__ constexpr int p3_lo(int p) { return p < 8 ? p : p + 8; }

template <int BITS, bool BF16>
struct M1Fmt {
  static constexpr bool kPerm3 = BITS == 3 && !BF16;
  // scale classes: fp16 4-bit pairs alternate x1 / x16; fp16 2-bit cycle x1 x4 x16 x64;
  // fp16 3-bit pairs carry 2^s for their bit offset s in 0..7
  static constexpr int NCLS = BF16 ? 1 : BITS == 4 ? 2 : BITS == 2 ? 4 : BITS == 3 ? 8 : 1;
  static constexpr float kOff = BF16 ? (BITS == 8 ? 0.0f : 128.0f) : 1024.0f;
  static constexpr int cls(int p) { return kPerm3 ? (3 * p3_lo(p)) % 8 : p % NCLS; }
  static constexpr float mult(int c) { return static_cast<float>(1 << (kPerm3 ? c : BITS * c)); }
  static constexpr int pa(int p) { return kPerm3 ? p3_lo(p) : pair_a<BITS>(p); }
  static constexpr int pb(int p) { return kPerm3 ? p3_lo(p) + 8 : pair_b<BITS>(p); }
};

// byte-permute selector and source dword of fp16 3-bit pair P: output bytes
// (j, j + 1, j + 3, j + 4) of the 12-byte chunk, j = 3k / 8, read from the
// dword pair (d, d + 1); a byte the code does not reach selects zero (0x0c)
template <int P>
struct Perm3 {
  static constexpr int k = p3_lo(P), j = 3 * k / 8, s = 3 * k % 8;
  static constexpr int d = j / 4 < 1 ? 0 : 1;
  static constexpr uint32_t byte(int b, bool need) { return need ? static_cast<uint32_t>(b - 4 * d) : 0x0cu; }
  static constexpr uint32_t sel = byte(j, true) | (byte(j + 1, s + 3 > 8) << 8) | (byte(j + 3, true) << 16) |
                                  (byte(j + 4, s + 3 > 8) << 24);
  static constexpr uint32_t mask = (7u << s) | (7u << (s + 16));
  static_assert(j + 3 - 4 * d <= 7 && (s + 3 <= 8 || j + 4 - 4 * d <= 7), "3-bit pair outside its dword pair");
};

// pair P of the chunk with the magic exponent already or-ed in
template <int BITS, bool BF16, int P>
__device__ __forceinline__ uint32_t m1_pair(const uint32_t* dw, uint32_t magic) {
  if constexpr (BITS == 4) {
    constexpr int d = P / 4, i = P % 4;
    if constexpr (!BF16) {
      const uint32_t w = (i >= 2) ? (dw[d] >> 8) : dw[d];
      return (w & (0x000F000Fu << (4 * (i & 1)))) | magic;
    } else {
      return ((dw[d] >> (4 * i)) & 0x000F000Fu) | magic;
    }
  } else if constexpr (BITS == 2) {
    constexpr int d = P / 8, i = P % 8;
    if constexpr (!BF16) {
      const uint32_t w = (i >= 4) ? (dw[d] >> 8) : dw[d];
      return (w & (0x00030003u << (2 * (i & 3)))) | magic;
    } else {
      return ((dw[d] >> (2 * i)) & 0x00030003u) | magic;
    }
  } else if constexpr (BITS == 8) {
    constexpr int d = P / 2, i = P % 2;
    const uint32_t w = dw[d] >> (8 * i);
    if constexpr (!BF16) return (w & 0x00FF00FFu) | magic;
    else return bf16_pair_exact(w & 0x00FF00FFu);
  } else if constexpr (!BF16) {
    using Q = Perm3<P>;
    const uint32_t t = __builtin_amdgcn_perm(dw[Q::d + 1], dw[Q::d], Q::sel);
    return (t & Q::mask) | magic;
  } else {
    // 3-bit: code P at bit 3P, code P + 16 at bit 3P + 48 (funnel shifts)
    constexpr int b0 = 3 * P, b1 = 3 * P + 32;
    constexpr int d0 = b0 / 32, o0 = b0 % 32, d1 = b1 / 32, o1 = b1 % 32;
    const uint32_t lo = (o0 == 0 || d0 + 1 >= 3) ? (dw[d0] >> o0) : __builtin_amdgcn_alignbit(dw[d0 + 1], dw[d0], o0);
    const uint32_t hi = (o1 == 0 || d1 + 1 >= 3) ? (dw[d1] >> o1) : __builtin_amdgcn_alignbit(dw[d1 + 1], dw[d1], o1);
    return (lo & 7u) | (hi & 0x70000u) | magic;
  }
}

template <bool BF16>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
  if constexpr (BF16)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), acc, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), acc, false);
}

template <int BITS, bool BF16, int... Ps>
__device__ __forceinline__ void m1_dot(const uint32_t* dw, const uint32_t* xp, uint32_t magic,
                                       float (&acc)[M1Fmt<BITS, BF16>::NCLS], std::integer_sequence<int, Ps...>) {
  using F = M1Fmt<BITS, BF16>;
#pragma unroll
  for (int c = 0; c < F::NCLS; ++c) acc[c] = 0.0f;
  ((acc[F::cls(Ps)] = dot2<BF16>(m1_pair<BITS, BF16, Ps>(dw, magic), xp[Ps], acc[F::cls(Ps)])), ...);
}

// natural-order x of one 32-code chunk (64 bytes)
__device__ __forceinline__ void load_x_raw(const uint16_t* __restrict__ x, int c, u32x4 (&raw)[4]) {
  const u32x4* src = reinterpret_cast<const u32x4*>(x + static_cast<int64_t>(c) * 32);
#pragma unroll
  for (int v = 0; v < 4; ++v) raw[v] = src[v];
}

// x pairs of one 32-code chunk in pair order, their total X and the magic
// correction Y = sum_c (off / m_c) X_c
template <int BITS, bool BF16>
__device__ __forceinline__ void prep_x_chunk(const u32x4 (&raw)[4], uint32_t (&xr)[16], float& xs, float& ys) {
  using F = M1Fmt<BITS, BF16>;
  uint32_t d[16];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    d[4 * v] = raw[v][0]; d[4 * v + 1] = raw[v][1]; d[4 * v + 2] = raw[v][2]; d[4 * v + 3] = raw[v][3];
  }
#pragma unroll
  for (int p = 0; p < 16; ++p) {
    const int ia = F::pa(p), ib = F::pb(p);
    const uint32_t lo = (d[ia >> 1] >> (16 * (ia & 1))) & 0xffffu;
    const uint32_t hi = (d[ib >> 1] >> (16 * (ib & 1))) & 0xffffu;
    xr[p] = lo | (hi << 16);
  }
  const uint32_t one = BF16 ? 0x3F803F80u : 0x3C003C00u;
  float cs[F::NCLS];
#pragma unroll
  for (int c = 0; c < F::NCLS; ++c) cs[c] = 0.0f;
#pragma unroll
  for (int p = 0; p < 16; ++p) cs[F::cls(p)] = dot2<BF16>(xr[p], one, cs[F::cls(p)]);
  xs = 0.0f;
  ys = 0.0f;
#pragma unroll
  for (int c = 0; c < F::NCLS; ++c) {
    xs += cs[c];
    ys += (F::kOff / F::mult(c)) * cs[c];
  }
}

constexpr int kBufDword3 = 0x00020000;  // raw buffer descriptor word 3 (gfx950)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           kBufDword3);
}

// codes, scales and zeros of RB rows x MAXC chunks of one lane
template <int BITS, int MAXC, int RB>
struct M1Batch {
  uint32_t dw[RB][MAXC][BITS];
  uint16_t s[RB][MAXC], z[RB][MAXC];
  uint32_t b32;  // lane r < RB: bias of row n0 + r when the bias is fp32
  uint16_t b16;  // ... when it is 16-bit
};

// Each row is addressed through its own buffer descriptors (wave-uniform,
// scalar registers) and a lane's chunk offsets are loop-invariant vector
// registers, so a load costs no address arithmetic.  Rows at or beyond N get
// empty descriptors: their loads return zeros and touch no memory.
template <int BITS, int MAXC, int RB>
__device__ __forceinline__ void load_m1_batch(const LinArgs& a, int64_t n0, const uint32_t (&coff)[MAXC],
                                              const uint32_t (&goff)[MAXC], M1Batch<BITS, MAXC, RB>& b) {
  const uint16_t* sc = static_cast<const uint16_t*>(a.scales);
  const uint16_t* zr = static_cast<const uint16_t*>(a.zeros);
  {
    // bias of the batch's rows, one per lane, issued with the batch (never
    // behind a later prefetch): the descriptor of the other width is empty
    const int lane = threadIdx.x & 63;
    const int64_t left = n0 < a.N ? std::min<int64_t>(a.N - n0, RB) : 0;
    const bool f32 = a.bias_dtype == GPTQ_F32;
    const uint32_t n32 = a.bias && f32 ? static_cast<uint32_t>(left * 4) : 0u;
    const uint32_t n16 = a.bias && !f32 ? static_cast<uint32_t>(left * 2) : 0u;
    const char* bb = static_cast<const char*>(a.bias);
    const uint32_t ln = static_cast<uint32_t>(lane < RB ? lane : RB);
    b.b32 = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(bb + n0 * 4, n32), ln * 4, 0, 0);
    b.b16 = __builtin_amdgcn_raw_buffer_load_b16(make_rsrc(bb + n0 * 2, n16), ln * 2, 0, 0);
  }
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const int64_t n = n0 + r;
    const bool ok = n < a.N;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.packed + n * a.pitch, ok ? static_cast<uint32_t>(a.pitch) : 0u);
    const uint32_t gb = ok ? static_cast<uint32_t>(a.ngroups * 2) : 0u;
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(sc + n * a.ngroups, gb);
    const __amdgpu_buffer_rsrc_t zrs = make_rsrc(zr + n * a.ngroups, gb);
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      if constexpr (BITS % 4 == 0) {
#pragma unroll
        for (int v = 0; v < BITS / 4; ++v) {
          const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(wr, coff[i] + 16 * v, 0, 2);
          b.dw[r][i][4 * v] = t[0]; b.dw[r][i][4 * v + 1] = t[1];
          b.dw[r][i][4 * v + 2] = t[2]; b.dw[r][i][4 * v + 3] = t[3];
        }
      } else if constexpr (BITS == 2) {
        const u32x2 t = __builtin_amdgcn_raw_buffer_load_b64(wr, coff[i], 0, 2);
        b.dw[r][i][0] = t[0]; b.dw[r][i][1] = t[1];
      } else {
        typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
        const u32x3 t = __builtin_amdgcn_raw_buffer_load_b96(wr, coff[i], 0, 2);
        b.dw[r][i][0] = t[0]; b.dw[r][i][1] = t[1]; b.dw[r][i][2] = t[2];
      }
      b.s[r][i] = __builtin_amdgcn_raw_buffer_load_b16(srs, goff[i], 0, 0);
      b.z[r][i] = __builtin_amdgcn_raw_buffer_load_b16(zrs, goff[i], 0, 0);
    }
  }
}

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// sum over the 64 lanes, returned wave-uniform: butterflies inside each row
// of 16 lanes (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror),
// then the four row totals read from lanes 0, 16, 32, 48
__device__ __forceinline__ float wave_total(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x141>(v);
  v += dpp_mov<0x140>(v);
  const int b = __builtin_bit_cast(int, v);
  return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))) +
         (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48)));
}

// a 16-bit scale or zero: bf16 when SZBF, else fp16
template <bool SZBF>
__device__ __forceinline__ float sz_val(uint16_t b) {
  return SZBF ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

template <int BITS, bool BF16, bool SZBF, int MAXC, int RB>
__device__ __forceinline__ void m1_rows(const M1Batch<BITS, MAXC, RB>& b, const uint32_t (&xr)[MAXC][16],
                                        const float (&xsr)[MAXC], const float (&ysr)[MAXC], uint32_t magic,
                                        bool bias_bf, float (&acc)[RB], float& bias) {
  bias = __uint_as_float(b.b32) + (bias_bf ? bf16_bits_to_f32(b.b16) : f16_bits_to_f32(b.b16));
  using F = M1Fmt<BITS, BF16>;
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    float sacc = 0.0f;
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      float cacc[F::NCLS];
      m1_dot<BITS, BF16>(b.dw[r][i], xr[i], magic, cacc, std::make_integer_sequence<int, 16>{});
      float t = cacc[0];
#pragma unroll
      for (int c = 1; c < F::NCLS; ++c) t += cacc[c] * (1.0f / F::mult(c));
      t -= ysr[i];
      t -= sz_val<SZBF>(b.z[r][i]) * xsr[i];
      sacc += sz_val<SZBF>(b.s[r][i]) * t;
    }
    acc[r] = sacc;
  }
  // reductions after all rows, so that the rows' DPP chains interleave
#pragma unroll
  for (int r = 0; r < RB; ++r) acc[r] = wave_total(acc[r]);
}

// M = 1 (16-bit scales/zeros).  Each lane holds the x pairs of its 32-code
// chunks in registers and streams RB weight rows at a time.  WS = 1: every
// wave walks its own rows, lane l taking chunks l, l + 64, ...; WS = 4 (long
// rows): the four waves of a workgroup share each row, thread t taking chunks
// t, t + 256, ..., and the row totals meet in LDS.  Lanes past the last chunk
// hold zero x and read zeros.  Batches are double-buffered: the next batch's
// loads are issued before the current one is reduced.
template <int BITS, bool BF16, bool SZBF, int MAXC, int RB, int WS>
__global__ __launch_bounds__(256) void gemv_m1_k(LinArgs a) {
  __shared__ float red[2][4][RB];
  const int nch = static_cast<int>(a.K / 32);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int me = WS == 4 ? tid : lane;
  constexpr int kStride = 64 * WS;
  const int64_t nbatches = cdiv(a.N, RB);
  const int64_t step = WS == 4 ? gridDim.x : static_cast<int64_t>(gridDim.x) * 4;
  int64_t rb = WS == 4 ? blockIdx.x : blockIdx.x * 4LL + wave;
  if (rb >= nbatches) return;
  const int cpg = a.gs / 32;  // chunks per group

  uint32_t coff[MAXC], goff[MAXC];
  int cidx[MAXC];
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = me + kStride * i;
    const bool ok = c < nch;
    cidx[i] = ok ? c : nch - 1;
    coff[i] = ok ? static_cast<uint32_t>(c) * (4 * BITS) : static_cast<uint32_t>(a.pitch);      // out of range -> 0
    goff[i] = ok ? static_cast<uint32_t>(c / cpg) * 2 : static_cast<uint32_t>(a.ngroups * 2);  // out of range -> 0
  }
  u32x4 xraw[MAXC][4];
#pragma unroll
  for (int i = 0; i < MAXC; ++i) load_x_raw(a.x, cidx[i], xraw[i]);
  M1Batch<BITS, MAXC, RB> A, B;
  load_m1_batch<BITS, MAXC, RB>(a, rb * RB, coff, goff, A);

  uint32_t xr[MAXC][16];
  float xsr[MAXC], ysr[MAXC];
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    prep_x_chunk<BITS, BF16>(xraw[i], xr[i], xsr[i], ysr[i]);
    if (me + kStride * i >= nch) {
#pragma unroll
      for (int p = 0; p < 16; ++p) xr[i][p] = 0u;
      xsr[i] = ysr[i] = 0.0f;
    }
  }
  // the magic exponent lives in a vector register so that mask-and-or is one v_and_or_b32
  uint32_t magic;
  if constexpr (BF16) asm("v_mov_b32 %0, 0x43004300" : "=v"(magic));
  else asm("v_mov_b32 %0, 0x64006400" : "=v"(magic));

  int parity = 0;
  const bool bias_bf = a.bias_dtype == GPTQ_BF16;
  auto finish = [&](float (&acc)[RB], float bias, int64_t n0) {
    if constexpr (WS == 4) {
      if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RB; ++r) red[parity][wave][r] = acc[r];
      }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < RB; ++r)
        acc[r] = (red[parity][0][r] + red[parity][1][r]) + (red[parity][2][r] + red[parity][3][r]);
      parity ^= 1;
    }
    // lane r holds row r's bias: read it out while every lane is active
    float bv[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) bv[r] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, bias), r));
    if ((WS == 1 || wave == 0) && lane == 0) {
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int64_t n = n0 + r;
        if (n >= a.N) break;
        const float v = acc[r] + bv[r];
        a.y[n] = BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
      }
    }
  };
  // the next batch is prefetched only where there is one: a prefetch past
  // the last batch (empty descriptors, no memory traffic) still cost 3-10%
  // of the launch (measured on MI355X over the four config-4 shapes, 4- and
  // 3-bit, e.g. 3-bit 14336 x 4096 9.9 -> 8.9 us)
  for (;;) {
    float acc[RB], bias;
    if (rb + step < nbatches) load_m1_batch<BITS, MAXC, RB>(a, (rb + step) * RB, coff, goff, B);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the compute
    m1_rows<BITS, BF16, SZBF, MAXC, RB>(A, xr, xsr, ysr, magic, bias_bf, acc, bias);
    finish(acc, bias, rb * RB);
    rb += step;
    if (rb >= nbatches) break;
    if (rb + step < nbatches) load_m1_batch<BITS, MAXC, RB>(a, (rb + step) * RB, coff, goff, A);
    __builtin_amdgcn_sched_barrier(0);
    m1_rows<BITS, BF16, SZBF, MAXC, RB>(B, xr, xsr, ysr, magic, bias_bf, acc, bias);
    finish(acc, bias, rb * RB);
    rb += step;
    if (rb >= nbatches) break;
  }
}

// ------------------------------------------------------------ MFMA path ----
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// 8 consecutive codes (natural order) of a row at code index k (k % 8 == 0)
template <int BITS>
__device__ __forceinline__ void load8(const uint8_t* row, int64_t k, uint32_t (&c)[4]) {
  uint32_t w0 = 0, w1 = 0;
  if constexpr (BITS == 4) {
    w0 = *reinterpret_cast<const uint32_t*>(row + k / 2);
    c[0] = (w0 & 0xFu) | ((w0 & 0xF0u) << 12);
    c[1] = ((w0 >> 8) & 0xFu) | ((w0 & 0xF000u) << 4);
    c[2] = ((w0 >> 16) & 0xFu) | ((w0 >> 4) & 0xF0000u);
    c[3] = ((w0 >> 24) & 0xFu) | ((w0 >> 12) & 0xF0000u);
  } else if constexpr (BITS == 2) {
    w0 = *reinterpret_cast<const uint16_t*>(row + k / 4);
#pragma unroll
    for (int p = 0; p < 4; ++p) c[p] = ((w0 >> (4 * p)) & 3u) | (((w0 >> (4 * p + 2)) & 3u) << 16);
  } else if constexpr (BITS == 8) {
    const u32x2 v = *reinterpret_cast<const u32x2*>(row + k);
    w0 = v[0];
    w1 = v[1];
    c[0] = (w0 & 0xFFu) | ((w0 & 0xFF00u) << 8);
    c[1] = ((w0 >> 16) & 0xFFu) | ((w0 >> 8) & 0xFF0000u);
    c[2] = (w1 & 0xFFu) | ((w1 & 0xFF00u) << 8);
    c[3] = ((w1 >> 16) & 0xFFu) | ((w1 >> 8) & 0xFF0000u);
  } else {
    const uint8_t* p = row + (k * 3) / 8;
    const uint32_t v = p[0] | (static_cast<uint32_t>(p[1]) << 8) | (static_cast<uint32_t>(p[2]) << 16);
#pragma unroll
    for (int q = 0; q < 4; ++q) c[q] = ((v >> (6 * q)) & 7u) | (((v >> (6 * q + 3)) & 7u) << 16);
  }
}

constexpr int kMT = 8;  // activation tiles of 16 rows per pass (M <= 128)

template <int BITS, bool BF16>
__global__ __launch_bounds__(256) void dq_mfma_k(LinArgs a) {
  __shared__ float red[4][kMT * 16][17];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;
  const int64_t m_base = static_cast<int64_t>(blockIdx.y) * kMT * 16;
  const int mtiles = static_cast<int>(std::min<int64_t>(kMT, cdiv(a.M - m_base, 16)));
  const int64_t ksteps = a.K / 32;
  const int64_t per = cdiv(ksteps, 4);
  const int64_t ks0 = wave * per, ks1 = std::min<int64_t>(ksteps, ks0 + per);

  const int64_t nrow = std::min<int64_t>(n0 + (lane & 15), a.N - 1);
  const uint8_t* wrow = a.packed + nrow * a.pitch;
  const int koff = 8 * (lane >> 4);

  f32x4 tot[kMT], acc[kMT];
  float xs_acc[kMT];
#pragma unroll
  for (int t = 0; t < kMT; ++t) {
    tot[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    xs_acc[t] = 0.0f;
  }
  const float magic_fix = Magic<BITS, BF16>::kOffset;
  int64_t g_cur = ks0 < ks1 ? static_cast<int>(ks0 * 32) / a.gs : 0;

  auto fold = [&](int64_t g) {
    float s[4], z[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t n = std::min<int64_t>(n0 + 4 * (lane >> 4) + v, a.N - 1);
      s[v] = load_elem(a.scales, n * a.ngroups + g, a.sz_dtype);
      z[v] = load_elem(a.zeros, n * a.ngroups + g, a.sz_dtype) + magic_fix;
    }
#pragma unroll
    for (int t = 0; t < kMT; ++t) {
      if (t < mtiles) {
#pragma unroll
        for (int v = 0; v < 4; ++v) tot[t][v] += s[v] * (acc[t][v] - z[v] * xs_acc[t]);
      }
      acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
      xs_acc[t] = 0.0f;
    }
  };

  for (int64_t ks = ks0; ks < ks1; ++ks) {
    const int64_t k0 = ks * 32;
    const int64_t g = static_cast<int>(k0) / a.gs;
    if (g != g_cur) {
      fold(g_cur);
      g_cur = g;
    }
    uint32_t c[4];
    load8<BITS>(wrow, k0 + koff, c);
    u32x4 af;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      if constexpr (!BF16) {
        f16x2 h = __builtin_bit_cast(f16x2, c[p] | 0x64006400u) - f16x2{1024.0f16, 1024.0f16};
        af[p] = __builtin_bit_cast(uint32_t, h);
      } else {
        af[p] = Magic<BITS, BF16>::kBF16Offset ? (c[p] | 0x43004300u) : bf16_pair_exact(c[p]);
      }
    }
#pragma unroll
    for (int t = 0; t < kMT; ++t) {
      if (t < mtiles) {
        const int64_t m = m_base + t * 16 + (lane & 15);
        u32x4 bf = {0u, 0u, 0u, 0u};
        if (m < a.M) bf = *reinterpret_cast<const u32x4*>(a.x + m * a.K + k0 + koff);
        float xs = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xs += BF16 ? bf16_bits_to_f32(bf[e] & 0xffffu) : f16_bits_to_f32(bf[e] & 0xffffu);
          xs += BF16 ? bf16_bits_to_f32(bf[e] >> 16) : f16_bits_to_f32(bf[e] >> 16);
        }
        xs += __shfl_xor(xs, 16, 64);
        xs += __shfl_xor(xs, 32, 64);
        xs_acc[t] += xs;
        if constexpr (BF16)
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af), __builtin_bit_cast(bf16x8, bf),
                                                           acc[t], 0, 0, 0);
        else
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, af), __builtin_bit_cast(f16x8, bf),
                                                          acc[t], 0, 0, 0);
      }
    }
  }
  if (ks0 < ks1) fold(g_cur);

  // D layout: lane l, register v -> weight row 4*(l/16) + v, activation row l%16
#pragma unroll
  for (int t = 0; t < kMT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[wave][t * 16 + (lane & 15)][4 * (lane >> 4) + v] = tot[t][v];
  __syncthreads();
  for (int i = tid; i < mtiles * 16 * 16; i += 256) {
    const int ml = i / 16, nl = i % 16;
    const int64_t m = m_base + ml, n = n0 + nl;
    if (m >= a.M || n >= a.N) continue;
    float v = red[0][ml][nl] + red[1][ml][nl] + red[2][ml][nl] + red[3][ml][nl];
    if (a.bias) v += load_elem(a.bias, n, a.bias_dtype);
    store_elem(a.y, m * a.N + n, a.y_dtype, v);
  }
}

// --------------------------------------------- dequant GEMM (M > 4) ----
// Y (M x N) = X (M x K) W^T with W = s (q - z) dequantised on the fly into
// the activation type, as the reference dequantises its packed weights to the
// layer dtype before multiplying (one rounding of the exact product (q - z) s).
// One workgroup computes NT weight rows x MT activation rows; its WAVES waves
// split K into 128-column blocks taken round-robin (block b by wave b % WAVES),
// so each wave's serial chain is K / (128 WAVES) blocks long, and the waves'
// partial tiles are summed through LDS at the end (fixed order).  Per block a
// lane loads 32-code chunks (16 bytes at 4 bits) and their group's scale and
// zero, dequantises them into the wave's own LDS tile, and the wave
// multiplies 16 x 16 x 32 MFMA fragments: W from that tile, X straight from
// memory.  The next block's codes and X are in flight while the current
// block is multiplied.
template <int NT, int MT, int WAVES>
struct DsCfg {
  static constexpr int BN = NT / 16, BM = MT / 16;  // 16-row blocks of W and X
  static constexpr int CPL = NT / 16;               // 32-code chunks per lane and block
  static constexpr int P = 128 + 8;                 // LDS tile row pitch (halves)
  static constexpr size_t kTile = static_cast<size_t>(16) * P * 2;  // one 16-row block at a time
  static constexpr size_t kLds = WAVES * kTile + static_cast<size_t>(NT) * MT * 4;
};

// dequantised pair (exact (q - z), one rounding of the product by s), fp32 arithmetic
template <bool BF16>
__device__ __forceinline__ uint32_t dq_pair(uint32_t c, float s, float z) {
  const float lo = (static_cast<float>(c & 0xFFFFu) - z) * s;
  const float hi = (static_cast<float>(c >> 16) - z) * s;
  if constexpr (BF16) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
  } else {
    return __builtin_bit_cast(uint32_t, f16x2{static_cast<_Float16>(lo), static_cast<_Float16>(hi)});
  }
}

// the same for fp16 with an integer zero in [0, 1023]: packed fp16, where
// (1024 + q) - (1024 + z) is exact
__device__ __forceinline__ uint32_t dq_pair16(uint32_t c, uint32_t zz, uint32_t sh) {
  const f16x2 h = __builtin_bit_cast(f16x2, c | 0x64006400u) - __builtin_bit_cast(f16x2, zz);
  return __builtin_bit_cast(uint32_t, h * __builtin_bit_cast(f16x2, sh));
}

template <int BITS, bool BF16, int... PP>
__device__ __forceinline__ void dq_chunk(const uint32_t (&cw)[BITS], float s, float z, uint32_t (&d)[16],
                                         std::integer_sequence<int, PP...>) {
  if constexpr (!BF16) {
    // GPTQ zero points are integers: the packed path, chosen for the whole wave
    if (__all(z == rintf(z) && z >= 0.0f && z <= 1023.0f)) {
      const uint32_t zz = __builtin_bit_cast(uint32_t, f16x2{static_cast<_Float16>(1024.0f + z),
                                                              static_cast<_Float16>(1024.0f + z)});
      const uint32_t sh = __builtin_bit_cast(uint32_t, f16x2{static_cast<_Float16>(s), static_cast<_Float16>(s)});
      ((d[PP] = dq_pair16(chunk_pair<BITS, PP>(cw), zz, sh)), ...);
      return;
    }
  }
  ((d[PP] = dq_pair<BF16>(chunk_pair<BITS, PP>(cw), s, z)), ...);
}

// one 128-column block of a wave: codes, scales and zeros of its rows, and
// (for a single 16-row X block) its X fragments; with more X blocks the
// fragments are loaded one 32-column step ahead inside the block instead
template <int BITS, int NT, int MT>
struct DsBlock {
  static constexpr int XB = MT == 16 ? 4 : 1;
  uint32_t cw[NT / 16][BITS];
  uint32_t sw[NT / 16], zw[NT / 16];  // words holding the scales and zeros (converted when used)
  bool sh[NT / 16], zh[NT / 16];
  uint4 x[XB][MT / 16];
};

template <int BITS, bool BF16, int NT, int MT, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void dq_split_k(LinArgs a) {
  using C = DsCfg<NT, MT, WAVES>;
  constexpr int BN = C::BN, BM = C::BM, P = C::P;
  extern __shared__ __attribute__((aligned(16))) uint16_t dsm[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  uint16_t* tile = dsm + wave * (16 * P);
  float* red = reinterpret_cast<float*>(dsm + WAVES * 16 * P);
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * NT;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * MT;
  const int nblk = static_cast<int>(a.K / 128);
  const int r16 = lane & 15, oct = lane >> 4;

  const uint8_t* wrow[BN];
  int64_t wn[BN];
#pragma unroll
  for (int i = 0; i < BN; ++i) {
    wn[i] = std::min<int64_t>(n0 + 16 * i + r16, a.N - 1);
    wrow[i] = a.packed + wn[i] * a.pitch;
  }
  // X row of B-fragment block j (rows past M read as zeros)
  const uint16_t* xrow[BM];
  bool xok[BM];
#pragma unroll
  for (int j = 0; j < BM; ++j) {
    const int64_t m = m0 + 16 * j + r16;
    xok[j] = m < a.M;
    xrow[j] = a.x + (xok[j] ? m : 0) * a.K;
  }

  auto loadx = [&](int b, int kk, int j) {
    return xok[j] ? *reinterpret_cast<const uint4*>(xrow[j] + static_cast<int64_t>(b) * 128 + 32 * kk + 8 * oct)
                  : uint4{0u, 0u, 0u, 0u};
  };
  // lane (r16, oct): chunk oct (codes 32 oct .. + 31 of the block) of rows 16 i + r16
  auto load = [&](int b, DsBlock<BITS, NT, MT>& L) {
    const int64_t k = static_cast<int64_t>(b) * 128 + 32 * oct;
    const int64_t g = static_cast<int>(k) / a.gs;  // 32-bit division (K < 2^31)
#pragma unroll
    for (int i = 0; i < BN; ++i) {
      const uint32_t* src = reinterpret_cast<const uint32_t*>(wrow[i] + k * BITS / 8);
      if constexpr (BITS == 4) {
        const uint4 v = *reinterpret_cast<const uint4*>(src);
        L.cw[i][0] = v.x; L.cw[i][1] = v.y; L.cw[i][2] = v.z; L.cw[i][3] = v.w;
      } else if constexpr (BITS == 8) {
        const uint4 v0 = reinterpret_cast<const uint4*>(src)[0], v1 = reinterpret_cast<const uint4*>(src)[1];
        L.cw[i][0] = v0.x; L.cw[i][1] = v0.y; L.cw[i][2] = v0.z; L.cw[i][3] = v0.w;
        L.cw[i][4] = v1.x; L.cw[i][5] = v1.y; L.cw[i][6] = v1.z; L.cw[i][7] = v1.w;
      } else if constexpr (BITS == 2) {
        const uint2 v = *reinterpret_cast<const uint2*>(src);
        L.cw[i][0] = v.x; L.cw[i][1] = v.y;
      } else {
        L.cw[i][0] = src[0]; L.cw[i][1] = src[1]; L.cw[i][2] = src[2];
      }
      L.sw[i] = elem_word(a.scales, wn[i] * a.ngroups + g, a.sz_dtype, L.sh[i]);
      L.zw[i] = elem_word(a.zeros, wn[i] * a.ngroups + g, a.sz_dtype, L.zh[i]);
    }
    // B fragments: lane (r16, oct) holds X row 16 j + r16, columns 32 kk + 8 oct .. + 7
    if constexpr (BM == 1) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) L.x[kk][0] = loadx(b, kk, 0);
    }
  };

  f32x4 acc[BN][BM];
#pragma unroll
  for (int i = 0; i < BN; ++i)
#pragma unroll
    for (int j = 0; j < BM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto block = [&](int b, const DsBlock<BITS, NT, MT>& L) {
    // row blocks one at a time through the wave's 16-row tile: dequantise this
    // lane's chunk (row r16, columns 32 oct ..), then 4 MFMA steps against X
#pragma unroll
    for (int i = 0; i < BN; ++i) {
      uint32_t d[16];
      dq_chunk<BITS, BF16>(L.cw[i], elem_value(L.sw[i], L.sh[i], a.sz_dtype), elem_value(L.zw[i], L.zh[i], a.sz_dtype),
                           d, std::make_integer_sequence<int, 16>{});
      uint4* dst = reinterpret_cast<uint4*>(tile + r16 * P + 32 * oct);
#pragma unroll
      for (int q = 0; q < 4; ++q) dst[q] = uint4{d[4 * q], d[4 * q + 1], d[4 * q + 2], d[4 * q + 3]};
      wave_sync();
      uint4 xs[2][BM];
      if constexpr (BM > 1) {
#pragma unroll
        for (int j = 0; j < BM; ++j) xs[0][j] = loadx(b, 0, j);
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        if constexpr (BM > 1) {
          if (kk + 1 < 4) {
#pragma unroll
            for (int j = 0; j < BM; ++j) xs[(kk + 1) & 1][j] = loadx(b, kk + 1, j);
          }
        }
        const uint4 fa = *reinterpret_cast<const uint4*>(tile + r16 * P + 32 * kk + 8 * oct);
#pragma unroll
        for (int j = 0; j < BM; ++j) {
          const uint4 fb = BM == 1 ? L.x[kk & (DsBlock<BITS, NT, MT>::XB - 1)][0] : xs[kk & 1][j];
          if constexpr (BF16)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, fa),
                                                                __builtin_bit_cast(bf16x8, fb), acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, fa),
                                                               __builtin_bit_cast(f16x8, fb), acc[i][j], 0, 0, 0);
        }
      }
      wave_sync();  // the tile is rewritten next
    }
  };

  // blocks b = wave, wave + WAVES, ...: two in flight
  DsBlock<BITS, NT, MT> A, B;
  int b = wave;
  if (b < nblk) load(b, A);
  for (;;) {
    if (b >= nblk) break;
    if (b + WAVES < nblk) load(b + WAVES, B);
    block(b, A);
    b += WAVES;
    if (b >= nblk) break;
    if (b + WAVES < nblk) load(b + WAVES, A);
    block(b, B);
    b += WAVES;
  }

  // sum the waves' tiles in wave order; 16x16 layout: lane l, register v ->
  // W row 4 (l / 16) + v, X row l % 16
  for (int w = 0; w < WAVES; ++w) {
    if (wave == w) {
#pragma unroll
      for (int i = 0; i < BN; ++i)
#pragma unroll
        for (int j = 0; j < BM; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            float& r = red[(16 * j + r16) * NT + 16 * i + 4 * oct + v];
            r = (w == 0 ? 0.0f : r) + acc[i][j][v];
          }
    }
    __syncthreads();
  }
  for (int e = tid; e < NT * MT; e += 64 * WAVES) {
    const int ml = e / NT, nl = e % NT;
    const int64_t m = m0 + ml, n = n0 + nl;
    if (m < a.M && n < a.N) {
      float v = red[e];
      if (a.bias) v += load_elem(a.bias, n, a.bias_dtype);
      store_elem(a.y, m * a.N + n, a.y_dtype, v);
    }
  }
}

// M <= 16, 4- or 3-bit codes (fp16 or bf16 activations): the dequantised codes go straight
// from registers into the MFMA, with no LDS tile.  Lane (r, g) of a wave loads
// codes 32 g .. 32 g + 31 of the 128-column block for weight row r (one
// 16-byte load); at MFMA step kk it supplies the 8 codes of word kk, so step
// kk covers columns {32 g + 8 kk + t} over the four lane groups g -- a fixed
// bijection of the block's columns onto (step, lane group, element), which
// the X fragments follow (lane (m, g) at step kk holds X row m at the same 8
// columns).  Within a word the codes are decoded as pairs (t, t + 4) (a
// shift and mask per pair), so both operands carry their 8
// elements in the order 0 4 1 5 2 6 3 7 (X is permuted with v_perm).  The
// dequantised value is (q - z) (exact) times s, rounded once, as in the LDS
// path.  The waves of a workgroup split the blocks and sum their partial
// tiles in wave order.
template <int NT, int BITS>
struct DrBlock {
  uint32_t cw[NT / 16][BITS];  // a lane's 32 codes of each row block
  uint4 x[4];
};

// the code pairs (8 kk + t, 8 kk + t + 4), t = 0..3, of MFMA step kk from a
// lane's 32 codes (4-bit: word kk; 3-bit: the 24 bits at 24 kk of 3 words)
template <int BITS>
__device__ __forceinline__ void step_pairs(const uint32_t (&cw)[BITS], int kk, uint32_t (&p)[4]) {
  if constexpr (BITS == 4) {
#pragma unroll
    for (int t = 0; t < 4; ++t) p[t] = (cw[kk] >> (4 * t)) & 0x000F000Fu;
  } else {
    const uint32_t v = kk == 0 ? cw[0]
                     : kk == 1 ? __builtin_amdgcn_alignbit(cw[1], cw[0], 24)
                     : kk == 2 ? __builtin_amdgcn_alignbit(cw[2], cw[1], 16)
                               : cw[2] >> 8;
#pragma unroll
    for (int t = 0; t < 4; ++t) p[t] = ((v >> (3 * t)) & 7u) | (((v >> (3 * t + 12)) & 7u) << 16);
  }
}

// step_pairs without the final mask: word v >> 3t (3-bit) or >> 4t (4-bit),
// whose low fields at bits 0 and 16 are the pair; the caller masks
template <int BITS>
__device__ __forceinline__ void step_fields(const uint32_t (&cw)[BITS], int kk, uint32_t (&p)[4]) {
  if constexpr (BITS == 4) {
#pragma unroll
    for (int t = 0; t < 4; ++t) p[t] = cw[kk] >> (4 * t);
  } else {
    const uint32_t v = kk == 0 ? cw[0]
                     : kk == 1 ? __builtin_amdgcn_alignbit(cw[1], cw[0], 24)
                     : kk == 2 ? __builtin_amdgcn_alignbit(cw[2], cw[1], 16)
                               : cw[2] >> 8;
    // bits 3t..3t+2 -> 0..2 and 3t+12..3t+14 -> 16..18: the upper field moves
    // 4 bits further than the lower one
#pragma unroll
    for (int t = 0; t < 4; ++t) p[t] = ((v >> (3 * t)) & 0x7u) | (((v >> (3 * t + 12)) & 0x7u) << 16);
  }
}

__device__ __forceinline__ uint4 perm_0415(uint4 v) {
  return uint4{__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
               __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u)};
}

// the code pairs of a step -> 4 dwords of dequantised (code t, code t + 4)
template <bool kPacked, bool BF16 = false>
__device__ __forceinline__ uint4 dq_word_0415(uint32_t (&p)[4], uint32_t zz, uint32_t sh, float s, float z) {
  if constexpr (kPacked) {
#pragma unroll
    for (int t = 0; t < 4; ++t) p[t] = dq_pair16(p[t], zz, sh);
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t) p[t] = dq_pair<BF16>(p[t], s, z);
  }
  return uint4{p[0], p[1], p[2], p[3]};
}

// The workgroup's scales and zeros (contiguous rows of the [N][ngroups]
// arrays) staged once in LDS: per block a lane then reads its pairs from LDS
// instead of 16-row gathers.  Element e = r ng + g of the rows' chunk goes to
// sz[g][r].  Where both chunks are 16-byte aligned a lane loads 16 bytes of
// each per round (8 halves or 4 floats; rows past N read as zeros through the
// buffer descriptors) and steps (r, g) along them: one round for up to 4096
// halves per array, where one element pair per lane and round made the
// staging a chain of memory round trips.  kPer threads take part.
template <int NT>
__device__ __forceinline__ void stage_sz(const LinArgs& a, int64_t n0, float2* sz, int tid, int lane, int kPer) {
  const int ng = static_cast<int>(a.ngroups);
  const int tot = NT * ng;
  const int esz = a.sz_dtype == GPTQ_F32 ? 4 : 2;
  const char* sb = static_cast<const char*>(a.scales) + n0 * a.ngroups * esz;
  const char* zb = static_cast<const char*>(a.zeros) + n0 * a.ngroups * esz;
  if (((reinterpret_cast<uintptr_t>(sb) | reinterpret_cast<uintptr_t>(zb)) & 15u) == 0) {
    const uint32_t bytes = static_cast<uint32_t>(std::min<int64_t>(NT, a.N - n0) * ng * esz);
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(sb, bytes), zrs = make_rsrc(zb, bytes);
    const int epv = 16 / esz;
    const int nvec = static_cast<int>(cdiv(tot, epv));
    for (int v = tid; v - lane < nvec; v += kPer) {
      const uint32_t off = 16u * static_cast<uint32_t>(v);
      const u32x4 sv = __builtin_amdgcn_raw_buffer_load_b128(srs, off, 0, 0);
      const u32x4 zv = __builtin_amdgcn_raw_buffer_load_b128(zrs, off, 0, 0);
      const int e0 = v * epv;
      if (e0 >= tot) continue;
      int r = e0 / ng, g = e0 - r * ng;
      auto put = [&](float sv_, float zv_) {
        if (r < NT) sz[g * NT + r] = float2{sv_, zv_};
        if (++g == ng) { g = 0; ++r; }
      };
      if (esz == 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) put(__builtin_bit_cast(float, sv[j]), __builtin_bit_cast(float, zv[j]));
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          put(elem_value((sv[j / 2] >> (16 * (j & 1))) & 0xFFFFu, false, a.sz_dtype),
              elem_value((zv[j / 2] >> (16 * (j & 1))) & 0xFFFFu, false, a.sz_dtype));
      }
    }
  } else {
    for (int e = tid; e < tot; e += kPer) {
      const int64_t off = std::min<int64_t>(n0 + e / ng, a.N - 1) * a.ngroups + e % ng;
      sz[(e % ng) * NT + e / ng] =
          float2{load_elem(a.scales, off, a.sz_dtype), load_elem(a.zeros, off, a.sz_dtype)};
    }
  }
}

// kFold (group size a multiple of 128, so a block is one group): the codes
// enter the MFMA as small integers (fp16: q, from 1024 + q less 1024; bf16:
// 128 + q straight from the OR, exact in bf16), products are exact in fp32,
// and each block's 16 x 16 result is corrected per weight row as
// s (sum q' x - z' sum x) with z' = z (fp16) or z + 128 (bf16), sum x from
// one more MFMA chain against an all-ones operand.  This is the per-group
// zero folding of the reference's fused kernels; it skips the per-weight
// subtract, multiply and rounding of the dequantised weight.
template <int BITS, int NT, int WAVES, bool kFold, bool BF16>
__global__ __launch_bounds__(64 * WAVES) void dq_reg4_k(LinArgs a) {
  constexpr int BN = NT / 16;
  __shared__ float red[WAVES][BN][4][64];
  extern __shared__ __attribute__((aligned(16))) float2 sz[];  // [ngroups][NT]: (scale, zero) of the workgroup's rows
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * NT;
  // split-K over grid.y: this workgroup's 128-column blocks kb0 .. kb0 + nblk - 1
  const int ktot = static_cast<int>(a.K / 128);
  const int bps = static_cast<int>(cdiv(ktot, gridDim.y));
  const int kb0 = static_cast<int>(blockIdx.y) * bps;
  const int nblk = std::min(ktot - kb0, bps);
  const int r16 = lane & 15, g4 = lane >> 4;

  const uint8_t* wrow[BN];
  int64_t wn[BN];
#pragma unroll
  for (int i = 0; i < BN; ++i) {
    wn[i] = std::min<int64_t>(n0 + 16 * i + r16, a.N - 1);
    wrow[i] = a.packed + wn[i] * a.pitch;
  }
  const bool xok = r16 < a.M;
  const uint16_t* xrow = a.x + (xok ? r16 : 0) * a.K;

  auto load = [&](int b, DrBlock<NT, BITS>& L) {
    const int64_t k = static_cast<int64_t>(kb0 + b) * 128 + 32 * g4;
#pragma unroll
    for (int i = 0; i < BN; ++i) {
      const uint32_t* src = reinterpret_cast<const uint32_t*>(wrow[i] + k * BITS / 8);
      if constexpr (BITS == 4) {
        const uint4 v = *reinterpret_cast<const uint4*>(src);
        L.cw[i][0] = v.x; L.cw[i][1] = v.y; L.cw[i][2] = v.z; L.cw[i][3] = v.w;
      } else {
        L.cw[i][0] = src[0]; L.cw[i][1] = src[1]; L.cw[i][2] = src[2];
      }
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) L.x[kk] = *reinterpret_cast<const uint4*>(xrow + k + 8 * kk);
  };

  f32x4 acc[BN];
#pragma unroll
  for (int i = 0; i < BN; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto block = [&](int b, const DrBlock<NT, BITS>& L) {
    uint4 xb[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) xb[kk] = xok ? perm_0415(L.x[kk]) : uint4{0u, 0u, 0u, 0u};
    // the lane's group: with groups of >= 128 columns the block's (one
    // wave-uniform division), else per lane (32-bit division, K < 2^31)
    const int g = kFold ? __builtin_amdgcn_readfirstlane((kb0 + b) * 128 / a.gs) : ((kb0 + b) * 128 + 32 * g4) / a.gs;
    const float2* szg = sz + g * NT;
    auto mfma = [](uint4 fa, uint4 fb, f32x4 c) {
      if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, fa), __builtin_bit_cast(bf16x8, fb),
                                                       c, 0, 0, 0);
      else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, fa), __builtin_bit_cast(f16x8, fb), c,
                                                      0, 0, 0);
    };
    if constexpr (kFold) {
      f32x4 sx = f32x4{0.f, 0.f, 0.f, 0.f};
      constexpr uint32_t kOne = BF16 ? 0x3f803f80u : 0x3c003c00u;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) sx = mfma(uint4{kOne, kOne, kOne, kOne}, xb[kk], sx);
      // the codes enter as 128 + q (bf16) or 1024 + q (fp16), both exact,
      // straight from an AND-OR (the masks in registers let the compiler fuse
      // the two), and the offset joins the zero in the correction
      uint32_t mask = 0x000F000Fu, magic = BF16 ? 0x43004300u : 0x64006400u;
      if constexpr (BITS == 3) mask = 0x00070007u;
      asm volatile("" : "+v"(mask), "+v"(magic));
      constexpr float kZoff = BF16 ? 128.0f : 1024.0f;
#pragma unroll
      for (int i = 0; i < BN; ++i) {
        f32x4 t = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          uint32_t q[4];
          step_fields<BITS>(L.cw[i], kk, q);
#pragma unroll
          for (int u = 0; u < 4; ++u) q[u] = (q[u] & mask) | magic;
          t = mfma(uint4{q[0], q[1], q[2], q[3]}, xb[kk], t);
        }
        const float4 p01 = *reinterpret_cast<const float4*>(szg + 16 * i + 4 * g4);
        const float4 p23 = *reinterpret_cast<const float4*>(szg + 16 * i + 4 * g4 + 2);
        const float ps[4] = {p01.x, p01.z, p23.x, p23.z}, pz[4] = {p01.y, p01.w, p23.y, p23.w};
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[i][v] = fmaf(ps[v], fmaf(-(pz[v] + kZoff), sx[v], t[v]), acc[i][v]);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < BN; ++i) {
      const float2 p = szg[16 * i + r16];
      const float s = p.x, z = p.y;
      uint4 fa[4];
      uint32_t pr[4][4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) step_pairs<BITS>(L.cw[i], kk, pr[kk]);
      // GPTQ zero points are integers: the packed path (fp16 activations and
      // fp16 scales, so that s is exact in fp16 and (q - z) * s rounds once),
      // chosen for the whole wave
      if (!BF16 && a.sz_dtype == GPTQ_F16 && __all(z == rintf(z) && z >= 0.0f && z <= 1023.0f)) {
        const uint32_t zz = __builtin_bit_cast(uint32_t, f16x2{static_cast<_Float16>(1024.0f + z),
                                                                static_cast<_Float16>(1024.0f + z)});
        const uint32_t sh = __builtin_bit_cast(uint32_t, f16x2{static_cast<_Float16>(s), static_cast<_Float16>(s)});
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) fa[kk] = dq_word_0415<true>(pr[kk], zz, sh, s, z);
      } else {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) fa[kk] = dq_word_0415<false, BF16>(pr[kk], 0u, 0u, s, z);
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) acc[i] = mfma(fa[kk], xb[kk], acc[i]);
    }
  };

  // blocks b = wave, wave + WAVES, ...: two in flight; the first two are
  // issued before the scales and zeros are staged
  DrBlock<NT, BITS> A, B;
  int b = wave;
  if (b < nblk) load(b, A);
  if (b + WAVES < nblk) load(b + WAVES, B);

  stage_sz<NT>(a, n0, sz, tid, lane, 64 * WAVES);
  __syncthreads();

  for (bool first = true;; first = false) {
    if (b >= nblk) break;
    if (!first && b + WAVES < nblk) load(b + WAVES, B);
    block(b, A);
    b += WAVES;
    if (b >= nblk) break;
    if (b + WAVES < nblk) load(b + WAVES, A);
    block(b, B);
    b += WAVES;
  }

  // partial tiles summed in wave order (then, split over grid.y, written as
  // fp32 partial sums for splitk_reduce_k); 16x16 layout: lane l, register
  // v -> W row 4 (l / 16) + v, X row l % 16
#pragma unroll
  for (int i = 0; i < BN; ++i)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[wave][i][v][lane] = acc[i][v];
  __syncthreads();
  for (int e = tid; e < BN * 4 * 64; e += 64 * WAVES) {
    const int i = e / 256, v = (e / 64) % 4, l = e % 64;
    float r = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) r += red[w][i][v][l];
    const int64_t m = l % 16, n = n0 + 16 * i + 4 * (l / 16) + v;
    if (m < a.M && n < a.N) {
      if (gridDim.y > 1) {
        a.part[(blockIdx.y * a.M + m) * a.N + n] = r;
      } else {
        if (a.bias) r += load_elem(a.bias, n, a.bias_dtype);
        store_elem(a.y, m * a.N + n, a.y_dtype, r);
      }
    }
  }
}

// y = bias + sum of the split-K partial sums, in split order (deterministic);
// four outputs per thread
__global__ __launch_bounds__(256) void splitk_reduce_k(const float* __restrict__ part, int S, int64_t M, int64_t N,
                                                       const void* __restrict__ bias, int bias_dtype, void* y,
                                                       int y_dtype) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t e = 4 * q;
  if (e >= M * N) return;
  const int64_t plane = M * N;
  // partials added in split order, up to eight loads in flight before their
  // adds (one load and wait per split was S - 1 round trips in a row; the
  // call measured the same in HIP graphs, where the reduce's launch and its
  // traffic dominate), the quad's four outputs in one store
  f32x4 v = *reinterpret_cast<const f32x4*>(part + e);
  int s = 1;
  for (; s + 8 <= S; s += 8) {
    f32x4 w[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) w[u] = *reinterpret_cast<const f32x4*>(part + (s + u) * plane + e);
#pragma unroll
    for (int u = 0; u < 8; ++u) v += w[u];
  }
  if (s < S) {
    f32x4 w[7];
#pragma unroll
    for (int u = 0; u < 7; ++u)
      if (s + u < S) w[u] = *reinterpret_cast<const f32x4*>(part + (s + u) * plane + e);
#pragma unroll
    for (int u = 0; u < 7; ++u)
      if (s + u < S) v += w[u];
  }
  const int64_t n = e % N;  // N % 4 == 0: the quad lies in one row
  float r[4] = {v[0], v[1], v[2], v[3]};
  if (bias) {
    float b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) b[u] = load_elem(bias, n + u, bias_dtype);
#pragma unroll
    for (int u = 0; u < 4; ++u) r[u] += b[u];
  }
  if (y_dtype != GPTQ_F32 && (reinterpret_cast<uintptr_t>(y) & 7) == 0) {
    uint32_t h[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) h[u] = y_dtype == GPTQ_BF16 ? f32_to_bf16_bits(r[u]) : f32_to_f16_bits(r[u]);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(y) + e) = uint2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
  } else {
#pragma unroll
    for (int u = 0; u < 4; ++u) store_elem(y, e + u, y_dtype, r[u]);
  }
}

// splits > 1: K split over grid.y, the fp32 partial sums in a.part (the
// caller checked that they fit), then splitk_reduce_k
template <int BITS, int NT, int WAVES, bool BF16>
int launch_reg4(hipStream_t st, const LinArgs& a, int splits = 1) {
  const size_t lds = static_cast<size_t>(NT) * a.ngroups * sizeof(float2);
  // static partial-tile buffer + the staged scales and zeros within the CU's LDS
  GPTQ_REQUIRE(static_cast<size_t>(WAVES) * NT * 16 * sizeof(float) + lds <= 160 * 1024, GPTQ_ERR_SHAPE,
               "dq_reg4: %lld groups per row exceed the LDS budget", static_cast<long long>(a.ngroups));
  const dim3 grid(static_cast<unsigned>(cdiv(a.N, NT)), static_cast<unsigned>(splits));
  if (a.gs % 128 == 0)
    hipLaunchKernelGGL((dq_reg4_k<BITS, NT, WAVES, true, BF16>), grid, dim3(64 * WAVES), lds, st, a);
  else
    hipLaunchKernelGGL((dq_reg4_k<BITS, NT, WAVES, false, BF16>), grid, dim3(64 * WAVES), lds, st, a);
  int rc = check_launch("dq_reg4");
  if (rc != GPTQ_OK || splits == 1) return rc;
  const int64_t quads = a.M * a.N / 4;
  hipLaunchKernelGGL(splitk_reduce_k, dim3(static_cast<unsigned>(cdiv(quads, 256))), dim3(256), 0, st, a.part, splits,
                     a.M, a.N, a.bias, a.bias_dtype, static_cast<void*>(a.y), a.y_dtype);
  return check_launch("splitk_reduce");
}

// M <= 16 on layers of 241-256 workgroups of 112 rows (26881-28672 rows; K <=
// 4096, groups of >= 128 columns, 4- or 3-bit codes): each wave owns 16
// weight rows over the whole of K and streams its rows' codes through a ring
// of D register slots (loads clamped to the last block, so every slot is
// refilled unconditionally and each wait covers one slot's load), decoding
// them as dq_reg4_k's kFold path does.  X
// (16 x K, rows past M as zeros) is staged once per workgroup in LDS, already
// in the lanes' order (perm_0415 per 16 bytes: slot [b][g][kk][r] holds X row
// r, columns 128 b + 32 g + 8 kk .. + 7), with the per-block sums of X from
// the same all-ones MFMA chain.  No K split and no cross-wave reduction: a
// wave's 16 x 16 tile is summed over the blocks in order and stored.  In
// dq_reg4_k the waves of a workgroup split K, so each streamed 4 of the 32
// blocks at 28672 x 4096 with two in flight, and the prologue and the
// cross-wave reduction took about half of the launch.
constexpr int kRow16MaxBlk = 32;  // K <= 4096: X takes 128 KB of LDS
__shared__ __attribute__((aligned(16))) uint4 g_row16_x[kRow16MaxBlk * 256];
__shared__ float g_row16_sx[kRow16MaxBlk][16];

template <int BITS, int W, int D, bool BF16>
__global__ __launch_bounds__(64 * W) void dq_row16_k(LinArgs a) {
  constexpr int NT = 16 * W;
  extern __shared__ __attribute__((aligned(16))) float2 sz[];  // [ngroups][NT]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * NT;
  const int nblk = static_cast<int>(a.K / 128);
  const int r16 = lane & 15, g4 = lane >> 4;
  const uint8_t* wrow = a.packed + std::min<int64_t>(n0 + 16 * wave + r16, a.N - 1) * a.pitch;

  auto mfma = [](uint4 fa, uint4 fb, f32x4 c) {
    if constexpr (BF16)
      return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, fa), __builtin_bit_cast(bf16x8, fb), c,
                                                     0, 0, 0);
    else
      return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, fa), __builtin_bit_cast(f16x8, fb), c, 0,
                                                    0, 0);
  };

  // X into LDS in the lanes' order.  All of a thread's loads are issued
  // before any is waited for (in batches of kXB), and before the code
  // prefetch, so that waiting for them leaves the code loads in flight.
  // Slots past the last block repeat the last one and rows past M are
  // zeroed after the load: every load and store is unconditional, which
  // keeps the compiler's waits exact.
  {
    constexpr int kXB = 64 * W >= 448 ? 20 : 16;  // 8192 slots / threads, per batch
    const int tot = nblk * 256;
    for (int base = tid; base < tot; base += kXB * 64 * W) {
      uint4 v[kXB];
#pragma unroll
      for (int j = 0; j < kXB; ++j) {
        const int idx = std::min(base + j * 64 * W, tot - 1);
        const int b = idx >> 8, g = (idx >> 6) & 3, kk = (idx >> 4) & 3, r = idx & 15;
        const int row = r < a.M ? r : 0;
        v[j] = *reinterpret_cast<const uint4*>(a.x + static_cast<int64_t>(row) * a.K + b * 128 + 32 * g + 8 * kk);
      }
#pragma unroll
      for (int j = 0; j < kXB; ++j) {
        const int idx = std::min(base + j * 64 * W, tot - 1);
        const uint4 pv = perm_0415(v[j]);
        const bool live = (idx & 15) < a.M;
        g_row16_x[idx] = uint4{live ? pv.x : 0u, live ? pv.y : 0u, live ? pv.z : 0u, live ? pv.w : 0u};
      }
    }
  }

  // slot loads: codes 32 g4 .. 32 g4 + 31 of block b (clamped) of the lane's row
  uint32_t cw[D][BITS];
  auto load = [&](int b, auto slot) {
    constexpr int S = decltype(slot)::value;
    b = std::min(b, nblk - 1);
    const uint32_t* src = reinterpret_cast<const uint32_t*>(wrow + static_cast<int64_t>(b * 128 + 32 * g4) * BITS / 8);
    if constexpr (BITS == 4) {
      const uint4 v = *reinterpret_cast<const uint4*>(src);
      cw[S][0] = v.x; cw[S][1] = v.y; cw[S][2] = v.z; cw[S][3] = v.w;
    } else {
      cw[S][0] = src[0]; cw[S][1] = src[1]; cw[S][2] = src[2];
    }
  };
  sfor<0, D>([&](auto sc) { load(decltype(sc)::value, sc); });

  stage_sz<NT>(a, n0, sz, tid, lane, 64 * W);
  __syncthreads();
  // the blocks' sums of X (X row l % 16 in every register of lane l)
  for (int b = wave; b < nblk; b += W) {
    constexpr uint32_t kOne = BF16 ? 0x3f803f80u : 0x3c003c00u;
    f32x4 t = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) t = mfma(uint4{kOne, kOne, kOne, kOne}, g_row16_x[((b * 4 + g4) * 4 + kk) * 16 + r16], t);
    if (g4 == 0) g_row16_sx[b][r16] = t[0];
  }
  __syncthreads();

  // a block's LDS operands (X fragments, sum of X, scales and zeros of the
  // lane's four rows), read one block ahead of their MFMAs
  struct Lds {
    uint4 x[4];
    float sx;
    float4 p01, p23;
  };
  auto fetch = [&](int b, Lds& L) {
    b = std::min(b, nblk - 1);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) L.x[kk] = g_row16_x[((b * 4 + g4) * 4 + kk) * 16 + r16];
    L.sx = g_row16_sx[b][r16];
    const float2* szg = sz + __builtin_amdgcn_readfirstlane(b * 128 / a.gs) * NT + 16 * wave;
    L.p01 = *reinterpret_cast<const float4*>(szg + 4 * g4);
    L.p23 = *reinterpret_cast<const float4*>(szg + 4 * g4 + 2);
  };

  // codes enter as 128 + q (bf16) or 1024 + q (fp16) from an AND-OR; the
  // offset joins the zero in the per-row correction s (sum q' x - z' sum x)
  uint32_t mask = BITS == 3 ? 0x00070007u : 0x000F000Fu, magic = BF16 ? 0x43004300u : 0x64006400u;
  asm volatile("" : "+v"(mask), "+v"(magic));
  constexpr float kZoff = BF16 ? 128.0f : 1024.0f;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  auto block = [&](const Lds& L, auto slot) {
    constexpr int S = decltype(slot)::value;
    f32x4 t = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      uint32_t q[4];
      step_fields<BITS>(cw[S], kk, q);
#pragma unroll
      for (int u = 0; u < 4; ++u) q[u] = (q[u] & mask) | magic;
      t = mfma(uint4{q[0], q[1], q[2], q[3]}, L.x[kk], t);
    }
    const float ps[4] = {L.p01.x, L.p01.z, L.p23.x, L.p23.z}, pz[4] = {L.p01.y, L.p01.w, L.p23.y, L.p23.w};
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[v] = fmaf(ps[v], fmaf(-(pz[v] + kZoff), L.sx, t[v]), acc[v]);
  };
  // slots of an even ring alternate the two LDS operand sets.  Trips of D
  // blocks refill each slot after use while D more blocks remain; the last
  // (up to D) blocks drain the ring with no loads, so that every trip's
  // loads are unconditional and each wait covers exactly one slot
  static_assert(D % 2 == 0, "ring of an even number of slots");
  Lds L0, L1;
  fetch(0, L0);
  auto trip = [&](int b0, auto refill) {
    sfor<0, D>([&](auto sc) {
      constexpr int S = decltype(sc)::value;
      Lds& cur = S % 2 == 0 ? L0 : L1;
      Lds& nxt = S % 2 == 0 ? L1 : L0;
      fetch(b0 + S + 1, nxt);
      // the next block's LDS reads go out before this block's decode and
      // MFMAs (left alone, the compiler sank them below the MFMAs and waited
      // for them at the top of the next block)
      __builtin_amdgcn_sched_barrier(0);
      if (b0 + S < nblk) block(cur, sc);
      if constexpr (decltype(refill)::value) load(b0 + S + D, sc);
    });
  };
  int b0 = 0;
  for (; b0 + D < nblk; b0 += D) trip(b0, std::true_type{});
  trip(b0, std::false_type{});

  // 16x16 layout: lane l, register v -> W row 4 (l / 16) + v, X row l % 16
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int64_t m = r16, n = n0 + 16 * wave + 4 * g4 + v;
    if (m < a.M && n < a.N) {
      float r = acc[v];
      if (a.bias) r += load_elem(a.bias, n, a.bias_dtype);
      store_elem(a.y, m * a.N + n, a.y_dtype, r);
    }
  }
}

// a ring of 4 slots: at 28672 x 4096, M = 16 / 2 (4-bit), 2 / 4 / 6 / 8 / 16 /
// 32 slots took 22.3 / 19.7 / 20.3 / 20.6 / 22.5 / 26.5 and 20.3 / 17.8 /
// 18.5 / 18.9 / 20.9 / 24.6 us (refilling pairs of slots together, so that
// both halves of each 128-byte line go out back to back, changed nothing)
template <int BITS, int W, bool BF16>
int launch_row16(hipStream_t st, const LinArgs& a) {
  constexpr int D = 4;
  const size_t lds = static_cast<size_t>(16 * W) * a.ngroups * sizeof(float2);
  const dim3 grid(static_cast<unsigned>(cdiv(a.N, 16 * W)));
  hipLaunchKernelGGL((dq_row16_k<BITS, W, D, BF16>), grid, dim3(64 * W), lds, st, a);
  return check_launch("dq_row16");
}

// dq_row16_k's layout: K a multiple of 128 up to 4096, one group per block,
// and X, the block sums and the workgroup's scales and zeros within the LDS
inline bool row16_fits(const LinArgs& a, int W) {
  const size_t stat = sizeof(uint4) * kRow16MaxBlk * 256 + sizeof(float) * kRow16MaxBlk * 16;
  return a.K % 128 == 0 && a.K <= 128 * kRow16MaxBlk && a.gs % 128 == 0 &&
         stat + static_cast<size_t>(16 * W) * a.ngroups * sizeof(float2) <= 160 * 1024;
}

// (K splits of the register path on 4097-8192-row layers, 1 < M <= 16, and
// on 3072-4096-row layers, 8 < M <= 16: plan::reg4_mid_splits,
// plan::reg4_wide_splits and plan::reg4_narrow_splits)

// Large products (M > 16 and enough output tiles): one workgroup per NT x MT
// tile of (weight rows x activation rows), NT = 128 (K in steps of 64) or 64
// (steps of 128) so that the grid fills the GPU.  Each thread loads one
// 32-code chunk of one weight row per step, dequantises it into a
// double-buffered LDS tile, and stages a piece of X beside it; the 4 waves
// (2 x 2) multiply 32x32x16 MFMA fragments from LDS.  The codes and X of the
// next two steps are in registers while the current step is multiplied.
template <int NT, int MT, int KB_>
struct DtCfg {
  static constexpr int KB = KB_, CPR = KB / 32;  // NT * CPR <= 256 chunks of 32 codes per step
  static constexpr int CW = NT * CPR / 64;       // waves that load and dequantise codes
  static constexpr int P = KB + 8;               // LDS row pitch (halves): conflict-free fragment reads
  static constexpr int XV = MT * KB / 8 / 256;   // 16-byte X pieces per thread and step
  static_assert(NT * CPR <= 256 && (NT * CPR) % 64 == 0, "code chunks per step");
};

template <int BITS, int XV>
struct DtStage {
  uint32_t cw[BITS];
  uint32_t csw, czw;  // words holding the scale and zero (converted when stored)
  bool csh, czh;
  uint4 xr[XV];
  uint32_t xok;  // bit v: X piece v lies inside X
};

template <int BITS, bool BF16, int NT, int MT, int KB_>
__global__ __launch_bounds__(256) void dq_tile_k(LinArgs a) {
  using C = DtCfg<NT, MT, KB_>;
  constexpr int KB = C::KB, P = C::P, XV = C::XV;
  static_assert(XV <= 32, "validity bits");
  __shared__ __attribute__((aligned(16))) uint16_t sW[2][NT * P];
  __shared__ __attribute__((aligned(16))) uint16_t sX[2][MT * P];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * NT;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * MT;
  const int nsteps = static_cast<int>(a.K / KB);
  const bool coder = wave < C::CW;  // wave-uniform: this wave loads and dequantises codes

  const int wr = (tid / C::CPR) % NT, wc = tid % C::CPR;
  const int64_t wn = std::min<int64_t>(n0 + wr, a.N - 1);
  const uint8_t* wrow = a.packed + wn * a.pitch;
  using St = DtStage<BITS, XV>;
  // loads are branch-free (rows past M read row 0 and are zeroed when stored)
  // so that a stage's loads stay in flight across the multiply
  auto load = [&](int step, St& R) {
    const int64_t k = static_cast<int64_t>(step) * KB + 32 * wc;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(wrow + k * BITS / 8);
    if (!coder) {
    } else if constexpr (BITS == 4) {
      const uint4 v = *reinterpret_cast<const uint4*>(src);
      R.cw[0] = v.x; R.cw[1] = v.y; R.cw[2] = v.z; R.cw[3] = v.w;
    } else if constexpr (BITS == 8) {
      const uint4 v0 = reinterpret_cast<const uint4*>(src)[0], v1 = reinterpret_cast<const uint4*>(src)[1];
      R.cw[0] = v0.x; R.cw[1] = v0.y; R.cw[2] = v0.z; R.cw[3] = v0.w;
      R.cw[4] = v1.x; R.cw[5] = v1.y; R.cw[6] = v1.z; R.cw[7] = v1.w;
    } else if constexpr (BITS == 2) {
      const uint2 v = *reinterpret_cast<const uint2*>(src);
      R.cw[0] = v.x; R.cw[1] = v.y;
    } else {
      R.cw[0] = src[0]; R.cw[1] = src[1]; R.cw[2] = src[2];
    }
    // a 64-bit division here is a divergent branch that made the compiler wait for the loads
    const int64_t g = static_cast<int>(k) / a.gs;
    if (coder) {
      R.csw = elem_word(a.scales, wn * a.ngroups + g, a.sz_dtype, R.csh);
      R.czw = elem_word(a.zeros, wn * a.ngroups + g, a.sz_dtype, R.czh);
    }
    R.xok = 0;
#pragma unroll
    for (int v = 0; v < XV; ++v) {
      const int e = tid + 256 * v;
      const int64_t m = m0 + e / (KB / 8);
      const bool in = m < a.M;
      R.xr[v] = *reinterpret_cast<const uint4*>(a.x + (in ? m : 0) * a.K + static_cast<int64_t>(step) * KB +
                                                8 * (e % (KB / 8)));
      R.xok |= in ? 1u << v : 0u;
    }
  };
  auto store = [&](int buf, const St& R) {
    if (coder) {
      uint32_t d[16];
      dq_chunk<BITS, BF16>(R.cw, elem_value(R.csw, R.csh, a.sz_dtype), elem_value(R.czw, R.czh, a.sz_dtype), d,
                           std::make_integer_sequence<int, 16>{});
      uint4* dst = reinterpret_cast<uint4*>(&sW[buf][wr * P + 32 * wc]);
#pragma unroll
      for (int q = 0; q < 4; ++q) dst[q] = uint4{d[4 * q], d[4 * q + 1], d[4 * q + 2], d[4 * q + 3]};
    }
#pragma unroll
    for (int v = 0; v < XV; ++v) {
      const int e = tid + 256 * v;
      *reinterpret_cast<uint4*>(&sX[buf][(e / (KB / 8)) * P + 8 * (e % (KB / 8))]) =
          (R.xok >> v) & 1u ? R.xr[v] : uint4{0u, 0u, 0u, 0u};
    }
  };

  // waves 2 x 2: NT / 2 weight rows x MT / 2 activation rows each, 32 x 32 blocks
  constexpr int BN = NT / 64, BM = MT / 64;
  const int wbase = (NT / 2) * (wave >> 1), mbase = (MT / 2) * (wave & 1);
  f32x16 acc[BN][BM];
#pragma unroll
  for (int i = 0; i < BN; ++i)
#pragma unroll
    for (int j = 0; j < BM; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
  auto compute = [&](int buf) {
#pragma unroll
    for (int kk = 0; kk < KB / 16; ++kk) {
      uint4 fa[BN], fb[BM];
#pragma unroll
      for (int i = 0; i < BN; ++i)
        fa[i] = *reinterpret_cast<const uint4*>(&sW[buf][(wbase + 32 * i + (lane & 31)) * P + 16 * kk + 8 * (lane >> 5)]);
#pragma unroll
      for (int j = 0; j < BM; ++j)
        fb[j] = *reinterpret_cast<const uint4*>(&sX[buf][(mbase + 32 * j + (lane & 31)) * P + 16 * kk + 8 * (lane >> 5)]);
#pragma unroll
      for (int i = 0; i < BN; ++i)
#pragma unroll
        for (int j = 0; j < BM; ++j) {
          if constexpr (BF16)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fa[i]),
                                                                __builtin_bit_cast(bf16x8, fb[j]), acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, fa[i]),
                                                               __builtin_bit_cast(f16x8, fb[j]), acc[i][j], 0, 0, 0);
        }
    }
  };

  // two register stages: the loads of step s + 2 are issued before step s is
  // multiplied, so each has two steps of multiply to land before its store
  St R0, R1;
  load(0, R0);
  if (nsteps > 1) load(1, R1);
  store(0, R0);
  __syncthreads();
  for (int step = 0; step < nsteps; step += 2) {
    if (step + 2 < nsteps) load(step + 2, R0);
    compute(0);
    if (step + 1 < nsteps) store(1, R1);
    __syncthreads();
    if (step + 1 >= nsteps) break;
    if (step + 3 < nsteps) load(step + 3, R1);
    compute(1);
    if (step + 2 < nsteps) store(0, R0);
    __syncthreads();
  }
  // 32x32 layout: lane l, register v -> W row 8 (v / 4) + 4 (l / 32) + v % 4, X row l % 32
#pragma unroll
  for (int i = 0; i < BN; ++i)
#pragma unroll
    for (int j = 0; j < BM; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t n = n0 + wbase + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        const int64_t m = m0 + mbase + 32 * j + (lane & 31);
        if (n < a.N && m < a.M) {
          float r = acc[i][j][v];
          if (a.bias) r += load_elem(a.bias, n, a.bias_dtype);
          store_elem(a.y, m * a.N + n, a.y_dtype, r);
        }
      }
}

// Products with 4- or 3-bit codes and 16 < M <= 384 (K % 128 == 0, group
// size % 32 == 0): the weights never pass through LDS.  A workgroup owns
// NW * WAVES weight rows x MT activation rows over its range of K (all of K,
// or one of gridDim.z equal ranges of 128-column blocks), with
// WAVES compute waves and L loader waves.  Per 128-column block the loaders
// stage the workgroup's MT x 128 piece of X in LDS (double-buffered, each
// 8-column piece permuted into the order the codes decode in) and every
// compute wave reads all of it.  A compute wave's NW rows are its own: lane
// (r, g) loads codes 32 g .. 32 g + 31 of row r (the column bijection of
// dq_reg4_k), decodes the block's four words into the A operands of its four
// MFMA steps ((q - z) exact, one rounding of the product by s, as in the LDS
// paths) and multiplies each against the MT / 16 X fragments of its step, so
// a code is decoded once and used MT times.  Loads complete in issue order per
// wave, so the X loads live in their own waves: a compute wave's queue holds
// only codes and scales, kept S blocks ahead in S register slots.
template <int NW, int BITS>
struct RxCodes {
  uint32_t cw[NW / 16][BITS];
  uint32_t sw[NW / 16], zw[NW / 16];
  bool sh[NW / 16], zh[NW / 16];
};

template <int BITS, bool BF16, int NW, int WAVES, int L, int MT, int S, int OCC, int XD>
__global__ __launch_bounds__(64 * (WAVES + L)) __attribute__((amdgpu_waves_per_eu(OCC, OCC))) void dq_rx_k(LinArgs a) {
  static_assert(BITS == 4 || BITS == 3, "4- or 3-bit codes");
  constexpr int NB = NW / 16, MB = MT / 16;
  constexpr int P = 128 + 8;              // LDS row pitch (halves)
  constexpr int XP = MT * 16 / (64 * L);  // 16-byte X pieces per loader lane and block
  static_assert(NW % 16 == 0 && MT % 16 == 0 && (MT * 16) % (64 * L) == 0 && S >= 2 && S % 2 == 0, "tile shape");
  __shared__ __attribute__((aligned(16))) uint16_t sX[2][MT * P];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * MT;
  // split-K: this workgroup's 128-column blocks kb0 .. kb0 + nblk - 1
  const int ktot = static_cast<int>(a.K / 128);
  const int bps = static_cast<int>(cdiv(ktot, gridDim.z));
  const int kb0 = static_cast<int>(blockIdx.z) * bps;
  const int nblk = std::min(ktot - kb0, bps);
  const int nsteps = static_cast<int>(cdiv(nblk, S)) * S;  // whole rounds of the S code slots

  if (wave >= WAVES) {
    // the loaders' LDS stores compete with the compute waves' fragment
    // reads; at the default priority they waited behind them and the
    // barrier held the compute waves (per-wave timestamps at 4096 x 14336,
    // M = 128: stores 3200 -> 1000 cycles a block, compute waves' barrier
    // wait 1550 -> 920 cycles)
    __builtin_amdgcn_s_setprio(3);
    // loaders: piece e = 64 (wave - WAVES) + 64 L v + lane is row e / 16,
    // columns 8 (e % 16) .. + 7 of the block, read through a buffer descriptor
    // that ends at the last row of X (rows past M read as zeros, with no
    // address arithmetic per piece)
    const int e0 = 64 * (wave - WAVES) + lane;
    const int64_t rows = std::min<int64_t>(MT, a.M - m0);
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x + m0 * a.K, static_cast<uint32_t>(rows * a.K * 2));
    const uint32_t voff = static_cast<uint32_t>((e0 / 16) * a.K * 2 + 16 * (e0 % 16));
    // XD register sets: block b is loaded into set b % XD, XD blocks before
    // it is stored.  With one set the loop waits a full memory round trip per
    // block; two give a load two blocks' time to arrive, where the compute
    // waves leave the registers for them.  The loads are unconditional (past
    // the last block they repeat it), so every path issues the same loads
    // and each wait is for the oldest set only
    uint4 xr[XD][XP];
    auto load_x = [&](int b, int set) {
      b = std::min(b, nblk - 1);
#pragma unroll
      for (int v = 0; v < XP; ++v) {
        const uint32_t off = static_cast<uint32_t>((4 * L * v * a.K + static_cast<int64_t>(kb0 + b) * 128) * 2);
        xr[set][v] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xrs, voff + off, 0, 0));
      }
    };
    auto store_x = [&](int buf, int set) {
#pragma unroll
      for (int v = 0; v < XP; ++v) {
        const int e = e0 + 64 * L * v;
        *reinterpret_cast<uint4*>(&sX[buf][(e / 16) * P + 8 * (e % 16)]) = perm_0415(xr[set][v]);
      }
    };
    if constexpr (XD == 1) {
      load_x(0, 0);
      store_x(0, 0);
      load_x(1, 0);
      __syncthreads();
      for (int j = 0; j < nsteps; ++j) {
        if (j + 1 < nblk) store_x((j + 1) & 1, 0);
        load_x(j + 2, 0);
        __syncthreads();
      }
    } else {
      load_x(0, 0);
      load_x(1, 1);
      store_x(0, 0);
      load_x(2, 0);
      __syncthreads();
      // steps in pairs, so that each set index is a constant (nsteps is a
      // multiple of S, which is even)
      for (int j = 0; j < nsteps; j += 2) {
        if (j + 1 < nblk) store_x(1, 1);
        load_x(j + 3, 1);
        __syncthreads();
        if (j + 2 < nblk) store_x(0, 0);
        load_x(j + 4, 0);
        __syncthreads();
      }
    }
    return;
  }

  const int r16 = lane & 15, g4 = lane >> 4;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * (NW * WAVES) + NW * wave;
  const uint8_t* wrow[NB];
  int64_t wn[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    wn[i] = std::min<int64_t>(n0 + 16 * i + r16, a.N - 1);
    wrow[i] = a.packed + wn[i] * a.pitch;
  }
  using Cd = RxCodes<NW, BITS>;
  auto load_codes = [&](int b, Cd& C) {
    const int64_t k = static_cast<int64_t>(kb0 + b) * 128 + 32 * g4;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const uint32_t* src = reinterpret_cast<const uint32_t*>(wrow[i] + k * BITS / 8);
      if constexpr (BITS == 4) {
        const uint4 v = *reinterpret_cast<const uint4*>(src);
        C.cw[i][0] = v.x; C.cw[i][1] = v.y; C.cw[i][2] = v.z; C.cw[i][3] = v.w;
      } else {
        C.cw[i][0] = src[0]; C.cw[i][1] = src[1]; C.cw[i][2] = src[2];
      }
    }
    const int64_t g = static_cast<int>(k) / a.gs;  // 32-bit division (K < 2^31)
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      C.sw[i] = elem_word(a.scales, wn[i] * a.ngroups + g, a.sz_dtype, C.sh[i]);
      C.zw[i] = elem_word(a.zeros, wn[i] * a.ngroups + g, a.sz_dtype, C.zh[i]);
    }
  };

  auto mfma = [](uint4 fa, uint4 fb, f32x4 c) {
    if constexpr (BF16)
      return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, fa), __builtin_bit_cast(bf16x8, fb), c,
                                                     0, 0, 0);
    else
      return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, fa), __builtin_bit_cast(f16x8, fb), c, 0,
                                                    0, 0);
  };
  // GPTQ zero points are integers: with fp16 activations, fp16 scales (exact
  // in the packed multiply, so (q - z) * s rounds once) and every zero the
  // wave uses (its rows, the groups of this workgroup's columns) an integer
  // in [0, 1023] the decode is packed fp16 math ((1024 + q) - (1024 + z)
  // exact, then * s), decided once.  Eight loads per lane are in flight: one
  // dependent load per group made the check a chain of memory round trips
  // ahead of the first block
  bool pk = !BF16 && a.sz_dtype == GPTQ_F16;
  if constexpr (!BF16) {
    if (pk) {
      const int64_t g_lo = static_cast<int64_t>(kb0) * 128 / a.gs;
      const int64_t g_hi = std::min<int64_t>(a.ngroups, (static_cast<int64_t>(kb0 + nblk) * 128 - 1) / a.gs + 1);
      // fp16 zeros (pk requires them); the check combines with `&`, not
      // `&&`: a short-circuit let the compiler load each zero only after the
      // previous one passed, a chain of 8 NB dependent loads with 32 rows per
      // wave (the same time at the Llama-3-8B layer shapes, where the zeros
      // hit the cache; now one round trip whatever the cache holds)
      const _Float16* zh = static_cast<const _Float16*>(a.zeros);
      bool ok = true;
      for (int64_t g0 = g_lo + g4; g0 < g_hi; g0 += 32) {
        float z[8][NB];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int64_t g = std::min<int64_t>(g0 + 4 * u, g_hi - 1);
#pragma unroll
          for (int i = 0; i < NB; ++i) z[u][i] = static_cast<float>(zh[wn[i] * a.ngroups + g]);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
          for (int i = 0; i < NB; ++i)
            ok = ok & (z[u][i] == rintf(z[u][i])) & (z[u][i] >= 0.0f) & (z[u][i] <= 1023.0f);
      }
      pk = ok;
    }
    pk = __all(pk);
  }

  f32x4 acc[NB][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // a block: its weight fragments are decoded first (one wave-uniform
  // branch between the packed and the fp32 decode), then the four MFMA steps
  // run as a software pipeline, the X fragments of step kk + 1 read while
  // step kk is multiplied (the scheduling groups fix that order; left alone
  // the compiler waits for each fragment right before its MFMA)
  auto compute = [&](int buf, const Cd& C) {
    uint4 fa[4][NB];
    auto decode = [&](auto packed) {
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const float s = elem_value(C.sw[i], C.sh[i], a.sz_dtype);
        const float z = elem_value(C.zw[i], C.zh[i], a.sz_dtype);
        const uint32_t zz = __builtin_bit_cast(uint32_t, f16x2{static_cast<_Float16>(1024.0f + z),
                                                                static_cast<_Float16>(1024.0f + z)});
        const uint32_t sh = __builtin_bit_cast(uint32_t, f16x2{static_cast<_Float16>(s), static_cast<_Float16>(s)});
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          uint32_t pr[4];
          step_pairs<BITS>(C.cw[i], kk, pr);
          if constexpr (decltype(packed)::value)
            fa[kk][i] = dq_word_0415<true>(pr, zz, sh, 0.0f, 0.0f);
          else
            fa[kk][i] = dq_word_0415<false, BF16>(pr, 0u, 0u, s, z);
        }
      }
    };
    if (pk)
      decode(std::true_type{});
    else
      decode(std::false_type{});
    const uint16_t* xs = &sX[buf][r16 * P + 32 * g4];
    uint4 fb[2][MB];
#pragma unroll
    for (int j = 0; j < MB; ++j) fb[0][j] = *reinterpret_cast<const uint4*>(xs + 16 * j * P);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int c = kk & 1, n = c ^ 1;
      if (kk + 1 < 4) {
#pragma unroll
        for (int j = 0; j < MB; ++j) fb[n][j] = *reinterpret_cast<const uint4*>(xs + 16 * j * P + 8 * (kk + 1));
      }
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < MB; ++j) acc[i][j] = mfma(fa[kk][i], fb[c][j], acc[i][j]);
      if (kk + 1 < 4) {
        __builtin_amdgcn_sched_group_barrier(0x100, MB, 0);       // the next step's X fragments first
        __builtin_amdgcn_sched_group_barrier(0x008, NB * MB, 0);  // then this step's MFMAs
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // block j is multiplied from slot j % S, which then takes the codes of
  // block j + S.  The loads are unconditional (past the last block they
  // repeat it) and the steps come in whole rounds, so every path through the
  // loop issues the same loads and each wait is for the oldest slot only.
  Cd C[S];
#pragma unroll
  for (int u = 0; u < S; ++u) load_codes(std::min(u, nblk - 1), C[u]);
  __syncthreads();
  for (int j0 = 0; j0 < nsteps; j0 += S) {
#pragma unroll
    for (int u = 0; u < S; ++u) {
      const int j = j0 + u;
      if (j < nblk) compute(j & 1, C[u]);
      load_codes(std::min(j + S, nblk - 1), C[u]);
      __syncthreads();
    }
  }

  // 16x16 layout: lane l, register v -> weight row 4 (l / 16) + v, X row l % 16;
  // four consecutive outputs of a row go out as one 8-byte store (split-K:
  // fp32 partial sums, 16 bytes, without the bias)
  if (gridDim.z > 1) {
    float* part = a.part + static_cast<int64_t>(blockIdx.z) * a.M * a.N;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int64_t n = n0 + 16 * i + 4 * g4;
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        const int64_t m = m0 + 16 * j + r16;
        if (m >= a.M) continue;
        if (n + 3 < a.N && (a.N & 3) == 0) {
          *reinterpret_cast<f32x4*>(part + m * a.N + n) = acc[i][j];
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v)
            if (n + v < a.N) part[m * a.N + n + v] = acc[i][j][v];
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int64_t n = n0 + 16 * i + 4 * g4;
    float bv[4] = {0.f, 0.f, 0.f, 0.f};
    if (a.bias) {
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (n + v < a.N) bv[v] = load_elem(a.bias, n + v, a.bias_dtype);
    }
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const int64_t m = m0 + 16 * j + r16;
      if (m >= a.M) continue;
      const float r[4] = {acc[i][j][0] + bv[0], acc[i][j][1] + bv[1], acc[i][j][2] + bv[2], acc[i][j][3] + bv[3]};
      if (a.y_dtype != GPTQ_F32 && n + 3 < a.N && (a.N & 3) == 0) {
        uint32_t h[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) h[v] = a.y_dtype == GPTQ_BF16 ? f32_to_bf16_bits(r[v]) : f32_to_f16_bits(r[v]);
        *reinterpret_cast<uint2*>(a.y + m * a.N + n) = uint2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (n + v < a.N) store_elem(a.y, m * a.N + n + v, a.y_dtype, r[v]);
      }
    }
  }
}

template <int BITS, bool BF16, int NW, int WAVES, int L, int MT, int S, int OCC, int XD>
int launch_rx(hipStream_t st, const LinArgs& a, int splits = 1) {
  const dim3 grid(static_cast<unsigned>(cdiv(a.N, NW * WAVES)), static_cast<unsigned>(cdiv(a.M, MT)),
                  static_cast<unsigned>(splits));
  hipLaunchKernelGGL((dq_rx_k<BITS, BF16, NW, WAVES, L, MT, S, OCC, XD>), grid, dim3(64 * (WAVES + L)), 0, st, a);
  int rc = check_launch("dq_rx");
  if (rc != GPTQ_OK || splits == 1) return rc;
  const int64_t quads = a.M * a.N / 4;
  hipLaunchKernelGGL(splitk_reduce_k, dim3(static_cast<unsigned>(cdiv(quads, 256))), dim3(256), 0, st, a.part, splits,
                     a.M, a.N, a.bias, a.bias_dtype, static_cast<void*>(a.y), a.y_dtype);
  return check_launch("splitk_reduce");
}

// Plan of the register-decoded kernel for 16 < M <= 384: compute waves per
// workgroup (8 or 7, i.e. 128 or 112 weight rows) and K splits, chosen so
// that the workgroups fill the 256 CUs as evenly as one round allows.  The
// grid counts below include the activation tiles (128 rows each for M > 128).
//  * >= 192 workgroups of 128 rows: unsplit, 7 waves when <= 256 workgroups
//    of 112 rows cover the layer (24449-28672 rows at M <= 128) or when the
//    grid takes more than one round anyway, else 8.
//  * otherwise, for each wave count, as many K splits as keep the grid
//    within 256 workgroups (none empty), and the wave count whose grid is
//    larger (8 on a tie); unsplit when that is one split and still >= 128
//    workgroups.
// splits = 0: the layout, or M <= 32 on layers of <= 2^24 weights, goes to
// the other kernels (measured at 4096 x 4096, M = 24 / 32: dq_split_k 12.5 /
// 13.6 us against 15.4 / 15.9 us), as does a plan of < 128 workgroups.
// Measured on MI355X (4-bit, M = 128 / 64 / 32, us): 17408-22016 x 4096
// unsplit on 7 waves 59-61 / 39-40 / 35-36 against 92-94 / 52 / 49-51 on the
// tile kernels; 14336 x 4096 split in 2 on 7 waves 42.8 / 29.4 / 24.9 against
// 45.3 / 30.4 / 26.2 on 8; 13824 x 5120 49.4 / 33.4 / 27.4 against 52.6 / 35.1
// / 29.1.  M = 192 / 256 / 320 (against the tile kernels): 4096 x 4096 31 /
// 31 / 38 against 40 / 41 / 48; 14336 x 4096 62 / 64 / 111 against 88 / 88 /
// 170; 4096 x 14336 71 / 73 / 110 against 129 / 129 / 156; 28672 x 4096 123
// / 128 / 176 against 174 / 178 / 257; 5120 x 13824 82 / 85 / 113 against
// 125 / 151 / 156.
// (the plan itself, compute waves and K splits: plan::rx_plan)
using plan::RxPlan;

// the register-decoded kernel with W compute waves, activation tiles of 32,
// 64 or 128 rows by M (M > 128: several tiles of 128)
template <int BITS, bool BF16, int W>
int launch_rx_w(hipStream_t st, const LinArgs& a, int splits) {
  if (a.M <= 32) return launch_rx<BITS, BF16, 16, W, 1, 32, 4, 2, 2>(st, a, splits);
  if (a.M <= 64) return launch_rx<BITS, BF16, 16, W, 2, 64, 4, 2, 2>(st, a, splits);
  return launch_rx<BITS, BF16, 16, W, 2, 128, 4, 2, 2>(st, a, splits);
}

template <int BITS, bool BF16, int NT, int MT, int WAVES>
int launch_split(hipStream_t st, const LinArgs& a) {
  using C = DsCfg<NT, MT, WAVES>;
  const dim3 grid(static_cast<unsigned>(cdiv(a.N, NT)), static_cast<unsigned>(cdiv(a.M, MT)));
  hipLaunchKernelGGL((dq_split_k<BITS, BF16, NT, MT, WAVES>), grid, dim3(64 * WAVES), C::kLds, st, a);
  return check_launch("dq_split");
}

// M <= 16: the register path (4/3-bit) or split-K with 16 waves, weight rows
// per workgroup chosen so that the grid stays >= 256 workgroups while X is
// re-read by fewer of them.  16 < M <= 384 with 4/3-bit codes: the
// register-decoded kernel where its layout and workspace allow.  Otherwise,
// M > 16 (measured on MI355X at N x K = 28672 x
// 4096, 14336 x 4096, 4096 x 14336 and 4096 x 4096, M = 32-128): 64 x 64
// tiles when there are >= 192 of them (128-column steps up to 512 tiles;
// beyond, 64-column steps, where two workgroups per CU pay, on 64 x 128
// tiles for M > 64), 128 x 128 tiles
// for M > 128 when there are >= 256 of those; otherwise split-K over
// 16-row workgroups (one per 16 weight rows fills the GPU at N = 4096),
// with M tiles of 32, 64 or 128 rows.
template <int BITS, bool BF16>
int launch_dq_gemm(hipStream_t st, const LinArgs& a) {
  if constexpr (BITS == 4 || BITS == 3) {
    // the register path stages the workgroup's scales and zeros in <= 64 KB of
    // LDS; 3-bit rows are read as dwords (the pitch must keep them aligned)
    if (a.M <= 16 && 64 * a.ngroups * sizeof(float2) <= 64 * 1024 && (BITS == 4 || a.pitch % 4 == 0)) {
      // measured best per shape class (28672 x 4096, 14336 x 4096, 4096 x 14336;
      // the 16-wave workgroups below 4097 rows: 6.7 / 15.8 us against 7.6 /
      // 19.1 us at 4096 x 4096 / 4096 x 14336, M <= 4)
      if (a.N >= 64 * 256) {
        // 241-256 workgroups of 112 rows fill the CUs once where 64-row ones
        // would leave a quarter of them with one workgroup and the rest with
        // two (measured at 28672 x 4096, M = 16 / 8 / 2: 26.4 / 24.1 / 22.5 us
        // against 26.8 / 25.1 / 23.6 (4-bit), 26.9 / 25.6 / 24.2 against
        // 28.8 / 27.1 / 26.1 (3-bit))
        // Where K <= 4096 and groups span >= 128 columns, dq_row16_k's 7 waves
        // of 16 rows over all of K: 28672 x 4096 at M = 16 / 2 19.7 / 17.8
        // against 23.6 / 20.1 us (4-bit), 22.8 / 20.7 against 24.6 / 22.6
        // (3-bit); slower at 14336 rows (16.9 against 14.9 us at M = 16 with
        // 4 waves, 1 per SIMD) and with 8 waves of 224 workgroups at 28672
        // rows (23.5 us)
        const int64_t w112 = cdiv(a.N, 112);
        if (w112 > 240 && w112 <= 256 && a.ngroups <= 64) {
          if (row16_fits(a, 7)) return launch_row16<BITS, 7, BF16>(st, a);
          return launch_reg4<BITS, 112, 8, BF16>(st, a);
        }
        return launch_reg4<BITS, 64, 4, BF16>(st, a);
      }
      if (a.N >= 32 * 256) {
        const int s = plan::reg4_wide_splits(a.M, a.N, a.K);
        // 8193-16383 rows at M <= 4: 32-row workgroups (measured on MI355X,
        // graph-timed, 4-bit M = 2, us: 14336 x 4096 11.3 against 12.0 with 64
        // rows, 11008 x 4096 11.0 against 11.6, 13824 x 5120 14.0 against 15.9;
        // 3-bit 3-4% faster; at M = 8 and 16 the 64-row workgroups stay faster)
        if (s == 0 && a.M <= 4) return launch_reg4<BITS, 32, 8, BF16>(st, a);
        const bool fits = s > 1 && a.part && static_cast<size_t>(s) * a.M * a.N * sizeof(float) <= a.part_bytes;
        return launch_reg4<BITS, 64, 8, BF16>(st, a, fits ? s : 1);
      }
      if (const int s = plan::reg4_mid_splits(a.M, a.N, a.K)) {
        const bool fits = a.part && static_cast<size_t>(s) * a.M * a.N * sizeof(float) <= a.part_bytes;
        return launch_reg4<BITS, 32, 8, BF16>(st, a, s > 1 && fits ? s : 1);
      }
      if (const int s = plan::reg4_narrow_splits(a.M, a.N, a.K)) {
        if (a.part && static_cast<size_t>(s) * a.M * a.N * sizeof(float) <= a.part_bytes)
          return launch_reg4<BITS, 32, 16, BF16>(st, a, s);
      }
      // 16-row workgroups: 16 waves over K, except for 8 < M <= 16 with
      // K >= 10240 (unsplit there, 8 waves measured 2-3% faster).  Measured
      // on MI355X against 8 waves (graph-timed, 4-bit, us): M = 8 / 12 / 16 at
      // 4096 x 4096 6.65 / 7.3 / 7.95 against 7.35 / 7.8 / 8.2, 4096 x 2048
      // 5.0 / 5.1 / 5.3 against 5.2 / 5.4 / 5.6, M = 5 / 8 at 4096 x 14336
      // 13.9 / 15.0 against 16.2 / 16.3
      if (a.M > 8 && a.K >= 10240) return launch_reg4<BITS, 16, 8, BF16>(st, a);
      return launch_reg4<BITS, 16, 16, BF16>(st, a);
    }
  }
  if constexpr (BITS == 4 || BITS == 3) {
    // 16 < M <= 384: the register-decoded kernel, split over K when the
    // caller's workspace holds the fp32 partial sums (else the kernels below).
    // Measured on MI355X (4-bit, us; before: the tile and split kernels below):
    // 28672 x 4096 at M = 128 / 64 / 32: 69 / 45 / 40 against 98 / 56 / 53;
    // 4096 x 14336 at M = 128 / 64 / 32: 50 / 38 / 33 against 112 / 67 / 39;
    // 14336 x 4096 at M = 128 / 64 / 32: 43 / 29 / 25 against 51 / 42 / 41.
    auto fits = [&](const RxPlan& q) {
      return q.splits == 1 ||
             (q.splits > 1 && a.part && static_cast<size_t>(q.splits) * a.M * a.N * sizeof(float) <= a.part_bytes);
    };
    RxPlan p = plan::rx_plan(a.M, a.N, a.K, a.pitch, BITS);
    if (p.rows == 32 && !fits(p)) p = plan::rx_plan(a.M, a.N, a.K, a.pitch, BITS, false);  // no room for its partial sums
    if (fits(p)) {
      // 32 rows per wave: 8 waves in all (one loader with one register set),
      // so that each has 256 registers (with 10 waves, or 9 with two loader
      // sets, they spilled), and two code slots
      if (p.rows == 32) return launch_rx<BITS, BF16, 32, 7, 1, 128, 2, 2, 1>(st, a, p.splits);
      return p.waves == 7 ? launch_rx_w<BITS, BF16, 7>(st, a, p.splits) : launch_rx_w<BITS, BF16, 8>(st, a, p.splits);
    }
  }
  if (a.M <= 16) {
    if (a.N >= 64 * 256) return launch_split<BITS, BF16, 64, 16, 8>(st, a);
    if (a.N >= 32 * 256) return launch_split<BITS, BF16, 32, 16, 16>(st, a);
    return launch_split<BITS, BF16, 16, 16, 16>(st, a);
  }
  if (a.M > 128 && cdiv(a.N, 128) * cdiv(a.M, 128) >= 256) {
    const dim3 grid(static_cast<unsigned>(cdiv(a.N, 128)), static_cast<unsigned>(cdiv(a.M, 128)));
    hipLaunchKernelGGL((dq_tile_k<BITS, BF16, 128, 128, 64>), grid, dim3(256), 0, st, a);
    return check_launch("dq_tile");
  }
  const int64_t t64 = cdiv(a.N, 64) * cdiv(a.M, 64);
  // 64 < M <= 128 on 5120-row layers (160 tiles): the tiles measured 46 / 114 us
  // against split-K's 84 / 206 us at 5120 x 5120 / 5120 x 13824 (M = 128);
  // at 4096 rows (128 tiles) split-K stays as fast or faster
  if (t64 >= 192 || (a.M > 64 && t64 >= 160)) {
    const dim3 grid(static_cast<unsigned>(cdiv(a.N, 64)), static_cast<unsigned>(cdiv(a.M, 64)));
    if (t64 <= 512) {
      hipLaunchKernelGGL((dq_tile_k<BITS, BF16, 64, 64, 128>), grid, dim3(256), 0, st, a);
    } else if (a.M > 64) {
      // beyond 512 tiles, 64 x 128 tiles (64-column steps) re-read each
      // weight row half as often
      const dim3 g2(static_cast<unsigned>(cdiv(a.N, 64)), static_cast<unsigned>(cdiv(a.M, 128)));
      hipLaunchKernelGGL((dq_tile_k<BITS, BF16, 64, 128, 64>), g2, dim3(256), 0, st, a);
    } else {
      hipLaunchKernelGGL((dq_tile_k<BITS, BF16, 64, 64, 64>), grid, dim3(256), 0, st, a);
    }
    return check_launch("dq_tile");
  }
  if (a.M <= 32) return launch_split<BITS, BF16, 16, 32, 8>(st, a);
  if (a.M <= 64) return launch_split<BITS, BF16, 16, 64, 8>(st, a);
  return launch_split<BITS, BF16, 16, 128, 8>(st, a);
}

// ------------------------------------------------------------- generic ----
__device__ __forceinline__ uint32_t code_at(const uint8_t* __restrict__ row, int64_t pitch, int64_t k, int bits) {
  if (bits == 0) return row[k];
  const int64_t bit = k * bits;
  const int64_t byte = bit >> 3;
  uint32_t v = row[byte];
  if (byte + 1 < pitch) v |= static_cast<uint32_t>(row[byte + 1]) << 8;
  return (v >> (bit & 7)) & ((1u << bits) - 1u);
}

__global__ __launch_bounds__(256) void linear_generic(const void* __restrict__ x, int x_dtype, int64_t M,
                                                      const uint8_t* __restrict__ packed, int bits, int64_t pitch,
                                                      const void* __restrict__ scales, const void* __restrict__ zeros,
                                                      int sz_dtype, const int32_t* __restrict__ g_idx, int gs,
                                                      int64_t ngroups, const void* __restrict__ bias, int bias_dtype,
                                                      int64_t N, int64_t K, void* __restrict__ y) {
  const int64_t w = blockIdx.x * 4LL + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (w >= M * N) return;
  const int64_t m = w / N, n = w - (w / N) * N;
  const uint8_t* row = packed + n * pitch;
  float acc = 0.0f;
  for (int64_t k = lane; k < K; k += 64) {
    const int64_t g = g_idx ? std::min<int64_t>(std::max<int64_t>(g_idx[k], 0), ngroups - 1) : k / gs;
    const float q = static_cast<float>(code_at(row, pitch, k, bits));
    const float z = load_elem(zeros, n * ngroups + g, sz_dtype);
    const float s = load_elem(scales, n * ngroups + g, sz_dtype);
    const float d = q - z;
    const float wv = d * s;
    acc += load_elem(x, m * K + k, x_dtype) * wv;
  }
  acc = wave_sum(acc);
  if (lane == 0) {
    if (bias) acc += load_elem(bias, n, bias_dtype);
    store_elem(y, m * N + n, x_dtype, acc);
  }
}

template <int BITS, bool BF16, bool SZBF, int MAXC, int WS>
int launch_m1(hipStream_t st, const LinArgs& a) {
  // rows per batch: at most 16 code dwords per lane and buffer (measured best on MI355X;
  // 24 for 3-bit codes measured 11-28% slower: uneven batches per wave)
  constexpr int kBudget = 16;
  constexpr int kFit = kBudget / (MAXC * BITS) > 0 ? kBudget / (MAXC * BITS) : 1;
  constexpr int RB = kFit >= 8 ? 8 : kFit >= 4 ? 4 : kFit >= 2 ? 2 : 1;
  const int64_t nbatches = cdiv(a.N, RB);
  const int64_t per_wg = WS == 4 ? 1 : 4;
  const unsigned blocks = static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(cdiv(nbatches, per_wg), 512)));
  hipLaunchKernelGGL((gemv_m1_k<BITS, BF16, SZBF, MAXC, RB, WS>), dim3(blocks), dim3(256), 0, st, a);
  return check_launch("gemv_m1");
}

template <int BITS, bool BF16, bool SZBF>
int launch_m1_k(hipStream_t st, const LinArgs& a) {
  const int64_t nch32 = a.K / 32;
  if (nch32 <= 64) return launch_m1<BITS, BF16, SZBF, 1, 1>(st, a);
  if (nch32 <= 128) return launch_m1<BITS, BF16, SZBF, 2, 1>(st, a);
  if (nch32 <= 512) return launch_m1<BITS, BF16, SZBF, 2, 4>(st, a);
  return launch_m1<BITS, BF16, SZBF, 4, 4>(st, a);
}

// fp16 scales with either activation type; bf16 scales with bf16 activations
template <int BITS, bool BF16>
int launch_m1_sz(hipStream_t st, const LinArgs& a) {
  if constexpr (BF16) {
    if (a.sz_dtype == GPTQ_BF16) return launch_m1_k<BITS, true, true>(st, a);
  }
  return launch_m1_k<BITS, BF16, false>(st, a);
}

// the M = 1 kernel's layout: buffer descriptors address a row (pitch bytes)
// and the scale/zero arrays with 31-bit offsets
bool m1_layout(const LinArgs& a) {
  const bool bf = a.y_dtype == GPTQ_BF16;
  return a.M == 1 && a.K % 32 == 0 && a.gs % 32 == 0 && a.K <= 4 * 256 * 32 &&
         (a.sz_dtype == GPTQ_F16 || (bf && a.sz_dtype == GPTQ_BF16)) && a.N * a.ngroups * 2 <= INT32_MAX &&
         (reinterpret_cast<uintptr_t>(a.x) % 16) == 0;
}

template <int BITS, bool BF16>
int launch_fast(hipStream_t st, const LinArgs& a) {
  using F = Fmt<BITS>;
  const int64_t nch = a.K / F::CB;
  if (m1_layout(a)) return launch_m1_sz<BITS, BF16>(st, a);
  // M = 2..4: the MFMA kernels below (measured 2-3x faster than gemv_k at
  // 28672 x 4096); gemv_k serves the layouts they do not take
  const bool dq_layout = a.K % 128 == 0 && a.gs % 32 == 0;
  if (a.M <= 4 && !dq_layout) {
    const size_t lds = static_cast<size_t>(a.M) * a.K * 2 + static_cast<size_t>(a.M) * nch * 4;
    if (lds <= 64 * 1024) {
      const int64_t nbatches = cdiv(a.N, kRB);
      const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(cdiv(nbatches, 4), 2048));
      switch (a.M) {
        case 1: hipLaunchKernelGGL((gemv_k<BITS, BF16, 1>), dim3(blocks), dim3(256), lds, st, a); break;
        case 2: hipLaunchKernelGGL((gemv_k<BITS, BF16, 2>), dim3(blocks), dim3(256), lds, st, a); break;
        case 3: hipLaunchKernelGGL((gemv_k<BITS, BF16, 3>), dim3(blocks), dim3(256), lds, st, a); break;
        default: hipLaunchKernelGGL((gemv_k<BITS, BF16, 4>), dim3(blocks), dim3(256), lds, st, a); break;
      }
      return check_launch("gemv");
    }
  }
  // 128-column blocks, one group per 32-code chunk
  if (dq_layout) return launch_dq_gemm<BITS, BF16>(st, a);
  const dim3 grid(static_cast<unsigned>(cdiv(a.N, 16)), static_cast<unsigned>(cdiv(a.M, kMT * 16)));
  hipLaunchKernelGGL((dq_mfma_k<BITS, BF16>), grid, dim3(256), 0, st, a);
  return check_launch("dq_mfma");
}

}  // namespace
}  // namespace gptq

using namespace gptq;

namespace gptq {
namespace {

// out[m][j] = x[m][perm[j]] (indices clamped to [0, K)).  One element per
// thread: measured faster than 8 columns per thread with 16-byte stores,
// whose grid is too small at M = 1 (7.0 against 7.9 us at K = 4096).
__global__ __launch_bounds__(256) void gather_cols_k(const void* __restrict__ x, int esz, int64_t M, int64_t K,
                                                     const int32_t* __restrict__ perm, void* __restrict__ out) {
  const int64_t j = blockIdx.x * 256LL + threadIdx.x;
  if (j >= K) return;
  const int64_t src = std::min<int64_t>(std::max<int64_t>(perm[j], 0), K - 1);
  for (int64_t m = blockIdx.y; m < M; m += gridDim.y) {
    if (esz == 4)
      static_cast<float*>(out)[m * K + j] = static_cast<const float*>(x)[m * K + src];
    else
      static_cast<uint16_t*>(out)[m * K + j] = static_cast<const uint16_t*>(x)[m * K + src];
  }
}

void launch_gather(hipStream_t st, const void* x, int esz, int64_t M, int64_t K, const int32_t* perm, void* out) {
  const dim3 grid(static_cast<unsigned>(cdiv(K, 256)), static_cast<unsigned>(std::min<int64_t>(M, 65535)));
  hipLaunchKernelGGL(gather_cols_k, grid, dim3(256), 0, st, x, esz, M, K, perm, out);
}

using plan::check_linear_args;

LinArgs make_linear_args(const void* x, int x_dtype, int64_t M, const uint8_t* packed, int bits, const void* scales,
                         const void* zeros, int sz_dtype, int group_size, int64_t ngroups, const void* bias,
                         int bias_dtype, int64_t N, int64_t K, void* y) {
  const int eb = bits == 0 ? 8 : bits;
  const int64_t pitch = (K * eb + 7) / 8;
  return LinArgs{static_cast<const uint16_t*>(x), M, packed, pitch, scales, zeros, sz_dtype, group_size, ngroups,
                 bias, bias_dtype, N, K, static_cast<uint16_t*>(y), x_dtype};
}

// the fast kernels take 16-bit activations, contiguous groups and chunks of
// whole 128-bit loads
bool fast_layout(const LinArgs& a, int bits, const int32_t* g_idx) {
  const int eb = bits == 0 ? 8 : bits;
  const int cb = eb == 4 ? 32 : eb == 2 ? 64 : eb == 8 ? 16 : 128;
  return a.y_dtype != GPTQ_F32 && !g_idx && a.K % cb == 0 && a.gs % cb == 0 && a.K % 32 == 0 &&
         (reinterpret_cast<uintptr_t>(a.packed) % 16) == 0 && (reinterpret_cast<uintptr_t>(a.x) % 16) == 0;
}

int dispatch_linear(hipStream_t st, const LinArgs& a, int bits, const int32_t* g_idx) {
  const int eb = bits == 0 ? 8 : bits;
  if (fast_layout(a, bits, g_idx)) {
    const bool bf = a.y_dtype == GPTQ_BF16;
    switch (eb) {
      case 4: return bf ? launch_fast<4, true>(st, a) : launch_fast<4, false>(st, a);
      case 3: return bf ? launch_fast<3, true>(st, a) : launch_fast<3, false>(st, a);
      case 2: return bf ? launch_fast<2, true>(st, a) : launch_fast<2, false>(st, a);
      default: return bf ? launch_fast<8, true>(st, a) : launch_fast<8, false>(st, a);
    }
  }
  const unsigned blocks = static_cast<unsigned>(cdiv(a.M * a.N, 4));
  hipLaunchKernelGGL(linear_generic, dim3(blocks), dim3(256), 0, st, static_cast<const void*>(a.x), a.y_dtype, a.M,
                     a.packed, bits == 0 ? 0 : bits, a.pitch, a.scales, a.zeros, a.sz_dtype, g_idx, a.gs, a.ngroups,
                     a.bias, a.bias_dtype, a.N, a.K, static_cast<void*>(a.y));
  return check_launch("linear_generic");
}

}  // namespace
}  // namespace gptq

using namespace gptq;

extern "C" int gptq_linear(const void* x, int x_dtype, int64_t M, const uint8_t* packed, int bits, const void* scales,
                           const void* zeros, int sz_dtype, const int32_t* g_idx, int group_size, int64_t ngroups,
                           const void* bias, int bias_dtype, int64_t N, int64_t K, void* y, gptq_stream_t stream) {
  clear_error();
  const int rc = check_linear_args(x, x_dtype, M, packed, bits, scales, zeros, sz_dtype, g_idx, group_size, ngroups,
                                   bias, bias_dtype, N, K, y);
  if (rc != GPTQ_OK || M == 0) return rc;
  const LinArgs a = make_linear_args(x, x_dtype, M, packed, bits, scales, zeros, sz_dtype, group_size, ngroups, bias,
                                     bias_dtype, N, K, y);
  return dispatch_linear(as_hip(stream), a, bits, g_idx);
}

// (gptq_linear_perm_workspace_size and gptq_linear_workspace_size, with the
// split-K partial-sum bytes, are in plan.cpp)

extern "C" int gptq_linear_ws(const void* x, int x_dtype, int64_t M, const int32_t* perm, const uint8_t* packed,
                              int bits, const void* scales, const void* zeros, int sz_dtype, const int32_t* g_idx,
                              int group_size, int64_t ngroups, const void* bias, int bias_dtype, int64_t N, int64_t K,
                              void* y, void* workspace, size_t workspace_bytes, gptq_stream_t stream) {
  clear_error();
  const int rc = check_linear_args(x, x_dtype, M, packed, bits, scales, zeros, sz_dtype, g_idx, group_size, ngroups,
                                   bias, bias_dtype, N, K, y);
  if (rc != GPTQ_OK || M == 0) return rc;
  hipStream_t st = as_hip(stream);
  LinArgs a = make_linear_args(x, x_dtype, M, packed, bits, scales, zeros, sz_dtype, group_size, ngroups, bias,
                               bias_dtype, N, K, y);
  size_t used = 0;
  if (perm) {
    const size_t need = static_cast<size_t>(M) * K * dtype_size(x_dtype);
    GPTQ_REQUIRE(workspace && workspace_bytes >= need, GPTQ_ERR_WORKSPACE,
                 "linear_ws: workspace of %zu bytes, %zu needed for the gathered activations", workspace_bytes, need);
    launch_gather(st, x, dtype_size(x_dtype), M, K, perm, workspace);
    const int lrc = check_launch("gather_cols");
    if (lrc != GPTQ_OK) return lrc;
    a.x = static_cast<const uint16_t*>(workspace);
    used = plan::round256(need);
  }
  // the rest of the workspace, from its first 256-byte boundary, holds
  // split-K partial sums when the kernel takes them and they fit (else the
  // layer runs unsplit)
  if (workspace) {
    const uintptr_t base = reinterpret_cast<uintptr_t>(workspace);
    const uintptr_t p0 = (base + used + 255) / 256 * 256;
    if (p0 < base + workspace_bytes) {
      a.part = reinterpret_cast<float*>(p0);
      a.part_bytes = base + workspace_bytes - p0;
    }
  }
  return dispatch_linear(st, a, bits, g_idx);
}

extern "C" int gptq_linear_perm(const void* x, int x_dtype, int64_t M, const int32_t* perm, const uint8_t* packed,
                                int bits, const void* scales, const void* zeros, int sz_dtype, const int32_t* g_idx,
                                int group_size, int64_t ngroups, const void* bias, int bias_dtype, int64_t N,
                                int64_t K, void* y, void* workspace, size_t workspace_bytes, gptq_stream_t stream) {
  clear_error();
  GPTQ_REQUIRE(perm, GPTQ_ERR_ARG, "linear_perm: null perm");
  const int rc = check_linear_args(x, x_dtype, M, packed, bits, scales, zeros, sz_dtype, g_idx, group_size, ngroups,
                                   bias, bias_dtype, N, K, y);
  if (rc != GPTQ_OK || M == 0) return rc;
  hipStream_t st = as_hip(stream);
  LinArgs a = make_linear_args(x, x_dtype, M, packed, bits, scales, zeros, sz_dtype, group_size, ngroups, bias,
                               bias_dtype, N, K, y);
  // x is gathered once, before the launch, for every M: inside the kernels
  // each wave would gather all of x with scattered loads, and one 16-bit load
  // per lane touches 64 cache lines (M = 1 at 4096 x 4096 measured 13.4 us
  // that way against 4.8 us for the GEMV alone); one gather per workgroup
  // into LDS, its first weight loads already issued, measured 7.4 / 18.9 us
  // against 7.1 / 11.2 us with this launch at 4096 x 4096 / 4096 x 14336
  const size_t need = gptq_linear_perm_workspace_size(M, K, x_dtype);
  GPTQ_REQUIRE(workspace && workspace_bytes >= need, GPTQ_ERR_WORKSPACE,
               "linear_perm: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  launch_gather(st, x, dtype_size(x_dtype), M, K, perm, workspace);
  const int lrc = check_launch("gather_cols");
  if (lrc != GPTQ_OK) return lrc;
  a.x = static_cast<const uint16_t*>(workspace);
  return dispatch_linear(st, a, bits, g_idx);
}

// ------------------------------------------------- no-allocation variant --
// gptq_linear_perm_noalloc keeps the gathered activations in `scratch`, a
// file-scope device array (every GPU the library runs on holds its own copy
// until the process ends), instead of a caller workspace.  Host code never
// uses the array's name as an address: at the first call on a device its
// address on that device is looked up once (hipGetSymbolAddress, with that
// device current) and kept per device.
constexpr size_t kNoAllocScratchBytes = size_t(4) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace gptq {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// this device's address of `scratch` (looked up once per device)
int scratch_address(hipStream_t st, void** out) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  GPTQ_REQUIRE(e == hipSuccess, GPTQ_ERR_DEVICE, "linear_perm_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  int dev = cur;
  if (st != nullptr) {
    e = hipStreamGetDevice(st, &dev);
    GPTQ_REQUIRE(e == hipSuccess, GPTQ_ERR_DEVICE, "linear_perm_noalloc: hipStreamGetDevice: %s",
                 hipGetErrorString(e));
  }
  GPTQ_REQUIRE(dev >= 0 && dev < kMaxDevices, GPTQ_ERR_DEVICE, "linear_perm_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    if (dev != cur) {
      e = hipSetDevice(dev);
      GPTQ_REQUIRE(e == hipSuccess, GPTQ_ERR_DEVICE, "linear_perm_noalloc: hipSetDevice(%d): %s", dev,
                   hipGetErrorString(e));
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t back = dev != cur ? hipSetDevice(cur) : hipSuccess;
    GPTQ_REQUIRE(e == hipSuccess && p != nullptr, GPTQ_ERR_DEVICE,
                 "linear_perm_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    GPTQ_REQUIRE(back == hipSuccess, GPTQ_ERR_DEVICE, "linear_perm_noalloc: hipSetDevice(%d): %s", cur,
                 hipGetErrorString(back));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return GPTQ_OK;
}

}  // namespace
}  // namespace gptq

extern "C" size_t gptq_linear_perm_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int gptq_linear_perm_noalloc(const void* x, int x_dtype, int64_t M, const int32_t* perm,
                                        const uint8_t* packed, int bits, const void* scales, const void* zeros,
                                        int sz_dtype, const int32_t* g_idx, int group_size, int64_t ngroups,
                                        const void* bias, int bias_dtype, int64_t N, int64_t K, void* y,
                                        gptq_stream_t stream) {
  clear_error();
  const size_t need = gptq_linear_perm_workspace_size(M, K, x_dtype);
  GPTQ_REQUIRE(need <= kNoAllocScratchBytes, GPTQ_ERR_WORKSPACE,
               "linear_perm_noalloc: %lld x %lld activations need %zu bytes of scratch; the limit is %zu",
               static_cast<long long>(M), static_cast<long long>(K), need, kNoAllocScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_address(as_hip(stream), &ws);
  if (rc != GPTQ_OK) return rc;
  return gptq_linear_perm(x, x_dtype, M, perm, packed, bits, scales, zeros, sz_dtype, g_idx, group_size, ngroups,
                          bias, bias_dtype, N, K, y, ws, kNoAllocScratchBytes, stream);
}
