// fp32 GEMM for the factorisation and the sweep (gfx950), in two forms:
//  * products whose A is not transposed and whose operand rows are 16-byte
//    vectors (every product of the factorisation's recursion and of the
//    sweep's trailing updates) run on bf16 MFMAs over an exact three-way
//    split of the fp32 operands (gemm_x3_kernel, below), at 6/16 of the
//    fp32 MFMA cycles per product;
//  * the rest (the transposed products of the reference-mode inverse,
//    unaligned operands) on v_mfma_f32_32x32x2_f32 (gemm_f32_kernel).
//
// fp32 MFMA kernel: TM x TN output tile per workgroup of 4 waves (2 x 2, each TM/2 x TN/2 =
// FM x FN MFMA 32x32 blocks), BK-deep k stages staged in LDS as [row][k]
// (pitch BK + 2 floats: the two k-rows a 32x32x2 fragment reads land in
// disjoint bank halves), next stage prefetched into registers while the
// current one is multiplied.  Tiles are 128 x 64 (64 x 64 for products that
// would give fewer than 4096 such tiles), 32 deep: small tiles keep enough
// waves resident per CU to hide the load latency of this single-buffered
// pipeline, which measured faster than 128 x 128 or 256 x 128 tiles, and
// than a double-buffered variant with one barrier per stage (fewer resident
// waves), for every product of the factorisation and the sweep.  Operand
// transposition is a compile-time parameter and the loads are branch-free
// (see load_op).  Triangular operands
// skip the k-tiles that are known to be zero; GEMM_C_LOWER skips tiles
// strictly above the diagonal.  With a single triangular flag the tiles are
// dispatched heaviest first (the tiles with the longest k range, or only the
// tiles on or below the diagonal for GEMM_C_LOWER), so that the grid does not
// end on a few long tiles: measured on MI355X at 7168^3 (A = B = C = 7168^2)
// 90.7 / 94.6 / 109.1 / 102.5 -> 117.9 / 116.4 / 115.7 / 110.5 TFLOP/s for
// B <= j, B >= j, A <= i and C lower, with bit-identical results.
#include "gemm.hpp"

namespace gptq {
namespace {

constexpr int kThreads = 256;

struct Operand {
  const float* p;
  int64_t ld;
  bool trans;   // element (r, k) of the operand is p[k * ld + r] when trans
  int64_t rows; // extent along r
};

// Loads the stage (r0..r0+TR-1, k0..k0+BK-1) of an operand viewed as [r][k]
// into registers: TR * BK / 4 float4, NQ per thread.  Elements outside the
// operand are flagged in `ok` (bit 4 q + e) and zeroed by store_op.  Branch-
// free: an out-of-range lane loads from the operand's first element.  Both
// choices keep the loads in flight across the stage's MFMAs: a divergent
// branch around each load, or a select right after it, made the compiler wait
// for the loads before the multiply.  kVec: every float4 is entirely inside
// or entirely outside the operand (16-byte aligned rows and a contiguous
// extent that is a multiple of 4).
template <int TR, int BK, bool kVec, bool kTrans>
__device__ __forceinline__ void load_op(const Operand& o, int64_t r0, int64_t k0, int64_t Kd, int tid,
                                        f32x4 (&pre)[TR * BK / 4 / kThreads], uint32_t& ok) {
  constexpr int NQ = TR * BK / 4 / kThreads;
  static_assert(NQ <= 8, "validity bits");
  ok = 0;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int idx = q * kThreads + tid;
    // contiguous along k (BK / 4 lanes per row), or along r when transposed (TR / 4 lanes per k-row)
    const int64_t r = kTrans ? r0 + (idx % (TR / 4)) * 4 : r0 + idx / (BK / 4);
    const int64_t k = kTrans ? k0 + idx / (TR / 4) : k0 + (idx % (BK / 4)) * 4;
    const int64_t off = kTrans ? k * o.ld + r : r * o.ld + k;
    if constexpr (kVec) {
      const bool in = r < o.rows && k < Kd;
      pre[q] = *reinterpret_cast<const f32x4*>(o.p + (in ? off : 0));
      ok |= in ? 0xFu << (4 * q) : 0u;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool in = kTrans ? (r + e < o.rows && k < Kd) : (r < o.rows && k + e < Kd);
        pre[q][e] = o.p[in ? off + e : 0];
        ok |= in ? 1u << (4 * q + e) : 0u;
      }
    }
  }
}

template <int TR, int BK, bool trans>
__device__ __forceinline__ void store_op(float* s, int tid, f32x4 (&pre)[TR * BK / 4 / kThreads], uint32_t ok) {
  constexpr int NQ = TR * BK / 4 / kThreads;
  constexpr int P = BK + 2;
#pragma unroll
  for (int q = 0; q < NQ; ++q)
#pragma unroll
    for (int e = 0; e < 4; ++e) pre[q][e] = (ok >> (4 * q + e)) & 1u ? pre[q][e] : 0.0f;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int idx = q * kThreads + tid;
    if constexpr (!trans) {
      const int r = idx / (BK / 4), k = (idx % (BK / 4)) * 4;
      float2* d = reinterpret_cast<float2*>(s + r * P + k);
      d[0] = make_float2(pre[q][0], pre[q][1]);
      d[1] = make_float2(pre[q][2], pre[q][3]);
    } else {
      const int k = idx / (TR / 4), r = (idx % (TR / 4)) * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) s[(r + e) * P + k] = pre[q][e];
    }
  }
}

// dispatch order of the output tiles (workgroup index -> tile)
enum TileOrder {
  ORDER_ROWS = 0,       // row-major
  ORDER_ROWS_DESC = 1,  // row-major, last tile row first (A <= i: work grows with i)
  ORDER_COLS_DESC = 2,  // column-major, last tile column first (B <= j)
  ORDER_COLS = 3,       // column-major (B >= j: work falls with j)
  ORDER_LOWER = 4       // only tiles on or below the diagonal, row by row
};

template <int TM, int TN>
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int order, int& tm, int& tn) {
  switch (order) {
    case ORDER_ROWS_DESC: tm = tiles_m - 1 - bid / tiles_n; tn = bid % tiles_n; break;
    case ORDER_COLS_DESC: tn = tiles_n - 1 - bid / tiles_m; tm = bid % tiles_m; break;
    case ORDER_COLS: tn = bid / tiles_m; tm = bid % tiles_m; break;
    case ORDER_LOWER: {
      // tile row r holds c (r + 1) tiles (c = TM / TN), so it starts at
      // c r (r + 1) / 2: r from the quadratic formula, then corrected
      // exactly in integers
      constexpr int c = TM / TN;
      const float q = static_cast<float>(2 * bid) / c;
      int r = static_cast<int>((sqrtf(1.0f + 4.0f * q) - 1.0f) * 0.5f);
      r = r < 0 ? 0 : r;
      while (c * (r + 1) * (r + 2) / 2 <= bid) ++r;
      while (c * r * (r + 1) / 2 > bid) --r;
      tm = r;
      tn = bid - c * r * (r + 1) / 2;
      break;
    }
    default: tm = bid / tiles_n; tn = bid % tiles_n; break;
  }
}

// one product, its tile grid and dispatch order
struct GemmDesc {
  int64_t M, N, Kd;
  float alpha;
  Operand a, b;
  float beta;
  float* C;
  int64_t ldc;
  int flags, tiles_m, tiles_n, order;
};

// output tile `bid` (in dispatch order) of the product d, staged through sA / sB
template <int TM, int TN, int BK, bool kVec, bool kTA, bool kTB>
__device__ __forceinline__ void gemm_tile(const GemmDesc& d, int bid, float* __restrict__ sA,
                                          float* __restrict__ sB) {
  constexpr int P = BK + 2;
  constexpr int FM = TM / 64, FN = TN / 64;  // 32x32 blocks per wave
  constexpr int QA = TM * BK / 4 / kThreads, QB = TN * BK / 4 / kThreads;
  const int64_t M = d.M, N = d.N, Kd = d.Kd, ldc = d.ldc;
  const float alpha = d.alpha, beta = d.beta;
  const Operand& a = d.a;
  const Operand& b = d.b;
  float* __restrict__ C = d.C;
  const int flags = d.flags;
  int tm = 0, tn = 0;
  tile_of<TM, TN>(bid, d.tiles_m, d.tiles_n, d.order, tm, tn);
  const int64_t i0 = static_cast<int64_t>(tm) * TM;
  const int64_t j0 = static_cast<int64_t>(tn) * TN;
  if ((flags & GEMM_C_LOWER) && j0 > i0 + TM - 1) return;

  int64_t kb = 0, ke = Kd;
  if (flags & GEMM_KLIM_A_LE_I) ke = std::min<int64_t>(ke, i0 + TM);
  if (flags & GEMM_KLIM_B_LE_J) ke = std::min<int64_t>(ke, j0 + TN);
  if (flags & GEMM_KLIM_A_GE_I) kb = std::max<int64_t>(kb, i0);
  if (flags & GEMM_KLIM_B_GE_J) kb = std::max<int64_t>(kb, j0);
  kb = (kb / BK) * BK;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 1) * (TM / 2);
  const int wn = (wave & 1) * (TN / 2);

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  f32x4 pa[QA], pb[QB];
  uint32_t oka = 0, okb = 0;
  if (kb < ke) {
    load_op<TM, BK, kVec, kTA>(a, i0, kb, Kd, tid, pa, oka);
    load_op<TN, BK, kVec, kTB>(b, j0, kb, Kd, tid, pb, okb);
  }
  for (int64_t k0 = kb; k0 < ke; k0 += BK) {
    __syncthreads();
    store_op<TM, BK, kTA>(sA, tid, pa, oka);
    store_op<TN, BK, kTB>(sB, tid, pb, okb);
    __syncthreads();
    if (k0 + BK < ke) {
      load_op<TM, BK, kVec, kTA>(a, i0, k0 + BK, Kd, tid, pa, oka);
      load_op<TN, BK, kVec, kTB>(b, j0, k0 + BK, Kd, tid, pb, okb);
    }
#pragma unroll
    for (int kk = 0; kk < BK / 2; ++kk) {
      const int k = kk * 2 + (lane >> 5);
      float fa[FM], fb[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) fa[i] = sA[(wm + i * 32 + (lane & 31)) * P + k];
#pragma unroll
      for (int j = 0; j < FN; ++j) fb[j] = sB[(wn + j * 32 + (lane & 31)) * P + k];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
  }

  // Epilogue, one 32 x 32 block at a time: its 16 reads of C are issued
  // before its stores (interleaved, each store would wait for the read
  // before it -- the compiler cannot tell the addresses apart -- one memory
  // round trip per element instead of one per block).
  const bool lower = (flags & GEMM_C_LOWER) != 0;
  const int64_t rbase = i0 + wm + 4 * (lane >> 5);
  const int64_t cbase = j0 + wn + (lane & 31);
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t col = cbase + j * 32;
      float* cp = C + (rbase + i * 32) * ldc + col;
      float cv[16];
      if (beta != 0.0f) {
        // branch-free: out-of-range lanes read C[0][0] (their value is not stored)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t row = rbase + i * 32 + 8 * (v >> 2) + (v & 3);
          cv[v] = *((row < M && col < N) ? cp + (8 * (v >> 2) + (v & 3)) * ldc : C);
        }
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = rbase + i * 32 + 8 * (v >> 2) + (v & 3);
        if (row < M && col < N && (!lower || row >= col)) {
          float r = alpha * acc[i][j][v];
          if (beta != 0.0f) r += beta * cv[v];
          cp[(8 * (v >> 2) + (v & 3)) * ldc] = r;
        }
      }
    }
}

// ------------------------------------------------ fp32 from bf16 MFMAs ----
// The same product on v_mfma_f32_32x32x16_bf16: every fp32 operand element
// is split exactly into three bf16 parts, v = hi + mid + lo, each part the
// round-to-nearest bf16 of what the previous ones leave (hi carries the top
// 8 significant bits, |mid| <= 2^-8 |v|, |lo| <= 2^-16 |v|), and the six
// cross products down to 2^-16 |a||b| are accumulated in fp32:
//   a b ~ lo_a hi_b + hi_a lo_b + mid_a mid_b + mid_a hi_b + hi_a mid_b + hi_a hi_b.
// Products of bf16 parts are exact in fp32.  The dropped ones (mid lo, lo
// mid, lo lo) are signed, so the error is unbiased, and at most 2^-23 |a||b|
// (measured over 10^6 normal pairs: 0.88 x 2^-24, below the 2^-24 of an fp32
// product's own rounding); each MFMA rounds its 16-product sum into the fp32
// accumulator once.  The bf16 MFMA does 16 times the MACs per cycle of
// v_mfma_f32_32x32x2_f32, so a product costs 6/16 of the fp32 MFMA cycles.
// The parts are made once per element when a stage is staged into LDS (two
// elements per v_cvt_pk_bf16_f32), as three bf16 planes [row][k] with a
// pitch of BK + 8 halves: the 16-byte fragment reads of 16 consecutive rows
// then cover 64 distinct banks.  Operand A is [i][k] (k contiguous); B is
// [j][k] or, kTB, stored [k][j] (j contiguous) and transposed in registers
// by 4 x KR blocks.  Stages that lie inside both operands (all of an
// interior tile's) skip the bounds checks.  Measured on MI355X against the
// fp32 MFMA kernels: the K = 14336 damped factorisation 29.0 -> 20.9 ms and
// the 4096 x 14336 column sweep 10.8 -> 8.0 ms; the factor's residual
// |U Hd U^T - I|_F / sqrt(K) 1.6e-6 -> 1.9e-6 (its distance to the fp64
// factor 1.0e-6 -> 1.5e-6).  Loads run two stages ahead (in two register
// sets; one stage ahead measured the same).  Tried and not kept: two LDS
// stage buffers with the split interleaved under the MFMAs, one workgroup
// per CU (21.9 ms); a start offset for every second workgroup (no change).

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float fl2 __attribute__((ext_vector_type(2)));

// (v0, v1) = hi + mid + lo exactly, each part a packed bf16 pair (element 0
// in the low half)
__device__ __forceinline__ void split3(float v0, float v1, uint32_t& h, uint32_t& m, uint32_t& l) {
  h = __builtin_bit_cast(uint32_t, __builtin_convertvector(fl2{v0, v1}, bf16x2));
  const float r0 = v0 - __uint_as_float(h << 16), r1 = v1 - __uint_as_float(h & 0xFFFF0000u);
  m = __builtin_bit_cast(uint32_t, __builtin_convertvector(fl2{r0, r1}, bf16x2));
  const float t0 = r0 - __uint_as_float(m << 16), t1 = r1 - __uint_as_float(m & 0xFFFF0000u);
  l = __builtin_bit_cast(uint32_t, __builtin_convertvector(fl2{t0, t1}, bf16x2));
}

template <int TR, int BK>
struct alignas(16) X3Planes {
  static constexpr int P = BK + 8;  // pitch in halves (80 bytes: rows stay 16-byte aligned)
  uint16_t v[3][TR * P];
};

// stage store of a [r][k] operand (load_op<..., false> order: float4 q of
// thread tid is row idx / (BK / 4), k (idx % (BK / 4)) * 4)
template <int TR, int BK, bool kFull>
__device__ __forceinline__ void store_x3(X3Planes<TR, BK>& s, int tid, f32x4 (&pre)[TR * BK / 4 / kThreads],
                                         uint32_t ok) {
  constexpr int NQ = TR * BK / 4 / kThreads;
  constexpr int P = X3Planes<TR, BK>::P;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int idx = q * kThreads + tid;
    const int r = idx / (BK / 4), k = (idx % (BK / 4)) * 4;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = kFull || ((ok >> (4 * q + e)) & 1u) ? pre[q][e] : 0.0f;
    uint32_t h[2], m[2], l[2];
    split3(v[0], v[1], h[0], m[0], l[0]);
    split3(v[2], v[3], h[1], m[1], l[1]);
    *reinterpret_cast<uint2*>(&s.v[0][r * P + k]) = uint2{h[0], h[1]};
    *reinterpret_cast<uint2*>(&s.v[1][r * P + k]) = uint2{m[0], m[1]};
    *reinterpret_cast<uint2*>(&s.v[2][r * P + k]) = uint2{l[0], l[1]};
  }
}

// a [k][j]-stored operand: thread tid owns j-quad jq = tid / (BK / KR) and
// the KR consecutive k-rows kg KR .. kg KR + KR - 1, kg = tid % (BK / KR)
// (KR = TR BK / (4 x 256) float4 loads, one per k-row); the 4 x KR block is
// written as 4 runs of KR halves per plane
template <int TR, int BK, bool kFull>
__device__ __forceinline__ void load_x3_trans(const Operand& o, int64_t r0, int64_t k0, int64_t Kd, int tid,
                                              f32x4 (&pre)[TR * BK / 4 / kThreads], uint32_t& ok) {
  constexpr int KR = TR * BK / 4 / kThreads;
  static_assert(KR == 2 || KR == 4, "4 x KR blocks");
  const int kg = tid % (BK / KR), jq = tid / (BK / KR);
  const int64_t r = r0 + 4 * jq;
  ok = 0;
#pragma unroll
  for (int e = 0; e < KR; ++e) {
    const int64_t k = k0 + kg * KR + e;
    const bool in = kFull || (r < o.rows && k < Kd);
    pre[e] = *reinterpret_cast<const f32x4*>(o.p + (in ? k * o.ld + r : 0));
    ok |= in ? 0xFu << (4 * e) : 0u;
  }
}

template <int TR, int BK, bool kFull>
__device__ __forceinline__ void store_x3_trans(X3Planes<TR, BK>& s, int tid, f32x4 (&pre)[TR * BK / 4 / kThreads],
                                               uint32_t ok) {
  constexpr int KR = TR * BK / 4 / kThreads;
  constexpr int P = X3Planes<TR, BK>::P;
  const int kg = tid % (BK / KR), jq = tid / (BK / KR);
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    float v[KR];
#pragma unroll
    for (int e = 0; e < KR; ++e) v[e] = kFull || ((ok >> (4 * e + jj)) & 1u) ? pre[e][jj] : 0.0f;
    uint32_t h[KR / 2], m[KR / 2], l[KR / 2];
#pragma unroll
    for (int e = 0; e < KR / 2; ++e) split3(v[2 * e], v[2 * e + 1], h[e], m[e], l[e]);
    const int at = (4 * jq + jj) * P + kg * KR;
    if constexpr (KR == 4) {
      *reinterpret_cast<uint2*>(&s.v[0][at]) = uint2{h[0], h[1]};
      *reinterpret_cast<uint2*>(&s.v[1][at]) = uint2{m[0], m[1]};
      *reinterpret_cast<uint2*>(&s.v[2][at]) = uint2{l[0], l[1]};
    } else {
      *reinterpret_cast<uint32_t*>(&s.v[0][at]) = h[0];
      *reinterpret_cast<uint32_t*>(&s.v[1][at]) = m[0];
      *reinterpret_cast<uint32_t*>(&s.v[2][at]) = l[0];
    }
  }
}

// load_op for a [r][k] operand with 16-byte rows; kFull: the stage lies
// inside the operand (no bounds checks)
template <int TR, int BK, bool kFull>
__device__ __forceinline__ void load_x3(const Operand& o, int64_t r0, int64_t k0, int64_t Kd, int tid,
                                        f32x4 (&pre)[TR * BK / 4 / kThreads], uint32_t& ok) {
  if constexpr (!kFull) {
    load_op<TR, BK, true, false>(o, r0, k0, Kd, tid, pre, ok);
  } else {
    constexpr int NQ = TR * BK / 4 / kThreads;
    ok = ~0u;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int idx = q * kThreads + tid;
      pre[q] = *reinterpret_cast<const f32x4*>(o.p + (r0 + idx / (BK / 4)) * o.ld + k0 + (idx % (BK / 4)) * 4);
    }
  }
}

template <int TM, int TN, int BK>
struct alignas(16) X3Smem {
  X3Planes<TM, BK> a;
  X3Planes<TN, BK> b;
};

// C tile (i0, j0) of d from the waves' 32x32 accumulators (the fp32
// kernel's epilogue)
template <int FM, int FN>
__device__ __forceinline__ void x3_epilogue(const GemmDesc& d, int64_t i0, int64_t j0, int wm, int wn, int lane,
                                            f32x16 (&acc)[FM][FN]) {
  const int64_t M = d.M, N = d.N, ldc = d.ldc;
  const float alpha = d.alpha, beta = d.beta;
  float* __restrict__ C = d.C;
  const bool lower = (d.flags & GEMM_C_LOWER) != 0;
  const int64_t rbase = i0 + wm + 4 * (lane >> 5);
  const int64_t cbase = j0 + wn + (lane & 31);
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t col = cbase + j * 32;
      float* cp = C + (rbase + i * 32) * ldc + col;
      float cv[16];
      if (beta != 0.0f) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t row = rbase + i * 32 + 8 * (v >> 2) + (v & 3);
          cv[v] = *((row < M && col < N) ? cp + (8 * (v >> 2) + (v & 3)) * ldc : C);
        }
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = rbase + i * 32 + 8 * (v >> 2) + (v & 3);
        if (row < M && col < N && (!lower || row >= col)) {
          float r = alpha * acc[i][j][v];
          if (beta != 0.0f) r += beta * cv[v];
          cp[(8 * (v >> 2) + (v & 3)) * ldc] = r;
        }
      }
    }
}

// output tile `bid` of d on the split-bf16 MFMAs (A [i][k] with 16-byte
// rows, as kVec; B as kTB)
template <int TM, int TN, int BK, bool kTB>
__device__ __forceinline__ void gemm_tile_x3(const GemmDesc& d, int bid, X3Smem<TM, TN, BK>& sm) {
  constexpr int FM = TM / 64, FN = TN / 64;  // 32x32 blocks per wave
  constexpr int QA = TM * BK / 4 / kThreads, QB = TN * BK / 4 / kThreads;
  constexpr int P = BK + 8;
  const int64_t Kd = d.Kd;
  const int flags = d.flags;
  int tm = 0, tn = 0;
  tile_of<TM, TN>(bid, d.tiles_m, d.tiles_n, d.order, tm, tn);
  const int64_t i0 = static_cast<int64_t>(tm) * TM;
  const int64_t j0 = static_cast<int64_t>(tn) * TN;
  if ((flags & GEMM_C_LOWER) && j0 > i0 + TM - 1) return;

  int64_t kb = 0, ke = Kd;
  if (flags & GEMM_KLIM_A_LE_I) ke = std::min<int64_t>(ke, i0 + TM);
  if (flags & GEMM_KLIM_B_LE_J) ke = std::min<int64_t>(ke, j0 + TN);
  if (flags & GEMM_KLIM_A_GE_I) kb = std::max<int64_t>(kb, i0);
  if (flags & GEMM_KLIM_B_GE_J) kb = std::max<int64_t>(kb, j0);
  kb = (kb / BK) * BK;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 1) * (TM / 2);
  const int wn = (wave & 1) * (TN / 2);

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // two register sets: stage s is loaded into set s % 2 two stages before
  // it is stored
  f32x4 pa[2][QA], pb[2][QB];
  uint32_t oka[2] = {0, 0}, okb[2] = {0, 0};
  // a stage inside both operands (every stage of an interior tile) skips
  // the bounds checks of its loads and stores (a wave-uniform branch)
  const bool rows_in = i0 + TM <= d.a.rows && j0 + TN <= d.b.rows;
  auto load = [&](int64_t k0, int set) {
    auto go = [&](auto full) {
      constexpr bool F = decltype(full)::value;
      load_x3<TM, BK, F>(d.a, i0, k0, Kd, tid, pa[set], oka[set]);
      if constexpr (kTB) load_x3_trans<TN, BK, F>(d.b, j0, k0, Kd, tid, pb[set], okb[set]);
      else load_x3<TN, BK, F>(d.b, j0, k0, Kd, tid, pb[set], okb[set]);
    };
    if (rows_in && k0 + BK <= Kd) go(std::true_type{});
    else go(std::false_type{});
  };
  auto stage = [&](int64_t k0, int set) {
    __syncthreads();
    auto put = [&](auto full) {
      constexpr bool F = decltype(full)::value;
      store_x3<TM, BK, F>(sm.a, tid, pa[set], oka[set]);
      if constexpr (kTB) store_x3_trans<TN, BK, F>(sm.b, tid, pb[set], okb[set]);
      else store_x3<TN, BK, F>(sm.b, tid, pb[set], okb[set]);
    };
    if (rows_in && k0 + BK <= Kd) put(std::true_type{});
    else put(std::false_type{});
    __syncthreads();
    if (k0 + 2 * BK < ke) load(k0 + 2 * BK, set);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int ko = ks * 16 + 8 * (lane >> 5);
      uint4 fa[3][FM], fb[3][FN];
#pragma unroll
      for (int p = 0; p < 3; ++p) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
          fa[p][i] = *reinterpret_cast<const uint4*>(&sm.a.v[p][(wm + i * 32 + (lane & 31)) * P + ko]);
#pragma unroll
        for (int j = 0; j < FN; ++j)
          fb[p][j] = *reinterpret_cast<const uint4*>(&sm.b.v[p][(wn + j * 32 + (lane & 31)) * P + ko]);
      }
      // smallest products first; the FM x FN blocks of one product are
      // independent, so consecutive MFMAs never wait for each other
      constexpr int kPa[6] = {2, 0, 1, 1, 0, 0}, kPb[6] = {0, 2, 1, 0, 1, 0};
#pragma unroll
      for (int t = 0; t < 6; ++t)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fa[kPa[t]][i]),
                                                                __builtin_bit_cast(bf16x8, fb[kPb[t]][j]),
                                                                acc[i][j], 0, 0, 0);
    }
  };
  if (kb < ke) load(kb, 0);
  if (kb + BK < ke) load(kb + BK, 1);
  // stages in pairs, so that each set index is a constant
  for (int64_t k0 = kb; k0 < ke; k0 += 2 * BK) {
    stage(k0, 0);
    if (k0 + BK < ke) stage(k0 + BK, 1);
  }

  x3_epilogue<FM, FN>(d, i0, j0, wm, wn, lane, acc);
}

// (two workgroups per CU: one's staging overlaps the other's MFMAs)
template <int TM, int TN, int BK, bool kTB>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void gemm_x3_kernel(GemmDesc d) {
  __shared__ X3Smem<TM, TN, BK> sm;
  gemm_tile_x3<TM, TN, BK, kTB>(d, static_cast<int>(blockIdx.x), sm);
}

template <int TM, int TN, int BK, bool kTB0, bool kTB1>
__global__ __launch_bounds__(kThreads) void gemm_x3_pair_kernel(GemmDesc d0, GemmDesc d1, int split) {
  __shared__ X3Smem<TM, TN, BK> sm;
  const int bid = static_cast<int>(blockIdx.x);
  if (bid < split) gemm_tile_x3<TM, TN, BK, kTB0>(d0, bid, sm);
  else gemm_tile_x3<TM, TN, BK, kTB1>(d1, bid - split, sm);
}

template <int TM, int TN, int BK, bool kVec, bool kTA, bool kTB>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(GemmDesc d) {
  __shared__ float sA[TM * (BK + 2)];
  __shared__ float sB[TN * (BK + 2)];
  gemm_tile<TM, TN, BK, kVec, kTA, kTB>(d, static_cast<int>(blockIdx.x), sA, sB);
}

// two independent products in one grid (16-byte operands, opA not
// transposed): workgroups [0, split) take tiles of d0, the rest tiles of d1
template <int TM, int TN, int BK, bool kTB0, bool kTB1>
__global__ __launch_bounds__(kThreads) void gemm_f32_pair_kernel(GemmDesc d0, GemmDesc d1, int split) {
  __shared__ float sA[TM * (BK + 2)];
  __shared__ float sB[TN * (BK + 2)];
  const int bid = static_cast<int>(blockIdx.x);
  if (bid < split) gemm_tile<TM, TN, BK, true, false, kTB0>(d0, bid, sA, sB);
  else gemm_tile<TM, TN, BK, true, false, kTB1>(d1, bid - split, sA, sB);
}

struct GemmArgs {
  int64_t M, N, Kd;
  float alpha;
  Operand a, b;
  float beta;
  float* C;
  int64_t ldc;
  int flags;
};

// the tile grid of g in TM x TN tiles and its dispatch order; returns the
// number of workgroups
template <int TM, int TN>
int64_t describe(const GemmArgs& g, GemmDesc& d) {
  const int tiles_m = static_cast<int>(cdiv(g.M, TM));
  const int tiles_n = static_cast<int>(cdiv(g.N, TN));
  int64_t tiles = static_cast<int64_t>(tiles_m) * tiles_n;
  int order = ORDER_ROWS;
  switch (g.flags) {
    case GEMM_KLIM_A_LE_I: order = ORDER_ROWS_DESC; break;
    case GEMM_KLIM_B_LE_J: order = ORDER_COLS_DESC; break;
    case GEMM_KLIM_B_GE_J: order = ORDER_COLS; break;
    case GEMM_C_LOWER:
      // square C whose tile rows hold exactly c (r + 1) tiles
      if (g.M == g.N && (TM / TN) * tiles_m == tiles_n) {
        order = ORDER_LOWER;
        tiles = static_cast<int64_t>(TM / TN) * tiles_m * (tiles_m + 1) / 2;
      }
      break;
    default: break;
  }
  d = GemmDesc{g.M, g.N, g.Kd, g.alpha, g.a, g.b, g.beta, g.C, g.ldc, g.flags, tiles_m, tiles_n, order};
  return tiles;
}

template <int TM, int TN, bool V, bool TA, bool TB>
void launch_one(hipStream_t st, const GemmArgs& g) {
  GemmDesc d;
  const int64_t tiles = describe<TM, TN>(g, d);
  hipLaunchKernelGGL((gemm_f32_kernel<TM, TN, 32, V, TA, TB>), dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0,
                     st, d);
}

// transposition and vector width are compile-time in the kernel
template <int TM, int TN, bool V>
void launch_trans(hipStream_t st, const GemmArgs& g) {
  if (!g.a.trans && !g.b.trans) launch_one<TM, TN, V, false, false>(st, g);
  else if (!g.a.trans) launch_one<TM, TN, V, false, true>(st, g);
  else if (!g.b.trans) launch_one<TM, TN, V, true, false>(st, g);
  else launch_one<TM, TN, V, true, true>(st, g);
}

template <int TM, int TN>
int launch_tiles(hipStream_t st, const GemmArgs& g, bool vec) {
  if (vec) launch_trans<TM, TN, true>(st, g);
  else launch_trans<TM, TN, false>(st, g);
  return check_launch("gemm_f32");
}

// every float4 of the operand is entirely inside or outside it
inline bool vec_ok(const Operand& o, int64_t Kd) {
  return o.ld % 4 == 0 && (reinterpret_cast<uintptr_t>(o.p) % 16) == 0 && (o.trans ? o.rows : Kd) % 4 == 0;
}

GemmArgs make_args(const GemmCall& c) {
  return GemmArgs{c.M, c.N, c.Kd, c.alpha, Operand{c.A, c.lda, c.transA, c.M},
                  Operand{c.B, c.ldb, !c.transB, c.N},  // B viewed as [j][k]
                  c.beta, c.C, c.ldc, c.flags};
}

// 64 x 64 tiles below 4096 tiles of 128 x 64 (measured on MI355X: the four
// triangular products at 3584^3 1.96 -> 1.76 ms, at 1792^3 0.42 -> 0.34 ms;
// at 7168^3 128 x 64 stays faster, 12.8 against 13.3 ms)
inline bool small_tiles(const GemmArgs& g) { return cdiv(g.M, 128) * cdiv(g.N, 64) < 4096; }

// the split-bf16 kernels take every product with 16-byte operand rows and
// A not transposed (all of the factorisation's and the sweep's): 128 x 128
// tiles from 512 of them, else 64 x 64 (measured on MI355X, the K = 14336
// factorisation with the threshold at 128 / 256 / 512 / 1024 / 2048 tiles:
// 23.1 / 22.0 / 21.9 / 22.5 / 22.6 ms)
constexpr int64_t kX3BigTiles = 512;
inline bool x3_ok(const GemmArgs& g, bool vec) { return vec && !g.a.trans; }
inline bool x3_big(const GemmArgs& g) { return cdiv(g.M, 128) * cdiv(g.N, 128) >= kX3BigTiles; }

template <int TM, int TN>
void launch_x3_tiles(hipStream_t st, const GemmArgs& g) {
  GemmDesc d;
  const int64_t tiles = describe<TM, TN>(g, d);
  const dim3 grid(static_cast<unsigned>(tiles));
  if (g.b.trans) hipLaunchKernelGGL((gemm_x3_kernel<TM, TN, 32, true>), grid, dim3(kThreads), 0, st, d);
  else hipLaunchKernelGGL((gemm_x3_kernel<TM, TN, 32, false>), grid, dim3(kThreads), 0, st, d);
}

int launch_args(hipStream_t st, const GemmArgs& g) {
  if (g.M <= 0 || g.N <= 0) return GPTQ_OK;
  const bool vec = vec_ok(g.a, g.Kd) && vec_ok(g.b, g.Kd);
  if (x3_ok(g, vec)) {
    if (x3_big(g)) launch_x3_tiles<128, 128>(st, g);
    else launch_x3_tiles<64, 64>(st, g);
    return check_launch("gemm_x3");
  }
  if (small_tiles(g)) return launch_tiles<64, 64>(st, g, vec);
  return launch_tiles<128, 64>(st, g, vec);
}

template <bool TB0, bool TB1>
void launch_pair(hipStream_t st, const GemmDesc& d0, int64_t t0, const GemmDesc& d1, int64_t t1) {
  hipLaunchKernelGGL((gemm_f32_pair_kernel<64, 64, 32, TB0, TB1>), dim3(static_cast<unsigned>(t0 + t1)),
                     dim3(kThreads), 0, st, d0, d1, static_cast<int>(t0));
}

}  // namespace

int launch_gemm_f32(hipStream_t st, int64_t M, int64_t N, int64_t Kd, float alpha, const float* A, int64_t lda,
                    bool transA, const float* B, int64_t ldb, bool transB, float beta, float* C, int64_t ldc,
                    int flags) {
  return launch_args(st, make_args(GemmCall{M, N, Kd, alpha, A, lda, transA, B, ldb, transB, beta, C, ldc, flags}));
}

template <bool TB0, bool TB1>
void launch_x3_pair(hipStream_t st, const GemmDesc& d0, int64_t t0, const GemmDesc& d1, int64_t t1) {
  hipLaunchKernelGGL((gemm_x3_pair_kernel<64, 64, 32, TB0, TB1>), dim3(static_cast<unsigned>(t0 + t1)),
                     dim3(kThreads), 0, st, d0, d1, static_cast<int>(t0));
}

int launch_gemm_f32_pair(hipStream_t st, const GemmCall& p, const GemmCall& q) {
  const GemmArgs g0 = make_args(p), g1 = make_args(q);
  const bool vec = vec_ok(g0.a, g0.Kd) && vec_ok(g0.b, g0.Kd) && vec_ok(g1.a, g1.Kd) && vec_ok(g1.b, g1.Kd);
  const bool nonempty = g0.M > 0 && g0.N > 0 && g1.M > 0 && g1.N > 0;
  if (nonempty && x3_ok(g0, vec) && x3_ok(g1, vec)) {
    if (x3_big(g0) || x3_big(g1)) {
      const int rc = launch_args(st, g0);
      return rc ? rc : launch_args(st, g1);
    }
    GemmDesc d0, d1;
    const int64_t t0 = describe<64, 64>(g0, d0), t1 = describe<64, 64>(g1, d1);
    if (!g0.b.trans && !g1.b.trans) launch_x3_pair<false, false>(st, d0, t0, d1, t1);
    else if (!g0.b.trans) launch_x3_pair<false, true>(st, d0, t0, d1, t1);
    else if (!g1.b.trans) launch_x3_pair<true, false>(st, d0, t0, d1, t1);
    else launch_x3_pair<true, true>(st, d0, t0, d1, t1);
    return check_launch("gemm_x3_pair");
  }
  const bool pair = nonempty && small_tiles(g0) && small_tiles(g1) && !g0.a.trans && !g1.a.trans && vec;
  if (!pair) {
    const int rc = launch_args(st, g0);
    return rc ? rc : launch_args(st, g1);
  }
  GemmDesc d0, d1;
  const int64_t t0 = describe<64, 64>(g0, d0), t1 = describe<64, 64>(g1, d1);
  if (!g0.b.trans && !g1.b.trans) launch_pair<false, false>(st, d0, t0, d1, t1);
  else if (!g0.b.trans) launch_pair<false, true>(st, d0, t0, d1, t1);
  else if (!g1.b.trans) launch_pair<true, false>(st, d0, t0, d1, t1);
  else launch_pair<true, true>(st, d0, t0, d1, t1);
  return check_launch("gemm_f32_pair");
}

}  // namespace gptq
