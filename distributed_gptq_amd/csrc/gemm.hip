// fp32 GEMM on v_mfma_f32_32x32x2_f32 (gfx950).
//
// TM x TN output tile per workgroup of 4 waves (2 x 2, each TM/2 x TN/2 =
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

int launch_args(hipStream_t st, const GemmArgs& g) {
  if (g.M <= 0 || g.N <= 0) return GPTQ_OK;
  const bool vec = vec_ok(g.a, g.Kd) && vec_ok(g.b, g.Kd);
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

int launch_gemm_f32_pair(hipStream_t st, const GemmCall& p, const GemmCall& q) {
  const GemmArgs g0 = make_args(p), g1 = make_args(q);
  const bool pair = g0.M > 0 && g0.N > 0 && g1.M > 0 && g1.N > 0 && small_tiles(g0) && small_tiles(g1) &&
                    !g0.a.trans && !g1.a.trans && vec_ok(g0.a, g0.Kd) && vec_ok(g0.b, g0.Kd) &&
                    vec_ok(g1.a, g1.Kd) && vec_ok(g1.b, g1.Kd);
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
