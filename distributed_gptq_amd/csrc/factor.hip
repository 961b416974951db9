// Damping + Cholesky-based inverse factors of the Hessian, fp32, on gfx950.
//
// Both outputs come from one factorisation of the reversed matrix
// A = J Hd J (J = index reversal):  A = L L^T,  X = L^-1.  Then
//   U  = J X J  is upper triangular with positive diagonal and U^T U = Hd^-1
//        (canonical GPTQ's chol(cholesky_inverse(chol(H)), upper=True)),
//   Hd^-1 = J (X^T X) J  (the reference's cholesky_inverse(cholesky(H))).
//
// L and X are built together by recursion on halves,
//   [A11    ]    L11 = chol(A11), X11 = L11^-1           (recursion)
//   [A21 A22]    L21 = A21 X11^T                        (GEMM)
//                S   = A22 - L21 L21^T                   (GEMM, lower only)
//                L22 = chol(S),  X22 = L22^-1            (recursion)
//                X21 = -X22 (L21 X11)                    (2 GEMMs)
// so that almost all of the 2K^3/3 flops run in large fp32-MFMA GEMMs; the
// 128 x 128 leaves are factorised and inverted by one workgroup.
#include "gemm.hpp"

namespace gptq {
namespace {

constexpr int kNB = 128;  // leaf size (one workgroup, registers + LDS)

// mean of the (possibly dead-fixed) scaled diagonal -> lambda; dead flags
__global__ __launch_bounds__(1024) void diag_stats(const float* __restrict__ H, int64_t K, float scale,
                                                   float percdamp, int32_t* __restrict__ dead,
                                                   float* __restrict__ lam, int32_t* __restrict__ info) {
  __shared__ double red[1024];
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < K; i += blockDim.x) {
    float d = scale * H[i * K + i];
    if (dead) {
      const bool is_dead = (d == 0.0f);
      dead[i] = is_dead ? 1 : 0;
      if (is_dead) d = 1.0f;
    }
    acc += d;
  }
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int s = blockDim.x / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    lam[0] = percdamp * static_cast<float>(red[0] / static_cast<double>(K));
    info[0] = 0;
  }
}

// value of the damped (permuted) matrix at sweep-order position (a, b)
__device__ __forceinline__ float damped(const float* H, int64_t K, float scale, const int32_t* perm, bool fix_dead,
                                        float lam, int64_t a, int64_t b) {
  const int64_t pa = perm ? perm[a] : a;
  const int64_t pb = perm ? perm[b] : b;
  float v = scale * H[pa * K + pb];
  if (a == b) {
    if (fix_dead && v == 0.0f) v = 1.0f;
    v += lam;
  }
  return v;
}

// A[i][j] = Hd[K-1-i][K-1-j] for i >= j (upper part of A untouched);
// Hd (optional, full) in sweep order.
__global__ void build_A(const float* __restrict__ H, int64_t K, float scale, const int32_t* __restrict__ perm,
                        int fix_dead, const float* __restrict__ lam, float* __restrict__ A,
                        float* __restrict__ Hd) {
  // rows over blockIdx.y, columns over threads: no 64-bit division per element
  const float l = lam[0];
  for (int64_t i = blockIdx.y; i < K; i += gridDim.y)
    for (int64_t j = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; j < K;
         j += static_cast<int64_t>(gridDim.x) * blockDim.x) {
      const int64_t idx = i * K + j;
      if (Hd) Hd[idx] = damped(H, K, scale, perm, fix_dead != 0, l, i, j);
      if (i >= j) A[idx] = damped(H, K, scale, perm, fix_dead != 0, l, K - 1 - i, K - 1 - j);
    }
}

// build_A without Hd, for K <= kRowLdsMax: one workgroup per row i of A
// stages its source row (H's row perm[K-1-i]) in LDS with 16-byte loads and
// gathers A[i][0..i] from there (coalesced writes), instead of gathering every
// element from global memory.  Same arithmetic as build_A.
constexpr int64_t kRowLdsMax = 32768;

__global__ __launch_bounds__(512) void build_A_rows(const float* __restrict__ H, int64_t K, float scale,
                                                    const int32_t* __restrict__ perm, int fix_dead,
                                                    const float* __restrict__ lam, int vec, float* __restrict__ A) {
  extern __shared__ __attribute__((aligned(16))) float shrow[];
  const float l = lam[0];
  const int k = static_cast<int>(K);
  for (int64_t i = blockIdx.x; i < K; i += gridDim.x) {
    const int64_t a = K - 1 - i;
    const float* src = H + (perm ? perm[a] : a) * K;
    if (vec) {
      for (int c = 4 * threadIdx.x; c < k; c += 4 * blockDim.x)
        *reinterpret_cast<f32x4*>(shrow + c) = *reinterpret_cast<const f32x4*>(src + c);
    } else {
      for (int c = threadIdx.x; c < k; c += blockDim.x) shrow[c] = src[c];
    }
    __syncthreads();
    float* dst = A + i * K;
    for (int j = threadIdx.x; j <= i; j += blockDim.x) {
      const int b = k - 1 - j;
      float v = scale * shrow[perm ? perm[b] : b];
      if (j == i) {
        if (fix_dead && v == 0.0f) v = 1.0f;
        v += l;
      }
      dst[j] = v;
    }
    __syncthreads();
  }
}

__global__ void fill_zero(float* __restrict__ p, int64_t n) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = 0.0f;
}

// One workgroup of 4 waves: Cholesky of the m x m (m <= 128) diagonal block
// of A at (n0, n0) and the inverse of its factor, blocked by 32:
//   for each diagonal block k:  one wave factors D_kk = L_kk L_kk^T and
//     inverts L_kk (X_kk) together (diag32) while the others form
//     S_kj = sum_{i=j}^{k-1} L_ki X_ij for X's row block k; then
//     X_kj = -X_kk S_kj and the panel L_ik = A_ik X_kk^T, then
//     A_ij -= L_ik L_jk^T (trailing), as 32x32x32 v_mfma_f32_32x32x2f32
//     products, one per wave.
// The tile is padded to 128 with the identity.  Writes X = L^-1 (zeros
// above) into X (A's block is left as scratch); a non-positive pivot records
// info = 1 + (column in A order) once.
constexpr int kLP = kNB + 1;  // LDS pitch (odd: conflict-free column reads)
constexpr int kLB = 32;       // diagonal block
constexpr size_t kLeafLds = sizeof(float) * (2 * kNB * kLP + 4 * kLB * (kLB + 1));

__device__ __forceinline__ float rdl(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// acc += P (32 x 32 at pa, rows r, k) x Q' where Q' = Q^T (Q[c][k] at pb) when
// bT, else Q (Q[k][c] at pb); one wave, 16 steps of v_mfma_f32_32x32x2f32
// (lane l: operand row/column l % 32, k = 2 s + l / 32)
__device__ __forceinline__ f32x16 mm32(const float* pa, int lda, const float* pb, int ldb, bool bT, f32x16 acc,
                                      int lane) {
  const int i = lane & 31, h = lane >> 5;
#pragma unroll
  for (int st = 0; st < 16; ++st) {
    const int k = 2 * st + h;
    const float x = pa[i * lda + k];
    const float y = bT ? pb[i * ldb + k] : pb[k * ldb + i];
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, acc, 0, 0, 0);
  }
  return acc;
}

// 32x32 accumulator layout: lane l, register v -> row 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32
__device__ __forceinline__ void put32(float* pc, int ldc, const f32x16& acc, float scale, int lane) {
#pragma unroll
  for (int v = 0; v < 16; ++v) pc[(8 * (v >> 2) + 4 * (lane >> 5) + (v & 3)) * ldc + (lane & 31)] = scale * acc[v];
}

__device__ __forceinline__ float bperm(int src_lane, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src_lane * 4, __builtin_bit_cast(int, v)));
}

// One wave: D (B x B at sD, lower part; B = 16 or 32) = L L^T and X = L^-1,
// written back over D and into sXd (zeros above).  Lane l holds the S x S
// sub-block (S = B / 8; rows S (l / 8) + u, columns S (l % 8) + v) of the
// working matrix and of Y (initially I).  Step j: the pivot comes from its
// lane (v_readlane); the lanes holding column j have L's column j, the lanes
// holding row j have Y's row j scaled by 1 / L[j][j]; every lane fetches the
// pieces it needs from them with ds_bpermute and applies the two rank-1
// updates
//   D[r][c] -= L[r][j] L[c][j]  (c > j),   Y[r][c] -= L[r][j] Y[j][c]  (r > j),
// right-looking Cholesky and forward elimination fused.  The leaf uses B = 16
// (diag32 below joins two such chains); one B = 32 chain took about 600 cycles
// a column step, and exchanging through LDS instead, or blocking by 4 columns
// (one exchange and a rank-4 update per 4 columns, same results bit for bit),
// measured no faster.
template <int B>
__device__ __forceinline__ void diag_blk(float* sD, float* sXd, int lane, int col0, int lim, int& first_bad) {
  constexpr int S = B / 8;
  const int ra = lane >> 3, cb = lane & 7;
  float a[S][S], y[S][S];
#pragma unroll
  for (int u = 0; u < S; ++u)
#pragma unroll
    for (int v = 0; v < S; ++v) {
      a[u][v] = sD[(S * ra + u) * kLP + S * cb + v];
      y[u][v] = (S * ra + u == S * cb + v) ? 1.0f : 0.0f;
    }
#pragma unroll
  for (int j = 0; j < B; ++j) {
    const int jb = j / S, jv = j % S;
    const float piv = rdl(a[jv][jv], jb * 8 + jb);
    if (!(piv > 0.0f) && first_bad < 0 && col0 + j < lim) first_bad = col0 + j;
    // hardware square root and reciprocal (1 ulp): they sit on the
    // sequential chain of the B steps
    const float d = __builtin_amdgcn_sqrtf(piv);
    const float id = __builtin_amdgcn_rcpf(d);
    // column j of L for rows S ra + u (kept by the lanes with cb == jb) and
    // row j of Y for columns S cb + v (kept by the lanes with ra == jb);
    // every lane computes them, the owners' values are broadcast with
    // ds_bpermute (no LDS round trip or wave barrier on the chain)
    float lv[S], yv[S];
#pragma unroll
    for (int u = 0; u < S; ++u) {
      const int r = S * ra + u;
      lv[u] = r > j ? a[u][jv] * id : (r == j ? d : 0.0f);
      if (cb == jb) a[u][jv] = lv[u];
    }
#pragma unroll
    for (int v = 0; v < S; ++v) {
      yv[v] = y[jv][v] * id;
      if (ra == jb) y[jv][v] = yv[v];
    }
    float lr[S], lc[S], yc[S];
#pragma unroll
    for (int u = 0; u < S; ++u) {
      lr[u] = bperm(8 * ra + jb, lv[u]);  // L[S ra + u][j]
      lc[u] = bperm(8 * cb + jb, lv[u]);  // L[S cb + u][j]
      yc[u] = bperm(8 * jb + cb, yv[u]);  // Y[j][S cb + u]
    }
#pragma unroll
    for (int u = 0; u < S; ++u) {
      const float lru = S * ra + u > j ? lr[u] : 0.0f;
#pragma unroll
      for (int v = 0; v < S; ++v) {
        a[u][v] = fmaf(-lr[u], S * cb + v > j ? lc[v] : 0.0f, a[u][v]);
        y[u][v] = fmaf(-lru, yc[v], y[u][v]);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < S; ++u)
#pragma unroll
    for (int v = 0; v < S; ++v) {
      const bool low = S * ra + u >= S * cb + v;
      sD[(S * ra + u) * kLP + S * cb + v] = low ? a[u][v] : 0.0f;
      sXd[(S * ra + u) * kLP + S * cb + v] = low ? y[u][v] : 0.0f;
    }
}

// acc += P (16 x 16 at pa, P[r][k] = pa[r * lda + k]) x Q', Q' = Q^T
// (pb[c * ldb + k]) when bT, else Q (pb[k * ldb + c]); one wave, 4 steps of
// v_mfma_f32_16x16x4f32 (lane l: operand row/column l % 16, k = 4 s + l / 16)
__device__ __forceinline__ f32x4 mm16(const float* pa, int lda, const float* pb, int ldb, bool bT, f32x4 acc,
                                     int lane) {
  const int i = lane & 15, h = lane >> 4;
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    const int k = 4 * st + h;
    const float x = pa[i * lda + k];
    const float y = bT ? pb[i * ldb + k] : pb[k * ldb + i];
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x, y, acc, 0, 0, 0);
  }
  return acc;
}

// 16x16 accumulator layout: lane l, register v -> row 4 (l / 16) + v, column l % 16
__device__ __forceinline__ int acc16_at(int lane, int v, int ld) { return (4 * (lane >> 4) + v) * ld + (lane & 15); }

// One wave: the 32 x 32 diagonal block at sD (lower part) = L L^T and
// X = L^-1 into sXd (zeros above), by halves:
//   L11, Y11 = diag(D11);  L21 = D21 Y11^T;  S = D22 - L21 L21^T;
//   L22, Y22 = diag(S);    Y21 = -Y22 (L21 Y11)
// Two 16-column chains take about half the time of one 32-column chain
// (a 16-column step exchanges and updates a quarter of the elements); the
// three products are v_mfma_f32_16x16x4f32.  sT: 16 x 17 floats of scratch.
// The upper 16 x 16 quarter of D is left as it is (the leaf does not read L's
// diagonal blocks again); that of sXd is never written and stays zero.
__device__ __forceinline__ void diag32(float* sD, float* sXd, float* sT, int lane, int col0, int lim,
                                       int& first_bad) {
  constexpr int H = 16;
  float* D21 = sD + H * kLP;
  float* D22 = D21 + H;
  float* Y21 = sXd + H * kLP;
  float* Y22 = Y21 + H;
  diag_blk<H>(sD, sXd, lane, col0, lim, first_bad);
  f32x4 l21 = {};
  l21 = mm16(D21, kLP, sXd, kLP, true, l21, lane);
#pragma unroll
  for (int v = 0; v < 4; ++v) D21[acc16_at(lane, v, kLP)] = l21[v];
  f32x4 s = {};
  s = mm16(D21, kLP, D21, kLP, true, s, lane);
#pragma unroll
  for (int v = 0; v < 4; ++v) D22[acc16_at(lane, v, kLP)] -= s[v];
  diag_blk<H>(D22, Y22, lane, col0 + H, lim, first_bad);
  f32x4 t = {};
  t = mm16(D21, kLP, sXd, kLP, false, t, lane);
#pragma unroll
  for (int v = 0; v < 4; ++v) sT[acc16_at(lane, v, H + 1)] = t[v];
  f32x4 y21 = {};
  y21 = mm16(Y22, kLP, sT, H + 1, false, y21, lane);
#pragma unroll
  for (int v = 0; v < 4; ++v) Y21[acc16_at(lane, v, kLP)] = -y21[v];
}

__global__ __launch_bounds__(256) void chol_inv_leaf(float* __restrict__ A, float* __restrict__ X, int64_t ld,
                                                     int64_t n0, int m, int32_t* __restrict__ info) {
  extern __shared__ float lds[];
  float* sA = lds;                      // [128][kLP]: A, then L
  float* sX = lds + kNB * kLP;          // [128][kLP]: X
  float* sS = sX + kNB * kLP;           // [wave][32][33]: partial sums of the inverse
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  constexpr int NB = kNB / kLB;
  static_assert(NB == 4, "waves 1..3 form the sums of row blocks 1..3, and each phase has NB - 1 blocks");

  // load the lower triangle (identity padding beyond m), 32 loads in flight per thread
  for (int e0 = tid; e0 < kNB * kNB; e0 += 256 * 32) {
    float v[32];
    // unconditional loads (clamped into the block), selected afterwards; the
    // scheduling barrier keeps every select after the last load (placed next
    // to its load, each select made the wave wait for that load before
    // issuing the next)
#pragma unroll
    for (int u = 0; u < 32; ++u) {
      const int e = e0 + u * 256;
      const int rr = e >> 7, cc = e & (kNB - 1);
      v[u] = A[(n0 + min(rr, m - 1)) * ld + n0 + min(cc, m - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 32; ++u) {
      const int e = e0 + u * 256;
      const int rr = e >> 7, cc = e & (kNB - 1);
      v[u] = (rr < m && cc < m && cc <= rr) ? v[u] : (rr == cc ? 1.0f : 0.0f);
    }
#pragma unroll
    for (int u = 0; u < 32; ++u) {
      const int e = e0 + u * 256;
      sA[(e >> 7) * kLP + (e & (kNB - 1))] = v[u];
      sX[(e >> 7) * kLP + (e & (kNB - 1))] = 0.0f;
    }
  }
  __syncthreads();

  int first_bad = -1;
  auto blk = [&](float* base, int bi, int bj) { return base + bi * kLB * kLP + bj * kLB; };
  // Row block kb of X off the diagonal, X_kj = -X_kk S_kj with
  // S_kj = sum_{i=j}^{k-1} L_ki X_ij (j < k), is built in the same loop: waves
  // 1..kb form S_kb,j (j = wave - 1, into their sS slots) while wave 0 factors
  // block kb, and the products by X_kk share the panel phase (waves j < kb
  // take X_kb,j, the others the panel blocks), so no pass follows the loop.
  for (int kb = 0; kb < NB; ++kb) {
    if (wave == 0) {
      diag32(blk(sA, kb, kb), blk(sX, kb, kb), sS, lane, kb * kLB, m, first_bad);
    } else if (wave - 1 < kb) {
      const int jb = wave - 1;
      f32x16 acc = {};
      for (int k = jb; k < kb; ++k) acc = mm32(blk(sA, kb, k), kLP, blk(sX, k, jb), kLP, false, acc, lane);
      put32(sS + wave * kLB * (kLB + 1), kLB + 1, acc, 1.0f, lane);
    }
    __syncthreads();
    // NB - 1 blocks per phase, one per wave: X_kb,j = -X_kk S_kb,j for
    // j = wave < kb, then the panel L_ib,kb = A_ib,kb X_kk^T for ib = wave + 1 > kb
    if (wave < NB - 1) {
      f32x16 acc = {};
      if (wave < kb) {
        acc = mm32(blk(sX, kb, kb), kLP, sS + (wave + 1) * kLB * (kLB + 1), kLB + 1, false, acc, lane);
        put32(blk(sX, kb, wave), kLP, acc, -1.0f, lane);
      } else {
        acc = mm32(blk(sA, wave + 1, kb), kLP, blk(sX, kb, kb), kLP, true, acc, lane);
        put32(blk(sA, wave + 1, kb), kLP, acc, 1.0f, lane);
      }
    }
    __syncthreads();
    // trailing: A_ij -= L_ik L_jk^T for kb < j <= i
    {
      int t = 0;
      for (int ib = kb + 1; ib < NB; ++ib)
        for (int jb = kb + 1; jb <= ib; ++jb, ++t) {
          if ((t & 3) != wave) continue;
          f32x16 acc = {};
          acc = mm32(blk(sA, ib, kb), kLP, blk(sA, jb, kb), kLP, true, acc, lane);
          float* pc = blk(sA, ib, jb);
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            float& c = pc[(8 * (v >> 2) + 4 * (lane >> 5) + (v & 3)) * kLP + (lane & 31)];
            c -= acc[v];
          }
        }
    }
    __syncthreads();
  }
  if (first_bad >= 0 && tid == 0) atomicCAS(info, 0, static_cast<int32_t>(n0 + first_bad + 1));
  // write back X (lower, zeros above) for the m x m block; L itself is not
  // needed beyond the leaf (the products above it take X)
#pragma unroll 8
  for (int e = tid; e < kNB * kNB; e += 256) {
    const int rr = e >> 7, cc = e & (kNB - 1);
    const float v = (cc <= rr) ? sX[rr * kLP + cc] : 0.0f;
    if (rr < m && cc < m) X[(n0 + rr) * ld + n0 + cc] = v;
  }
}

// in-place U = J X J over the full K x K matrix (swap (i,j) <-> (K-1-i, K-1-j))
__global__ void reverse_inplace(float* __restrict__ p, int64_t K) {
  const int64_t total = K * K;
  const int64_t half = total / 2;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < half;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t other = total - 1 - idx;
    const float t = p[idx];
    p[idx] = p[other];
    p[other] = t;
  }
}

__global__ void reverse_copy(const float* __restrict__ src, float* __restrict__ dst, int64_t K) {
  const int64_t total = K * K;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x)
    dst[idx] = src[total - 1 - idx];
}

unsigned grid_for(int64_t n, int threads) {
  int64_t b = cdiv(n, threads);
  return static_cast<unsigned>(std::min<int64_t>(b, 65536));
}

struct Ctx {
  hipStream_t st;
  float* A;     // K x K, ld K
  float* X;     // K x K, ld K
  float* tmp;   // per-level scratch
  int64_t K;
  int32_t* info;
};

static_assert(plan::kFactorLeaf == kNB, "the recursion's split rule and scratch size assume this leaf size");

// a node of size m splits into m1 = plan::factor_split(m) (whole leaves) and
// m - m1; the scratch below it (plan::factor_scratch_floats) holds L21 and T2
// of this node, then the right child's scratch
int chol_inv(Ctx& c, int64_t n0, int64_t m, float* tmp) {
  const int64_t ld = c.K;
  if (m <= kNB) {
    hipLaunchKernelGGL(chol_inv_leaf, dim3(1), dim3(256), kLeafLds, c.st, c.A, c.X, ld, n0,
                       static_cast<int>(m), c.info);
    return check_launch("chol_inv_leaf");
  }
  const int64_t m1 = plan::factor_split(m), m2 = m - m1;
  float* L21 = tmp;             // m2 x m1
  float* T2 = tmp + m2 * m1;    // m2 x m1
  float* deeper = tmp + 2 * m2 * m1;
  int rc = chol_inv(c, n0, m1, deeper);
  if (rc) return rc;
  const float* A21 = c.A + (n0 + m1) * ld + n0;
  float* A22 = c.A + (n0 + m1) * ld + n0 + m1;
  const float* X11 = c.X + n0 * ld + n0;
  float* X21 = c.X + (n0 + m1) * ld + n0;
  const float* X22 = c.X + (n0 + m1) * ld + n0 + m1;
  // L21 = A21 X11^T   (opB = X11^T is upper: k <= j)
  rc = launch_gemm_f32(c.st, m2, m1, m1, 1.0f, A21, ld, false, X11, ld, true, 0.0f, L21, m1, GEMM_KLIM_B_LE_J);
  if (rc) return rc;
  // S = A22 - L21 L21^T (lower triangle) and T2 = L21 X11 (opB = X11 lower:
  // k >= j): both need only L21, so they share one grid where their tiles
  // alone would leave CUs idle (T2 is kept until X21, below the recursion)
  const GemmCall S{m2, m2, m1, -1.0f, L21, m1, false, L21, m1, true, 1.0f, A22, ld, GEMM_C_LOWER};
  const GemmCall LX{m2, m1, m1, 1.0f, L21, m1, false, X11, ld, false, 0.0f, T2, m1, GEMM_KLIM_B_GE_J};
  rc = launch_gemm_f32_pair(c.st, S, LX);
  if (rc) return rc;
  rc = chol_inv(c, n0 + m1, m2, deeper);
  if (rc) return rc;
  // X21 = -X22 T2  (opA = X22 lower: k <= i)
  return launch_gemm_f32(c.st, m2, m1, m2, -1.0f, X22, ld, false, T2, m1, false, 0.0f, X21, ld, GEMM_KLIM_A_LE_I);
}

}  // namespace
}  // namespace gptq

using namespace gptq;

extern "C" int gptq_damp_factor(const float* H, int64_t K, float scale, float percdamp, const int32_t* perm, int mode,
                                float* Hd, float* out, int32_t* dead_cols, int32_t* info, void* workspace,
                                size_t workspace_bytes, gptq_stream_t stream) {
  clear_error();
  GPTQ_REQUIRE(H && out && info, GPTQ_ERR_ARG, "damp_factor: null pointer");
  GPTQ_REQUIRE(K > 0 && K <= (1 << 17), GPTQ_ERR_SHAPE, "damp_factor: bad K=%lld", (long long)K);
  GPTQ_REQUIRE(mode == GPTQ_FACTOR_FULL_INVERSE || mode == GPTQ_FACTOR_UPPER_CHOL_INV, GPTQ_ERR_ARG,
               "damp_factor: bad mode %d", mode);
  const size_t need = gptq_factor_workspace_size(K);
  GPTQ_REQUIRE(workspace && workspace_bytes >= need, GPTQ_ERR_WORKSPACE, "damp_factor: workspace %zu < %zu bytes",
               workspace_bytes, need);
  hipStream_t st = as_hip(stream);
  float* ws = static_cast<float*>(workspace);
  float* lam = ws;
  float* A = ws + 64;
  float* tmp = A + K * K;
  hipLaunchKernelGGL(diag_stats, dim3(1), dim3(1024), 0, st, H, K, scale, percdamp, dead_cols, lam, info);
  int rc = check_launch("diag_stats");
  if (rc) return rc;
  if (!Hd && K <= kRowLdsMax) {
    const int vec = (reinterpret_cast<uintptr_t>(H) % 16 == 0 && K % 4 == 0) ? 1 : 0;
    hipLaunchKernelGGL(build_A_rows, dim3(static_cast<unsigned>(K)), dim3(512), sizeof(float) * K, st, H, K, scale,
                       perm, dead_cols ? 1 : 0, lam, vec, A);
  } else {
    hipLaunchKernelGGL(build_A, dim3(static_cast<unsigned>(std::min<int64_t>(cdiv(K, 256), 64)),
                                    static_cast<unsigned>(std::min<int64_t>(K, 65535))),
                       dim3(256), 0, st, H, K, scale, perm, dead_cols ? 1 : 0, lam, A, Hd);
  }
  if ((rc = check_launch("build_A"))) return rc;
  hipLaunchKernelGGL(fill_zero, dim3(grid_for(K * K, 256)), dim3(256), 0, st, out, K * K);
  if ((rc = check_launch("fill_zero"))) return rc;
  Ctx c{st, A, out, tmp, K, info};
  if ((rc = chol_inv(c, 0, K, tmp))) return rc;
  if (mode == GPTQ_FACTOR_UPPER_CHOL_INV) {
    hipLaunchKernelGGL(reverse_inplace, dim3(grid_for(K * K / 2 + 1, 256)), dim3(256), 0, st, out, K);
    return check_launch("reverse_inplace");
  }
  // full inverse: P = X^T X (opA = X^T: k >= i; opB = X: k >= j) into A, then out = J P J
  rc = launch_gemm_f32(st, K, K, K, 1.0f, out, K, true, out, K, false, 0.0f, A, K, GEMM_KLIM_A_GE_I | GEMM_KLIM_B_GE_J);
  if (rc) return rc;
  hipLaunchKernelGGL(reverse_copy, dim3(grid_for(K * K, 256)), dim3(256), 0, st, A, out, K);
  return check_launch("reverse_copy");
}
