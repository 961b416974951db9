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
  const float l = lam[0];
  const int64_t total = K * K;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t i = idx / K, j = idx - (idx / K) * K;
    if (Hd) Hd[idx] = damped(H, K, scale, perm, fix_dead != 0, l, i, j);
    if (i >= j) A[idx] = damped(H, K, scale, perm, fix_dead != 0, l, K - 1 - i, K - 1 - j);
  }
}

__global__ void fill_zero(float* __restrict__ p, int64_t n) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = 0.0f;
}

// One workgroup of 256 threads: Cholesky of the m x m (m <= 128) diagonal
// block of A at (n0, n0) and the inverse of its factor.  Thread (ti, tk) of a
// 16 x 16 grid keeps rows 8*ti..8*ti+7, columns 8*tk..8*tk+7 of the block in
// registers; each right-looking step publishes only the next pivot column
// (Cholesky) or the next scaled row (inverse) through a double-buffered LDS
// vector, so a step costs one barrier, 16 LDS reads and 64 FMAs per thread.
// Writes L (zeros above) into A and X = L^-1 (zeros above) into X.  A
// non-positive pivot records info = 1 + (column in A order) once.
constexpr int kLP = kNB + 1;  // LDS pitch of L
constexpr size_t kLeafLds = sizeof(float) * (2 * kNB + kNB * kLP + 2 * kNB);

__global__ __launch_bounds__(256) void chol_inv_leaf(float* __restrict__ A, float* __restrict__ X, int64_t ld,
                                                     int64_t n0, int m, int32_t* __restrict__ info) {
  extern __shared__ float lds[];
  float* col = lds;                  // [2][kNB]
  float* Ls = lds + 2 * kNB;         // [kNB][kLP]
  float* xrow = Ls + kNB * kLP;      // [2][kNB]
  const int tid = threadIdx.x;
  const int ti = tid >> 4, tk = tid & 15;
  const int R0 = 8 * ti, C0 = 8 * tk;
  float a[8][8];
#pragma unroll
  for (int u = 0; u < 8; ++u)
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const int r = R0 + u, c = C0 + v;
      a[u][v] = (r < m && c <= r) ? A[(n0 + r) * ld + n0 + c] : 0.0f;
    }
  if (tk == 0) {
#pragma unroll
    for (int u = 0; u < 8; ++u) col[R0 + u] = a[u][0];
  }
  __syncthreads();
  int first_bad = -1;
  for (int j = 0; j < m; ++j) {
    const float* cj = col + (j & 1) * kNB;
    const float p = cj[j];
    if (!(p > 0.0f) && first_bad < 0) first_bad = j;
    const float d = sqrtf(p);
    const float inv = 1.0f / d;
    if (R0 + 7 >= j) {
      // unconditional vector reads, masked afterwards (a guarded read would
      // become a branch with its own LDS round trip)
      float cr[8], cc[8];
      *reinterpret_cast<f32x4*>(cr) = *reinterpret_cast<const f32x4*>(cj + R0);
      *reinterpret_cast<f32x4*>(cr + 4) = *reinterpret_cast<const f32x4*>(cj + R0 + 4);
      *reinterpret_cast<f32x4*>(cc) = *reinterpret_cast<const f32x4*>(cj + C0);
      *reinterpret_cast<f32x4*>(cc + 4) = *reinterpret_cast<const f32x4*>(cj + C0 + 4);
      float lr[8], lc[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) lr[u] = (R0 + u > j) ? cr[u] * inv : 0.0f;
#pragma unroll
      for (int v = 0; v < 8; ++v) lc[v] = (C0 + v > j) ? cc[v] * inv : 0.0f;
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int v = 0; v < 8; ++v) a[u][v] -= lr[u] * lc[v];
      if (C0 <= j && j < C0 + 8) {
        // column j of L: l = a / d below the diagonal, d on it
#pragma unroll
        for (int v = 0; v < 8; ++v)
          if (C0 + v == j) {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
              const int r = R0 + u;
              if (r > j) a[u][v] = lr[u];
              else if (r == j) a[u][v] = d;
            }
          }
      }
      const int jn = j + 1;
      if (jn < m && C0 <= jn && jn < C0 + 8) {
        float* cn = col + (jn & 1) * kNB;
#pragma unroll
        for (int v = 0; v < 8; ++v)
          if (C0 + v == jn) {
#pragma unroll
            for (int u = 0; u < 8; ++u) cn[R0 + u] = a[u][v];
          }
      }
    }
    __syncthreads();
  }
  if (first_bad >= 0 && tid == 0) atomicCAS(info, 0, static_cast<int32_t>(n0 + first_bad + 1));
#pragma unroll
  for (int u = 0; u < 8; ++u)
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const int r = R0 + u, c = C0 + v;
      const float val = (c <= r) ? a[u][v] : 0.0f;
      Ls[r * kLP + c] = val;
      if (r < m && c < m) A[(n0 + r) * ld + n0 + c] = val;
    }
  __syncthreads();
  // X = L^-1, right-looking on rows: row j is scaled by 1/L[j][j] when it is
  // published, then subtracted from the rows below with weights L[r][j]
  float x[8][8];
#pragma unroll
  for (int u = 0; u < 8; ++u)
#pragma unroll
    for (int v = 0; v < 8; ++v) x[u][v] = (R0 + u == C0 + v && R0 + u < m) ? 1.0f : 0.0f;
  if (ti == 0) {
    const float s0 = 1.0f / Ls[0];
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      x[0][v] *= s0;
      xrow[C0 + v] = x[0][v];
    }
  }
  __syncthreads();
  for (int j = 0; j < m; ++j) {
    const float* xj = xrow + (j & 1) * kNB;
    if (R0 + 7 > j) {
      float lt[8], lr[8], xc[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) lt[u] = Ls[(R0 + u) * kLP + j];
      *reinterpret_cast<f32x4*>(xc) = *reinterpret_cast<const f32x4*>(xj + C0);
      *reinterpret_cast<f32x4*>(xc + 4) = *reinterpret_cast<const f32x4*>(xj + C0 + 4);
#pragma unroll
      for (int u = 0; u < 8; ++u) lr[u] = (R0 + u > j) ? lt[u] : 0.0f;
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int v = 0; v < 8; ++v) x[u][v] -= lr[u] * xc[v];
      const int jn = j + 1;
      if (jn < m && R0 <= jn && jn < R0 + 8) {
        const float sn = 1.0f / Ls[jn * kLP + jn];
        float* xn = xrow + (jn & 1) * kNB;
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (R0 + u == jn) {
#pragma unroll
            for (int v = 0; v < 8; ++v) {
              x[u][v] *= sn;
              xn[C0 + v] = x[u][v];
            }
          }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int u = 0; u < 8; ++u)
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const int r = R0 + u, c = C0 + v;
      if (r < m && c < m) X[(n0 + r) * ld + n0 + c] = (c <= r) ? x[u][v] : 0.0f;
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

int64_t split_of(int64_t m) {
  const int64_t nb = cdiv(m, kNB);
  return ((nb + 1) / 2) * kNB;
}

// scratch needed below a node of size m: 2 * m2 * m1 floats at this node +
// whatever the right child needs (the left child's scratch is reused)
int64_t scratch_floats(int64_t m) {
  if (m <= kNB) return 0;
  const int64_t m1 = split_of(m), m2 = m - m1;
  return 2 * m2 * m1 + std::max(scratch_floats(m1), scratch_floats(m2));
}

int chol_inv(Ctx& c, int64_t n0, int64_t m, float* tmp) {
  const int64_t ld = c.K;
  if (m <= kNB) {
    hipLaunchKernelGGL(chol_inv_leaf, dim3(1), dim3(256), kLeafLds, c.st, c.A, c.X, ld, n0,
                       static_cast<int>(m), c.info);
    return check_launch("chol_inv_leaf");
  }
  const int64_t m1 = split_of(m), m2 = m - m1;
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
  // S = A22 - L21 L21^T (lower triangle)
  rc = launch_gemm_f32(c.st, m2, m2, m1, -1.0f, L21, m1, false, L21, m1, true, 1.0f, A22, ld, GEMM_C_LOWER);
  if (rc) return rc;
  rc = chol_inv(c, n0 + m1, m2, deeper);
  if (rc) return rc;
  // T2 = L21 X11   (opB = X11 lower: k >= j)
  rc = launch_gemm_f32(c.st, m2, m1, m1, 1.0f, L21, m1, false, X11, ld, false, 0.0f, T2, m1, GEMM_KLIM_B_GE_J);
  if (rc) return rc;
  // X21 = -X22 T2  (opA = X22 lower: k <= i)
  return launch_gemm_f32(c.st, m2, m1, m2, -1.0f, X22, ld, false, T2, m1, false, 0.0f, X21, ld, GEMM_KLIM_A_LE_I);
}

}  // namespace
}  // namespace gptq

using namespace gptq;

static size_t factor_ws_floats(int64_t K) {
  // [lambda pad 64 floats][A K*K][scratch]
  return 64 + static_cast<size_t>(K) * K + static_cast<size_t>(scratch_floats(K));
}

extern "C" size_t gptq_factor_workspace_size(int64_t K) {
  if (K <= 0) return 0;
  return factor_ws_floats(K) * sizeof(float);
}

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
  hipLaunchKernelGGL(build_A, dim3(grid_for(K * K, 256)), dim3(256), 0, st, H, K, scale, perm, dead_cols ? 1 : 0, lam,
                     A, Hd);
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
