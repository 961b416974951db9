// The GPTQ column sweep (quantise, propagate the error) on gfx950.
//
// Rows are independent given the read-only propagation matrix T, so the
// sweep is row-parallel: one wave owns R rows of a sub-block of at most 128
// columns, lane l holding columns l and l + 64 of every row in registers.
// Column j is quantised by every lane (only the owner lane's value is
// final), its error e is broadcast with v_readlane (uniform j, no barrier),
// and each lane updates its later columns with T[j][col] read from LDS,
// where the workgroup staged the T sub-block once.
//
// Per block of `blocksize` columns:
//   1. sweep_params: min-max parameters of every group that starts in the
//      block, from the weights as they stand at the block start;
//   2. for each sub-block of <= 128 columns: sweep_sub, then the lazy-batch
//      update W[:, j2:end] -= E T[j1:j2, j2:end] as one fp32-MFMA GEMM
//      (end = cols with the trailing update, the block end without it).
// Splitting a block into sub-blocks with an update in between is an exact
// re-association of the column-by-column updates.
#include "gemm.hpp"

namespace gptq {
namespace {

constexpr int kSub = 128;

__device__ __forceinline__ void group_params(float xmin, float xmax, int maxq, bool ref, float& s, float& z,
                                             bool sym = false) {
  if (!ref && sym) {
    // symmetric canonical form: xmax = max(|xmin|, xmax), xmin = -xmax
    // where xmin < 0; zero point in the middle of the code range
    xmin = fminf(xmin, 0.0f);
    xmax = fmaxf(fmaxf(fabsf(xmin), xmax), 0.0f);
    if (xmin < 0.0f) xmin = -xmax;
    if (xmin == 0.0f && xmax == 0.0f) {
      xmin = -1.0f;
      xmax = 1.0f;
    }
    s = (xmax - xmin) / static_cast<float>(maxq);
    z = static_cast<float>((maxq + 1) / 2);
    return;
  }
  if (!ref) {
    xmin = fminf(xmin, 0.0f);
    xmax = fmaxf(xmax, 0.0f);
    if (xmin == 0.0f && xmax == 0.0f) {
      xmin = -1.0f;
      xmax = 1.0f;
    }
  }
  s = (xmax - xmin) / static_cast<float>(maxq);
  if (s == 0.0f) s = 1.0f;  // constant group (reference mode): guard against 0/0
  z = rintf(-xmin / s);
}

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// one wave per (row, group starting in [c_lo, c_hi))
__global__ __launch_bounds__(256) void sweep_params(const float* __restrict__ src, int64_t ld, int64_t rows,
                                                    int64_t cols, int gs, int maxq, int ref, int64_t g_first,
                                                    int64_t g_count, float* __restrict__ scale,
                                                    float* __restrict__ zero, int64_t ngroups, int sym = 0) {
  const int64_t w = blockIdx.x * 4LL + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (w >= rows * g_count) return;
  const int64_t row = w / g_count;
  const int64_t g = g_first + (w - row * g_count);
  const int64_t c0 = g * gs;
  const int64_t c1 = std::min<int64_t>(c0 + gs, cols);
  float mn = INFINITY, mx = -INFINITY;
  for (int64_t c = c0 + lane; c < c1; c += 64) {
    const float v = src[row * ld + c];
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
  mn = wave_min(mn);
  mx = wave_max(mx);
  if (lane == 0) {
    float s, z;
    group_params(mn, mx, maxq, ref != 0, s, z, sym != 0);
    scale[row * ngroups + g] = s;
    zero[row * ngroups + g] = z;
  }
}

struct SubArgs {
  const float* W;
  const float* T;
  int64_t ldt;
  int64_t cols, rows, j1;
  int n;          // sub-block width (<= 128)
  int gs;         // <= 0: one group per row
  int maxq;
  int ref;
  const float* scale;
  const float* zero;
  int64_t ngroups;
  int64_t g_lo;
  int G;          // groups spanned by the sub-block
  const int32_t* out_cols;
  uint8_t* codes;
  void* dq;
  int dq_dtype;
  float* err_sq;
  float* losses;
  float* Err;
  int64_t lde;
  int64_t e_off;
};

template <int R, int NC>
__global__ __launch_bounds__(256) void sweep_sub(SubArgs a) {
  extern __shared__ float smem[];
  constexpr int P = 64 * NC;  // pitch of the T sub-block in LDS
  float* Tb = smem;
  float* prm = smem + P * P;  // [wave][r][g][2]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = a.n;

  for (int e = tid; e < n * n; e += 256) {
    const int r = e / n, c = e - (e / n) * n;
    Tb[r * P + c] = a.T[(a.j1 + r) * a.ldt + a.j1 + c];
  }
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * R;
  float* wp = prm + wave * (R * a.G * 2);
  for (int e = lane; e < R * a.G; e += 64) {
    const int r = e / a.G, g = e - (e / a.G) * a.G;
    const int64_t row = row0 + r;
    float s = 1.0f, z = 0.0f;
    if (row < a.rows) {
      s = a.scale[row * a.ngroups + a.g_lo + g];
      z = a.zero[row * a.ngroups + a.g_lo + g];
    }
    wp[e * 2] = s;
    wp[e * 2 + 1] = z;
  }
  __syncthreads();
  if (row0 >= a.rows) return;

  float w[R][NC], qv[R][NC], dv[R][NC], ev[R][NC], lv[R][NC];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int col = c * 64 + lane;
      const int64_t row = row0 + r;
      w[r][c] = (row < a.rows && col < n) ? a.W[row * a.cols + a.j1 + col] : 0.0f;
      qv[r][c] = dv[r][c] = ev[r][c] = lv[r][c] = 0.0f;
    }
  float esq[R];
#pragma unroll
  for (int r = 0; r < R; ++r) esq[r] = 0.0f;

  const float fmaxq = static_cast<float>(a.maxq);
  for (int j = 0; j < n; ++j) {
    const int slot = j >> 6;
    const int owner = j & 63;
    const int g = a.gs > 0 ? static_cast<int>((a.j1 + j) / a.gs - a.g_lo) : 0;
    const float d = Tb[j * P + j];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float wj = (NC == 1 || slot == 0) ? w[r][0] : w[r][NC - 1];
      const float s = wp[(r * a.G + g) * 2];
      const float z = wp[(r * a.G + g) * 2 + 1];
      float q;
      if (a.ref)
        q = fminf(fmaxf(rintf(wj / s + z), 0.0f), fmaxq);
      else
        q = fminf(fmaxf(rintf(wj / s) + z, 0.0f), fmaxq);
      const float dq = s * (q - z);
      const float diff = wj - dq;
      const float e = diff / d;
      const float eu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), owner));
      if (lane == owner) {
        const float loss = diff * diff / (d * d) * 0.5f;
        if (NC == 1 || slot == 0) {
          qv[r][0] = q; dv[r][0] = dq; ev[r][0] = e; lv[r][0] = loss;
        } else {
          qv[r][NC - 1] = q; dv[r][NC - 1] = dq; ev[r][NC - 1] = e; lv[r][NC - 1] = loss;
        }
      }
      esq[r] += eu * eu;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int col = c * 64 + lane;
        if (col > j && col < n) w[r][c] -= eu * Tb[j * P + col];
      }
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t row = row0 + r;
    if (row >= a.rows) continue;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int col = c * 64 + lane;
      if (col >= n) continue;
      const int64_t gc = a.j1 + col;
      const int64_t oc = a.out_cols ? a.out_cols[gc] : gc;
      a.codes[row * a.cols + oc] = static_cast<uint8_t>(qv[r][c]);
      if (a.dq) store_elem(a.dq, row * a.cols + oc, a.dq_dtype, dv[r][c]);
      if (a.losses) a.losses[row * a.cols + oc] = lv[r][c];
      if (a.Err) a.Err[row * a.lde + a.e_off + col] = ev[r][c];
    }
    if (a.err_sq && lane == 0) a.err_sq[row] += esq[r];
  }
}

// ------------------------------------------------ lanes-own-rows sweep --
// Lane = row: every lane quantises its own row, so no work is discarded.  A
// wave's 64 rows x n (<= 128) columns live column-major in LDS (ws[c][lane],
// conflict-free); T^T of the sub-block is staged once per workgroup
// (Tt[c][r] = T[r][c]).  Columns are processed in 32-wide panels: the panel
// is held in registers and swept with a fully unrolled 32-step loop (T values
// are LDS broadcast reads), then every later column of the sub-block takes
// the panel's rank-32 update as a 32-term dot product.
constexpr int kPW = 32;
constexpr int kRowWaves = 2;  // waves (64 rows each) per workgroup
constexpr int kTt = 132;      // row pitch of Tt in floats (16-byte aligned)
constexpr int kMaxG = 6;      // groups a 128-column sub-block can touch when g >= 32

// a / b from a correctly rounded reciprocal rb of b: one FMA residual step
// (Markstein), so the quotient is the correctly rounded one except in rare
// near-midpoint cases, at three dependent operations instead of an IEEE
// division sequence on the column recurrence
__device__ __forceinline__ float div_rcp(float a, float b, float rb) {
  const float q0 = a * rb;
  const float r = fmaf(-q0, b, a);
  return fmaf(r, rb, q0);
}

template <bool REF>
__global__ __launch_bounds__(64 * kRowWaves) void sweep_rows(SubArgs a) {
  extern __shared__ float smem[];
  float* Tt = smem;                                   // 128 x kTt
  float* ws_all = smem + 128 * kTt;                   // [wave][128][64]
  float* prm_all = ws_all + kRowWaves * 128 * 64;     // [wave][kMaxG][2][64]
  float* invd = prm_all + kRowWaves * kMaxG * 2 * 64;  // [128] 1 / T[j][j]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = a.n;
  float* ws = ws_all + wave * 128 * 64;
  float* prm = prm_all + wave * kMaxG * 2 * 64;

  // Stage the T block transposed (Tt[c][r]) and this lane's row of W (ws),
  // with eight loads per thread in flight before any is stored: a load-then-
  // store loop would pay one memory round trip per element.
  constexpr int kThr = 64 * kRowWaves;
  constexpr int kBatch = 8;
  const float* tsrc = a.T + a.j1 * a.ldt + a.j1;
  if ((n & 3) == 0 && (a.ldt & 3) == 0 && (reinterpret_cast<uintptr_t>(tsrc) & 15) == 0) {
    // vector e covers columns 4 (e / n) .. +3 of row e % n (consecutive
    // threads, consecutive rows: conflict-free transposed stores)
    const int tot = n * (n >> 2);
    for (int e0 = tid; e0 < tot; e0 += kThr * kBatch) {
      f32x4 v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int e = e0 + u * kThr;
        if (e < tot) v[u] = *reinterpret_cast<const f32x4*>(tsrc + (e % n) * a.ldt + 4 * (e / n));
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int e = e0 + u * kThr;
        if (e < tot) {
          const int r = e % n, c = 4 * (e / n);
#pragma unroll
          for (int q = 0; q < 4; ++q) Tt[(c + q) * kTt + r] = v[u][q];
        }
      }
    }
  } else {
    const int tot = n * n;
    for (int e0 = tid; e0 < tot; e0 += kThr * kBatch) {
      float v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int e = e0 + u * kThr;
        if (e < tot) v[u] = tsrc[(e % n) * a.ldt + e / n];
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int e = e0 + u * kThr;
        if (e < tot) Tt[(e / n) * kTt + e % n] = v[u];
      }
    }
  }
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (64 * kRowWaves) + wave * 64 + lane;
  const bool valid = row < a.rows;
  const int64_t rrow = valid ? row : a.rows - 1;
  {
    const float* src = a.W + rrow * a.cols + a.j1;
    int c = 0;
    if ((reinterpret_cast<uintptr_t>(src) & 15) == 0) {
      for (; c + 4 * kBatch <= n; c += 4 * kBatch) {
        f32x4 v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) v[u] = *reinterpret_cast<const f32x4*>(src + c + 4 * u);
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
#pragma unroll
          for (int q = 0; q < 4; ++q) ws[(c + 4 * u + q) * 64 + lane] = v[u][q];
      }
    }
    for (; c < n; ++c) ws[c * 64 + lane] = src[c];
  }
  for (int g = 0; g < a.G; ++g) {
    prm[(g * 2) * 64 + lane] = a.scale[rrow * a.ngroups + a.g_lo + g];
    prm[(g * 2 + 1) * 64 + lane] = a.zero[rrow * a.ngroups + a.g_lo + g];
  }
  __syncthreads();
  for (int j = tid; j < n; j += kThr) invd[j] = 1.0f / Tt[j * kTt + j];
  __syncthreads();

  const float fmaxq = static_cast<float>(a.maxq);
  const int gs = a.gs;
  const int j1 = static_cast<int>(a.j1 - a.g_lo * static_cast<int64_t>(gs > 0 ? gs : 0));  // offset in group 0
  float esq = 0.0f;
  for (int p0 = 0; p0 < n; p0 += kPW) {
    // groups of this panel: g0 for columns before `brk`, g0 + 1 after (g >= 32)
    int g0 = 0, brk = kPW;
    if (gs > 0) {
      g0 = (j1 + p0) / gs;
      brk = (g0 + 1) * gs - (j1 + p0);
    }
    const float s0 = prm[(g0 * 2) * 64 + lane], z0 = prm[(g0 * 2 + 1) * 64 + lane];
    const int g1 = (g0 + 1 < a.G) ? g0 + 1 : g0;
    const float s1 = prm[(g1 * 2) * 64 + lane], z1 = prm[(g1 * 2 + 1) * 64 + lane];
    const float is0 = 1.0f / s0, is1 = 1.0f / s1;
    float ep[kPW], qp[kPW], dp[kPW], lp[kPW];
#pragma unroll
    for (int i = 0; i < kPW; ++i) {
      const int j = p0 + i;
      ep[i] = qp[i] = dp[i] = lp[i] = 0.0f;
      if (j < n) {
        // left-looking: apply the panel's earlier errors to column j
        float w = ws[j * 64 + lane];
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        const f32x4* trow = reinterpret_cast<const f32x4*>(Tt + j * kTt + p0);
#pragma unroll
        for (int k4 = 0; k4 < (i + 3) / 4; ++k4) {
          const f32x4 t = trow[k4];
#pragma unroll
          for (int u = 0; u < 4; ++u)
            if (4 * k4 + u < i) acc[u] += ep[4 * k4 + u] * t[u];
        }
        w -= (acc[0] + acc[1]) + (acc[2] + acc[3]);
        const bool second = i >= brk;
        const float s = second ? s1 : s0;
        const float is = second ? is1 : is0;
        const float z = second ? z1 : z0;
        const float t = div_rcp(w, s, is);
        float q;
        if constexpr (REF)
          q = fminf(fmaxf(rintf(t + z), 0.0f), fmaxq);
        else
          q = fminf(fmaxf(rintf(t) + z, 0.0f), fmaxq);
        const float dq = s * (q - z);
        const float d = Tt[j * kTt + j];
        const float diff = w - dq;
        const float e = div_rcp(diff, d, invd[j]);
        ep[i] = e;
        qp[i] = q;
        dp[i] = dq;
        lp[i] = 0.5f * e * e;
        esq += e * e;
      }
    }
    // rank-32 update of the rest of the sub-block
    for (int c = p0 + kPW; c < n; ++c) {
      const f32x4* tv = reinterpret_cast<const f32x4*>(Tt + c * kTt + p0);
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int v = 0; v < kPW / 4; ++v) {
        const f32x4 t = tv[v];
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[u] += ep[4 * v + u] * t[u];
      }
      ws[c * 64 + lane] -= (acc[0] + acc[1]) + (acc[2] + acc[3]);
    }
    if (valid) {
      const int64_t gc0 = a.j1 + p0;
      const bool full = p0 + kPW <= n;
      const bool vec = full && !a.out_cols && ((row * a.cols + gc0) & 15) == 0;
      if (vec) {
        u32x4 cw[2];
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const uint32_t w4 = static_cast<uint32_t>(qp[4 * v]) | (static_cast<uint32_t>(qp[4 * v + 1]) << 8) |
                              (static_cast<uint32_t>(qp[4 * v + 2]) << 16) |
                              (static_cast<uint32_t>(qp[4 * v + 3]) << 24);
          cw[v / 4][v % 4] = w4;
        }
        u32x4* cdst = reinterpret_cast<u32x4*>(a.codes + row * a.cols + gc0);
        cdst[0] = cw[0];
        cdst[1] = cw[1];
        if (a.losses) {
          f32x4* ldst = reinterpret_cast<f32x4*>(a.losses + row * a.cols + gc0);
#pragma unroll
          for (int v = 0; v < 8; ++v) ldst[v] = f32x4{lp[4 * v], lp[4 * v + 1], lp[4 * v + 2], lp[4 * v + 3]};
        }
        if (a.dq) {
#pragma unroll
          for (int i = 0; i < kPW; ++i) store_elem(a.dq, row * a.cols + gc0 + i, a.dq_dtype, dp[i]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < kPW; ++i) {
          const int j = p0 + i;
          if (j < n) {
            const int64_t gc = a.j1 + j;
            const int64_t oc = a.out_cols ? a.out_cols[gc] : gc;
            a.codes[row * a.cols + oc] = static_cast<uint8_t>(qp[i]);
            if (a.dq) store_elem(a.dq, row * a.cols + oc, a.dq_dtype, dp[i]);
            if (a.losses) a.losses[row * a.cols + oc] = lp[i];
          }
        }
      }
      if (a.Err) {
        float* edst = a.Err + row * a.lde + a.e_off + p0;
        if (full && ((reinterpret_cast<uintptr_t>(edst) & 15) == 0)) {
#pragma unroll
          for (int v = 0; v < 8; ++v)
            reinterpret_cast<f32x4*>(edst)[v] = f32x4{ep[4 * v], ep[4 * v + 1], ep[4 * v + 2], ep[4 * v + 3]};
        } else {
#pragma unroll
          for (int i = 0; i < kPW; ++i)
            if (p0 + i < n) edst[i] = ep[i];
        }
      }
    }
  }
  if (valid && a.err_sq) a.err_sq[row] += esq;
}

__global__ void fill_zero_f(float* __restrict__ p, int64_t n) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = 0.0f;
}

__global__ void quantize_rows_k(const float* __restrict__ x, int64_t rows, int64_t cols, int gs, int maxq, int ref,
                                const float* __restrict__ scale, const float* __restrict__ zero, int64_t ngroups,
                                uint8_t* __restrict__ codes, float* __restrict__ dq) {
  const int64_t total = rows * cols;
  const float fmaxq = static_cast<float>(maxq);
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = idx / cols, c = idx - (idx / cols) * cols;
    const int64_t g = gs > 0 ? c / gs : 0;
    const float s = scale[r * ngroups + g], z = zero[r * ngroups + g];
    const float w = x[idx];
    float q;
    if (ref)
      q = fminf(fmaxf(rintf(w / s + z), 0.0f), fmaxq);
    else
      q = fminf(fmaxf(rintf(w / s) + z, 0.0f), fmaxq);
    if (codes) codes[idx] = static_cast<uint8_t>(q);
    if (dq) dq[idx] = s * (q - z);
  }
}

// out[r][c] = w[r][perm[c]] (or w[perm[c]][r] transposed), dead columns -> 0
__global__ void prepare_weight_k(const void* __restrict__ w, int dtype, int64_t rows, int64_t cols, int64_t ldw,
                                 const int32_t* __restrict__ perm, const int32_t* __restrict__ dead, int transpose,
                                 float* __restrict__ out) {
  const int64_t total = rows * cols;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = idx / cols, c = idx - (idx / cols) * cols;
    const int64_t pc = perm ? perm[c] : c;
    float v;
    if (transpose)
      v = load_elem(w, pc * ldw + r, dtype);
    else
      v = load_elem(w, r * ldw + pc, dtype);
    if (dead && dead[pc]) v = 0.0f;
    out[idx] = v;
  }
}

int launch_rows(hipStream_t st, const SubArgs& a) {
  const unsigned blocks = static_cast<unsigned>(cdiv(a.rows, 64LL * kRowWaves));
  const size_t lds = sizeof(float) * (128 * kTt + kRowWaves * 128 * 64 + kRowWaves * kMaxG * 2 * 64 + 128);
  if (a.ref)
    hipLaunchKernelGGL(sweep_rows<true>, dim3(blocks), dim3(64 * kRowWaves), lds, st, a);
  else
    hipLaunchKernelGGL(sweep_rows<false>, dim3(blocks), dim3(64 * kRowWaves), lds, st, a);
  return check_launch("sweep_rows");
}

template <int R, int NC>
int launch_sub(hipStream_t st, const SubArgs& a) {
  const unsigned blocks = static_cast<unsigned>(cdiv(a.rows, 4LL * R));
  const size_t lds = sizeof(float) * (static_cast<size_t>(64 * NC) * (64 * NC) + 4 * R * a.G * 2);
  hipLaunchKernelGGL((sweep_sub<R, NC>), dim3(blocks), dim3(256), lds, st, a);
  return check_launch("sweep_sub");
}

}  // namespace
}  // namespace gptq

using namespace gptq;

extern "C" size_t gptq_sweep_workspace_size(int64_t rows, int64_t cols, int blocksize) {
  (void)cols;
  (void)blocksize;
  if (rows <= 0) return 0;
  return static_cast<size_t>(rows) * kSub * sizeof(float);
}

extern "C" int gptq_minmax_params(const float* src, int64_t rows, int64_t cols, int64_t ld, int bits, int group_size,
                                  int flags, float* scale, float* zero, gptq_stream_t stream) {
  clear_error();
  GPTQ_REQUIRE(src && scale && zero, GPTQ_ERR_ARG, "minmax_params: null pointer");
  GPTQ_REQUIRE(rows > 0 && cols > 0 && ld >= cols, GPTQ_ERR_SHAPE, "minmax_params: bad shape");
  GPTQ_REQUIRE(bits >= 1 && bits <= 8, GPTQ_ERR_ARG, "minmax_params: bits=%d", bits);
  const int64_t gs = group_size > 0 ? std::min<int64_t>(group_size, cols) : cols;
  const int64_t ng = cdiv(cols, gs);
  const unsigned blocks = static_cast<unsigned>(cdiv(rows * ng, 4));
  hipLaunchKernelGGL(sweep_params, dim3(blocks), dim3(256), 0, as_hip(stream), src, ld, rows, cols, static_cast<int>(gs),
                     (1 << bits) - 1, (flags & GPTQ_SWEEP_REF_QUANTIZER) ? 1 : 0, 0LL, ng, scale, zero, ng,
                     (flags & GPTQ_PARAMS_SYM) ? 1 : 0);
  return check_launch("minmax_params");
}

extern "C" int gptq_quantize_rows(const float* x, int64_t rows, int64_t cols, int bits, int group_size, int flags,
                                  const float* scale, const float* zero, uint8_t* codes, float* dequant,
                                  gptq_stream_t stream) {
  clear_error();
  GPTQ_REQUIRE(x && scale && zero, GPTQ_ERR_ARG, "quantize_rows: null pointer");
  GPTQ_REQUIRE(rows > 0 && cols > 0, GPTQ_ERR_SHAPE, "quantize_rows: bad shape");
  GPTQ_REQUIRE(bits >= 1 && bits <= 8, GPTQ_ERR_ARG, "quantize_rows: bits=%d", bits);
  const int gs = group_size > 0 ? group_size : 0;
  const int64_t ng = gs > 0 ? cdiv(cols, gs) : 1;
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(cdiv(rows * cols, 256), 65536));
  hipLaunchKernelGGL(quantize_rows_k, dim3(blocks), dim3(256), 0, as_hip(stream), x, rows, cols, gs, (1 << bits) - 1,
                     (flags & GPTQ_SWEEP_REF_QUANTIZER) ? 1 : 0, scale, zero, ng, codes, dequant);
  return check_launch("quantize_rows");
}

extern "C" int gptq_prepare_weight(const void* w, int dtype, int64_t rows, int64_t cols, int64_t ldw,
                                   const int32_t* perm, const int32_t* dead_cols, int transpose, float* out,
                                   gptq_stream_t stream) {
  clear_error();
  GPTQ_REQUIRE(w && out, GPTQ_ERR_ARG, "prepare_weight: null pointer");
  GPTQ_REQUIRE(valid_dtype(dtype), GPTQ_ERR_DTYPE, "prepare_weight: bad dtype %d", dtype);
  GPTQ_REQUIRE(rows > 0 && cols > 0 && ldw >= (transpose ? rows : cols), GPTQ_ERR_SHAPE,
               "prepare_weight: bad shape");
  const int64_t total = rows * cols;
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(cdiv(total, 256), 65536));
  hipLaunchKernelGGL(prepare_weight_k, dim3(blocks), dim3(256), 0, as_hip(stream), w, dtype, rows, cols, ldw, perm,
                     dead_cols, transpose, out);
  return check_launch("prepare_weight");
}

extern "C" int gptq_quantize_sweep(float* W, const float* W0, const float* T, int64_t ldt, int64_t rows, int64_t cols, int bits,
                                   int group_size, int blocksize, int flags, const int32_t* out_cols, uint8_t* codes,
                                   void* dequant, int dequant_dtype, float* scale, float* zero, float* err_sq,
                                   float* losses, void* workspace, size_t workspace_bytes, gptq_stream_t stream) {
  clear_error();
  GPTQ_REQUIRE(W && T && codes && scale && zero, GPTQ_ERR_ARG, "quantize_sweep: null pointer");
  GPTQ_REQUIRE(rows > 0 && cols > 0 && ldt >= cols, GPTQ_ERR_SHAPE, "quantize_sweep: bad shape");
  GPTQ_REQUIRE(bits >= 1 && bits <= 8, GPTQ_ERR_ARG, "quantize_sweep: bits=%d", bits);
  GPTQ_REQUIRE(blocksize > 0, GPTQ_ERR_ARG, "quantize_sweep: blocksize=%d", blocksize);
  GPTQ_REQUIRE(!dequant || valid_dtype(dequant_dtype), GPTQ_ERR_DTYPE, "quantize_sweep: bad dequant dtype");
  GPTQ_REQUIRE(!(flags & GPTQ_SWEEP_GROUPS_FROM_W0) || W0, GPTQ_ERR_ARG, "quantize_sweep: GROUPS_FROM_W0 needs W0");
  const size_t need = gptq_sweep_workspace_size(rows, cols, blocksize);
  GPTQ_REQUIRE(workspace && workspace_bytes >= need, GPTQ_ERR_WORKSPACE, "quantize_sweep: workspace %zu < %zu",
               workspace_bytes, need);
  hipStream_t st = as_hip(stream);
  const int maxq = (1 << bits) - 1;
  const bool ref = (flags & GPTQ_SWEEP_REF_QUANTIZER) != 0;
  const bool trailing = (flags & GPTQ_SWEEP_TRAILING) != 0;
  const int gs = group_size > 0 ? group_size : 0;
  const int64_t ngroups = gs > 0 ? cdiv(cols, gs) : 1;
  const float* psrc = (flags & GPTQ_SWEEP_GROUPS_FROM_W0) ? W0 : W;
  float* Err = static_cast<float*>(workspace);
  int rc;
  if (err_sq) {
    hipLaunchKernelGGL(fill_zero_f, dim3(static_cast<unsigned>(std::min<int64_t>(cdiv(rows, 256), 65536))), dim3(256),
                       0, st, err_sq, rows);
    if ((rc = check_launch("fill_zero"))) return rc;
  }
  // rows per wave: more rows per wave amortise the per-column work; fewer
  // rows give more waves when the layer is narrow
  const int R = rows >= 4096 ? 4 : (rows >= 1024 ? 2 : 1);
  for (int64_t i1 = 0; i1 < cols; i1 += blocksize) {
    const int64_t i2 = std::min<int64_t>(i1 + blocksize, cols);
    if (gs > 0) {
      const int64_t g_first = cdiv(i1, gs);
      const int64_t g_end = cdiv(i2, gs);  // groups whose start lies in [i1, i2)
      if (g_end > g_first) {
        const int64_t g_count = g_end - g_first;
        const unsigned blocks = static_cast<unsigned>(cdiv(rows * g_count, 4));
        hipLaunchKernelGGL(sweep_params, dim3(blocks), dim3(256), 0, st, psrc, cols, rows, cols, gs, maxq, ref ? 1 : 0,
                           g_first, g_count, scale, zero, ngroups);
        if ((rc = check_launch("sweep_params"))) return rc;
      }
    }
    for (int64_t j1 = i1; j1 < i2; j1 += kSub) {
      const int64_t j2 = std::min<int64_t>(j1 + kSub, i2);
      const int n = static_cast<int>(j2 - j1);
      SubArgs a;
      a.W = W; a.T = T; a.ldt = ldt; a.cols = cols; a.rows = rows; a.j1 = j1; a.n = n; a.gs = gs; a.maxq = maxq;
      a.ref = ref ? 1 : 0; a.scale = scale; a.zero = zero; a.ngroups = ngroups;
      a.g_lo = gs > 0 ? j1 / gs : 0;
      a.G = gs > 0 ? static_cast<int>((j2 - 1) / gs - j1 / gs + 1) : 1;
      a.out_cols = out_cols; a.codes = codes; a.dq = dequant; a.dq_dtype = dequant_dtype;
      a.err_sq = err_sq; a.losses = losses; a.Err = Err; a.lde = kSub; a.e_off = 0;
      const bool wide = n > 64;
      if ((gs <= 0 || gs >= kPW) && a.G <= kMaxG) {
        // one group boundary at most per 32-column panel
        rc = launch_rows(st, a);
      } else if (R == 4) {
        rc = wide ? launch_sub<4, 2>(st, a) : launch_sub<4, 1>(st, a);
      } else if (R == 2) {
        rc = wide ? launch_sub<2, 2>(st, a) : launch_sub<2, 1>(st, a);
      } else {
        rc = wide ? launch_sub<1, 2>(st, a) : launch_sub<1, 1>(st, a);
      }
      if (rc) return rc;
      const int64_t end = trailing ? cols : i2;
      if (j2 < end) {
        rc = launch_gemm_f32(st, rows, end - j2, n, -1.0f, Err, kSub, false, T + j1 * ldt + j2, ldt, false, 1.0f,
                             W + j2, cols, 0);
        if (rc) return rc;
      }
    }
  }
  return GPTQ_OK;
}
