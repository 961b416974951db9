// The GPTQ column sweep (quantise, propagate the error) on gfx950.
//
// Rows are independent given the read-only propagation matrix T, so the
// sweep is row-parallel: sixteen lanes share a row of a sub-block of at most
// 128 columns, eight columns each in registers; each column's error is
// broadcast across the row's lanes with one DPP move and applied at once to
// the later columns, with T's sub-block staged in LDS once per workgroup.
//
// Per block of `blocksize` columns:
//   1. sweep_params: min-max parameters of every group that starts in the
//      block, from the weights as they stand at the block start (for blocks
//      of one 128-column sub-block with groups dividing it, sweep_r16 takes
//      them itself from the weights it loads);
//   2. for each sub-block of <= 128 columns: sweep_r16, then the lazy-batch
//      update W[:, j2:end] -= E T[j1:j2, j2:end] as one fp32-MFMA GEMM
//      (end = the block end without the trailing update; with it, the end of
//      the run of blocks spanning >= 512 columns that holds the sub-block);
//   3. with the trailing update, at the end of each run [s1, s2):
//      W[:, s2:] -= E_run T[s1:s2, s2:] as one GEMM of depth s2 - s1.
// Both are exact re-associations of the column-by-column updates, and every
// column has all earlier columns' updates by the time its block starts.
#include "gemm.hpp"

#include <utility>

namespace gptq {
namespace {

constexpr int kSub = 128;
constexpr int kFuseGroups = 2;  // groups per sub-block whose parameters sweep_r16 may compute

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

// min / max over each 16-lane row of the wave, in every lane (quad swaps,
// then the half-row and row mirrors)
template <bool MAX, int CTL>
__device__ __forceinline__ float row16_step(float v) {
  const float o = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTL, 0xF, 0xF, false));
  return MAX ? fmaxf(v, o) : fminf(v, o);
}
template <bool MAX>
__device__ __forceinline__ float row16_reduce(float v) {
  v = row16_step<MAX, 0xB1>(v);
  v = row16_step<MAX, 0x4E>(v);
  v = row16_step<MAX, 0x141>(v);
  return row16_step<MAX, 0x140>(v);
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
  float* scale;   // read; written too when fuse
  float* zero;
  int64_t ngroups;
  int64_t g_lo;
  int G;          // groups spanned by the sub-block
  int fuse;       // the groups' min-max parameters are computed here (see sweep_r16)
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

// a / b from a correctly rounded reciprocal rb of b: one FMA residual step
// (Markstein), so the quotient is the correctly rounded one except in rare
// near-midpoint cases, at three dependent operations instead of an IEEE
// division sequence on the column recurrence
__device__ __forceinline__ float div_rcp(float a, float b, float rb) {
  const float q0 = a * rb;
  const float r = fmaf(-q0, b, a);
  return fmaf(r, rb, q0);
}

// ------------------------------------------------------ 16-lane sweep --
// Sixteen lanes per row: lane 16r + q of a wave holds columns 4q..4q+3
// (registers 0-3) and 64+4q..64+4q+3 (registers 4-7) of row r of the wave's
// 4 rows.  Column j is quantised by all 16 lanes on the register that holds
// column j in its owner lane (j < 64: lane j / 4, else (j - 64) / 4), the
// owner's error is broadcast across the row with one DPP move
// (row_newbcast), and every lane applies it at once to its later columns: the
// eager column-by-column update of the GPTQ recurrence, in the same order.
// A wave covers 4 rows, so a layer of N rows runs as N / 4 waves.
//
// The sub-block of T is staged row-major in LDS once per workgroup (a lane
// reads its coefficients for column j as two 16-byte vectors, consecutive
// lanes on consecutive vectors), with a per-(column, row) parameter record
// (scale, zero, 1 / scale of the column's group, 1 / T[j][j]).  Coefficients
// and parameters are prefetched one column ahead.
constexpr int kSW = 4;                 // waves per workgroup
constexpr int kSRows = 4 * kSW;        // rows per workgroup
constexpr size_t kSweepLds = sizeof(float) * 128 * 128 + sizeof(f32x4) * 128 * kSRows;

struct RowState {
  float w[8];      // working values of the lane's columns
  float ev[8];     // errors (owner lanes)
  uint32_t cq[2];  // codes, 4 per word
  f32x4 t0, t1;    // T[j][4q..4q+3], T[j][64+4q..+3] of the next column
  f32x4 pc;        // scale, zero, 1 / scale, 1 / T[j][j] of the next column for this row
  float d;         // T[j][j] of the next column
};

// column j: registers 4 (j >= 64) + j % 4, owner lane (j % 64) / 4
template <int J>
__device__ __forceinline__ void r16_fetch(RowState& st, const float* Tl, const f32x4* pcol, int q, int rl) {
  const float* tr = Tl + J * 128;
  if constexpr (J < 64) st.t0 = *reinterpret_cast<const f32x4*>(tr + 4 * q);
  st.t1 = *reinterpret_cast<const f32x4*>(tr + 64 + 4 * q);
  st.pc = pcol[J * kSRows + rl];
  st.d = tr[J];
}

template <bool REF, int J>
__device__ __forceinline__ void r16_step(RowState& st, const float* Tl, const f32x4* pcol, int q, int rl,
                                         float fmaxq) {
  constexpr int m = (J >= 64 ? 4 : 0) + (J & 3), q0 = (J & 63) >> 2;
  const f32x4 t0 = st.t0, t1 = st.t1, pc = st.pc;
  const float d = st.d;
  if constexpr (J + 1 < 128) r16_fetch<J + 1>(st, Tl, pcol, q, rl);
  const float sc = pc[0], z = pc[1], is = pc[2], id = pc[3];
  const float wj = st.w[m];
  const float tq = div_rcp(wj, sc, is);
  float qv;
  if constexpr (REF)
    qv = fminf(fmaxf(rintf(tq + z), 0.0f), fmaxq);
  else
    qv = fminf(fmaxf(rintf(tq) + z, 0.0f), fmaxq);
  const float e = div_rcp(wj - sc * (qv - z), d, id);
  const float eb = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, e), 0x150 + q0, 0xF, 0xF,
                                                                      false));
  // registers 0-3 hold columns < 64 (dead once j >= 64); register m first
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = (m + i) & 7;
    if (J < 64 || r >= 4) st.w[r] = fmaf(-eb, r < 4 ? t0[r] : t1[r - 4], st.w[r]);
  }
  // pin the updates to this step (sunk to their next use they would keep
  // several steps' coefficients live)
#pragma unroll
  for (int r = 0; r < 8; ++r) asm volatile("" : "+v"(st.w[r]));
  const bool own = q == q0;
  st.ev[m] = own ? e : st.ev[m];
  st.cq[m >> 2] = own ? st.cq[m >> 2] | (static_cast<uint32_t>(qv) << (8 * (m & 3))) : st.cq[m >> 2];
  // one step after the other: the next column's loads are in flight, and
  // nothing later may be hoisted into this step
  __builtin_amdgcn_sched_barrier(0);
}

template <bool REF, int... J>
__device__ __forceinline__ void r16_steps(RowState& st, const float* Tl, const f32x4* pcol, int q, int rl, float fmaxq,
                                          std::integer_sequence<int, J...>) {
  (r16_step<REF, J>(st, Tl, pcol, q, rl, fmaxq), ...);
}

template <bool REF>
__global__ __launch_bounds__(64 * kSW) void sweep_r16(SubArgs a) {
  extern __shared__ float smem[];
  float* Tl = smem;                                          // [128][128] T sub-block, zeros outside
  f32x4* pcol = reinterpret_cast<f32x4*>(smem + 128 * 128);  // [128][kSRows]
  const int tid = threadIdx.x;
  const int q = tid & 15;
  const int rl = tid >> 4;  // row within the workgroup
  const int n = a.n;
  constexpr int kThr = 64 * kSW;

  // Stage T: 16 vector loads per thread in flight before any is stored.  The
  // loads are branch-free (an element outside the block loads the block's
  // first element and is replaced by zero): loads under divergent branches
  // were each waited for before the next one was issued.
  const float* tsrc = a.T + a.j1 * a.ldt + a.j1;
  const bool tvec = (n & 3) == 0 && (a.ldt & 3) == 0 && (reinterpret_cast<uintptr_t>(tsrc) & 15) == 0;
  {
    f32x4 v[16];
    if (tvec) {
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int e = tid + u * kThr, j = e >> 5, c = 4 * (e & 31);
        const bool ok = j < n && c < n;
        const f32x4 x = *reinterpret_cast<const f32x4*>(tsrc + (ok ? j * a.ldt + c : 0));
        v[u] = ok ? x : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
    } else {
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int e = tid + u * kThr, j = e >> 5, c = 4 * (e & 31);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool ok = j < n && c + i < n;
          const float x = tsrc[ok ? j * a.ldt + c + i : 0];
          v[u][i] = ok ? x : 0.0f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) reinterpret_cast<f32x4*>(Tl)[tid + u * kThr] = v[u];
  }
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kSRows;
  const int64_t row = row0 + rl;
  const int64_t rrow = row < a.rows ? row : a.rows - 1;
  // this lane's columns of W
  RowState st;
  {
    const float* src = a.W + rrow * a.cols + a.j1;
    const bool wvec = (n & 3) == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0;
    if (wvec) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = 64 * h + 4 * q;
        const f32x4 x = *reinterpret_cast<const f32x4*>(src + (c < n ? c : 0));
        const f32x4 v = c < n ? x : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < 4; ++u) st.w[4 * h + u] = v[u];
      }
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int c = 64 * h + 4 * q + u;
          const float x = src[c < n ? c : 0];
          st.w[4 * h + u] = c < n ? x : 0.0f;
        }
    }
  }
  __syncthreads();
  // With fuse (the sub-block is a whole block starting at a group boundary,
  // and the group size is 64 or 128): the min-max parameters of the
  // sub-block's groups (at most kFuseGroups) from the row's weights as they
  // stand now, over each lane's columns and then the row's 16 lanes, kept in
  // registers and written out; otherwise they come from sweep_params.
  float fs[kFuseGroups], fz[kFuseGroups];
#pragma unroll
  for (int gg = 0; gg < kFuseGroups; ++gg) {
    fs[gg] = 1.0f;
    fz[gg] = 0.0f;
  }
  if (a.fuse) {
#pragma unroll
    for (int gg = 0; gg < kFuseGroups; ++gg) {
      if (gg < a.G) {
        float mn = INFINITY, mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const int c = r < 4 ? 4 * q + r : 60 + 4 * q + r;
          const bool in = c < n && c / a.gs == gg;
          mn = in ? fminf(mn, st.w[r]) : mn;
          mx = in ? fmaxf(mx, st.w[r]) : mx;
        }
        mn = row16_reduce<false>(mn);
        mx = row16_reduce<true>(mx);
        group_params(mn, mx, a.maxq, a.ref != 0, fs[gg], fz[gg]);
        if (q == 0 && row < a.rows) {
          a.scale[row * a.ngroups + a.g_lo + gg] = fs[gg];
          a.zero[row * a.ngroups + a.g_lo + gg] = fz[gg];
        }
      }
    }
  }
  // the parameters of local group g (fuse)
  auto fused = [&](int g, float& sg, float& zg) {
    sg = fs[0];
    zg = fz[0];
#pragma unroll
    for (int gg = 1; gg < kFuseGroups; ++gg) {
      sg = g == gg ? fs[gg] : sg;
      zg = g == gg ? fz[gg] : zg;
    }
  };
  // parameter records: thread (rl, q) fills columns q, q + 16, ... of its row.
  // Columns past n get (1, 0, 1, 1): they change no live column (their T
  // rows are zero) and stay finite.
  {
    const int c0 = a.gs > 0 ? static_cast<int>(a.j1 - a.g_lo * a.gs) : 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int c = q + 16 * u;
      const int cc = c < n ? c : 0;  // branch-free loads, as for T
      const int g = a.gs > 0 ? (c0 + cc) / a.gs : 0;
      float sg, zg;
      if (a.fuse) {
        fused(g, sg, zg);
      } else {
        sg = a.scale[rrow * a.ngroups + a.g_lo + g];
        zg = a.zero[rrow * a.ngroups + a.g_lo + g];
      }
      const f32x4 r = f32x4{sg, zg, 1.0f / sg, 1.0f / Tl[c * 128 + c]};
      pcol[c * kSRows + rl] = c < n ? r : f32x4{1.0f, 0.0f, 1.0f, 1.0f};
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) st.ev[i] = 0.0f;
  st.cq[0] = st.cq[1] = 0u;
  __syncthreads();
  r16_fetch<0>(st, Tl, pcol, q, rl);
  r16_steps<REF>(st, Tl, pcol, q, rl, static_cast<float>(a.maxq), std::make_integer_sequence<int, 128>{});

  // row sums of squared errors: lane q's columns, then across the row's 16 lanes
  float esq = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if ((i < 4 ? 4 * q + i : 60 + 4 * q + i) < n) esq = fmaf(st.ev[i], st.ev[i], esq);
  esq += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, esq), 0xB1, 0xF, 0xF, false));
  esq += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, esq), 0x4E, 0xF, 0xF, false));
  esq += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, esq), 0x141, 0xF, 0xF, false));
  esq += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, esq), 0x140, 0xF, 0xF, false));
  if (row >= a.rows) return;
  if (a.err_sq && q == 0) a.err_sq[row] += esq;
  const int c0 = a.gs > 0 ? static_cast<int>(a.j1 - a.g_lo * a.gs) : 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = (i < 4 ? 0 : 64) + 4 * q + (i & 3);
    if (c < n) {
      const int64_t gc = a.j1 + c;
      const int64_t oc = a.out_cols ? a.out_cols[gc] : gc;
      const uint32_t code = (st.cq[i >> 2] >> (8 * (i & 3))) & 0xFFu;
      a.codes[row * a.cols + oc] = static_cast<uint8_t>(code);
      if (a.dq) {
        const int g = a.gs > 0 ? (c0 + c) / a.gs : 0;
        float sg, zg;
        if (a.fuse) {
          fused(g, sg, zg);
        } else {
          sg = a.scale[row * a.ngroups + a.g_lo + g];
          zg = a.zero[row * a.ngroups + a.g_lo + g];
        }
        store_elem(a.dq, row * a.cols + oc, a.dq_dtype, sg * (static_cast<float>(code) - zg));
      }
      if (a.losses) a.losses[row * a.cols + oc] = 0.5f * st.ev[i] * st.ev[i];
      if (a.Err) a.Err[row * a.lde + a.e_off + c] = st.ev[i];
    }
  }
}

// row[perm[c]] = row[c] in place, through LDS: the whole row is read before
// any of it is written.  Entries of perm outside [0, cols) are skipped.
constexpr int64_t kUnpermMaxCols = 16384;

// 8 columns per thread and pass, loads branch-free (out-of-range lanes read
// column 0 and are not stored), so that a thread's loads are in flight
// together
template <typename E>
__device__ __forceinline__ void unpermute_one(E* row, const int32_t* perm, int64_t cols, E* buf) {
  const int n = static_cast<int>(cols);
  constexpr int U = 8;
  for (int c = threadIdx.x; c < n; c += 256 * U) {
    uint32_t o[U];
    E v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int cc = c + 256 * u;
      const bool in = cc < n;
      o[u] = in ? static_cast<uint32_t>(perm[cc]) : 0xFFFFFFFFu;
      v[u] = row[in ? cc : 0];
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (o[u] < static_cast<uint32_t>(n)) buf[o[u]] = v[u];
  }
  __syncthreads();
  for (int c = threadIdx.x; c < n; c += 256 * U) {
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (c + 256 * u < n) row[c + 256 * u] = buf[c + 256 * u];
  }
  __syncthreads();
}

// one workgroup per row; esz = bytes per dequantised value (0: none)
__global__ __launch_bounds__(256) void unpermute_rows(uint8_t* __restrict__ codes, void* __restrict__ dq, int esz,
                                                      float* __restrict__ losses, const int32_t* __restrict__ perm,
                                                      int64_t cols) {
  extern __shared__ float ubuf[];
  const int64_t r = blockIdx.x;
  unpermute_one(codes + r * cols, perm, cols, reinterpret_cast<uint8_t*>(ubuf));
  if (esz == 4) unpermute_one(static_cast<float*>(dq) + r * cols, perm, cols, ubuf);
  if (esz == 2) unpermute_one(static_cast<uint16_t*>(dq) + r * cols, perm, cols, reinterpret_cast<uint16_t*>(ubuf));
  if (losses) unpermute_one(losses + r * cols, perm, cols, ubuf);
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
  // rows over blockIdx.y, columns over threads: no 64-bit division per element
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y)
    for (int64_t c = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; c < cols;
         c += static_cast<int64_t>(gridDim.x) * blockDim.x) {
      const int64_t pc = perm ? perm[c] : c;
      float v = load_elem(w, transpose ? pc * ldw + r : r * ldw + pc, dtype);
      if (dead && dead[pc]) v = 0.0f;
      out[r * cols + c] = v;
    }
}

// Row-major weights with at most kPrepLdsCols columns: one workgroup per row
// copies the row's raw elements into LDS (16-byte loads when rows are 16-byte
// aligned) and writes it out in sweep order as fp32 (the column gather reads
// LDS; 16-byte stores), with the dead columns as a bit mask in LDS staged once
// per workgroup.  The element-wise kernel above gathers every element from
// global memory: 358 against 130 us for a 4096 x 14336 bf16 weight with a
// column order and dead flags on MI355X (14336 x 4096: 258 against 127 us).
constexpr int64_t kPrepLdsCols = 32768;

__global__ __launch_bounds__(512) void prepare_rows_k(const void* __restrict__ w, int dtype, int64_t rows,
                                                      int64_t cols, int64_t ldw, const int32_t* __restrict__ perm,
                                                      const int32_t* __restrict__ dead, int vec_in,
                                                      int vec_out, float* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) uint32_t sprep[];
  const int esz = dtype == GPTQ_F32 ? 4 : 2;
  const int ncol = static_cast<int>(cols);
  const int row_words = (ncol * esz + 15) / 16 * 4;  // the row, padded to 16 bytes
  uint32_t* mask = sprep + row_words;                // bit c: column c is dead
  if (dead) {
    // one 64-column ballot per wave step (coalesced reads of the flags)
    const int lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    const int nmask = (ncol + 31) / 32;
    for (int c0 = 64 * (threadIdx.x >> 6); c0 < ncol; c0 += 64 * nw) {
      const int c = c0 + lane;
      const uint64_t m = __ballot(c < ncol && dead[c] != 0);
      if (lane == 0) {
        mask[c0 / 32] = static_cast<uint32_t>(m);
        if (c0 / 32 + 1 < nmask) mask[c0 / 32 + 1] = static_cast<uint32_t>(m >> 32);
      }
    }
  }
  const uint8_t* base = static_cast<const uint8_t*>(w);
  uint8_t* srow = reinterpret_cast<uint8_t*>(sprep);
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const uint8_t* src = base + r * ldw * esz;
    if (vec_in) {
      for (int o = 16 * threadIdx.x; o < ncol * esz; o += 16 * blockDim.x)
        *reinterpret_cast<uint4*>(srow + o) = *reinterpret_cast<const uint4*>(src + o);
    } else if (esz == 2) {
      for (int c = threadIdx.x; c < ncol; c += blockDim.x)
        reinterpret_cast<uint16_t*>(srow)[c] = reinterpret_cast<const uint16_t*>(src)[c];
    } else {
      for (int c = threadIdx.x; c < ncol; c += blockDim.x)
        reinterpret_cast<uint32_t*>(srow)[c] = reinterpret_cast<const uint32_t*>(src)[c];
    }
    __syncthreads();
    auto value = [&](int c) {
      const int pc = perm ? perm[c] : c;
      const int off = pc * esz;
      const float v = elem_value(sprep[off >> 2], (off & 2) != 0, dtype);
      return (dead && ((mask[pc >> 5] >> (pc & 31)) & 1u)) ? 0.0f : v;
    };
    float* dst = out + r * cols;
    if (vec_out) {
      for (int c = 4 * threadIdx.x; c < ncol; c += 4 * blockDim.x)
        *reinterpret_cast<f32x4*>(dst + c) = f32x4{value(c), value(c + 1), value(c + 2), value(c + 3)};
    } else {
      for (int c = threadIdx.x; c < ncol; c += blockDim.x) dst[c] = value(c);
    }
    __syncthreads();
  }
}

int launch_r16(hipStream_t st, const SubArgs& a) {
  const unsigned blocks = static_cast<unsigned>(cdiv(a.rows, kSRows));
  if (a.ref)
    hipLaunchKernelGGL(sweep_r16<true>, dim3(blocks), dim3(64 * kSW), kSweepLds, st, a);
  else
    hipLaunchKernelGGL(sweep_r16<false>, dim3(blocks), dim3(64 * kSW), kSweepLds, st, a);
  return check_launch("sweep_r16");
}

}  // namespace
}  // namespace gptq

using namespace gptq;

// Trailing updates are batched two-level: each sub-block updates the rest of
// its run of blocks spanning >= plan::kSweepRun columns right away (the columns swept
// next), and the run's errors update everything after it in one GEMM of
// depth >= plan::kSweepRun at the run's end.  Errors of a run are kept side by side.
// (plan::kSweepRun = 512 columns, plan::sweep_run_blocks; the workspace
// size is gptq_sweep_workspace_size in plan.cpp)
static_assert(plan::kSweepSub == kSub, "the sweep workspace size assumes this sub-block width");

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
  if (!transpose && cols <= kPrepLdsCols) {
    const int esz = dtype_size(dtype);
    // 16-byte loads cover whole rows only: aligned start, pitch and length
    const int vec_in = reinterpret_cast<uintptr_t>(w) % 16 == 0 && (ldw * esz) % 16 == 0 && (cols * esz) % 16 == 0;
    const int vec_out = reinterpret_cast<uintptr_t>(out) % 16 == 0 && cols % 4 == 0;
    const size_t lds = static_cast<size_t>(cdiv(cols * esz, 16)) * 16 + static_cast<size_t>(cdiv(cols, 32)) * 4;
    hipLaunchKernelGGL(prepare_rows_k, dim3(static_cast<unsigned>(std::min<int64_t>(rows, 1 << 20))), dim3(512), lds,
                       as_hip(stream), w, dtype, rows, cols, ldw, perm, dead_cols, vec_in, vec_out, out);
    return check_launch("prepare_weight");
  }
  const dim3 grid(static_cast<unsigned>(std::min<int64_t>(cdiv(cols, 256), 64)),
                  static_cast<unsigned>(std::min<int64_t>(rows, 65535)));
  hipLaunchKernelGGL(prepare_weight_k, grid, dim3(256), 0, as_hip(stream), w, dtype, rows, cols, ldw, perm,
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
  // Blocks of one 128-column sub-block whose groups (64 or 128 columns) all
  // start and end inside them take their groups' parameters from W as
  // sweep_r16 loads it (the values sweep_params would read), in the sweep
  // kernel itself: one launch less per block (measured on MI355X: 4096 x 14336
  // sweep 11.18 -> 10.80 ms, 14336 x 4096 4.83 -> 4.56 ms, results
  // bit-identical; with 16- or 32-column groups the in-kernel reduction over
  // up to 8 groups cost more than the launch).
  const bool fuse = gs >= kSub / kFuseGroups && kSub % gs == 0 && blocksize == kSub &&
                    !(flags & GPTQ_SWEEP_GROUPS_FROM_W0);
  float* Err = static_cast<float*>(workspace);
  int rc;
  if (err_sq) {
    hipLaunchKernelGGL(fill_zero_f, dim3(static_cast<unsigned>(std::min<int64_t>(cdiv(rows, 256), 65536))), dim3(256),
                       0, st, err_sq, rows);
    if ((rc = check_launch("fill_zero"))) return rc;
  }
  // With a column order, codes / dequantised values / losses are written in
  // sweep order and put in place by one pass per row at the end (scattered
  // writes from every sub-block would each touch their own cache line).
  const bool defer = out_cols != nullptr && cols <= kUnpermMaxCols;
  // without the trailing update every block stands alone (one Err slot)
  const int64_t F = trailing ? plan::sweep_run_blocks(blocksize) : 1;
  const int64_t lde = trailing ? std::max<int64_t>(kSub, F * blocksize) : kSub;
  for (int64_t s1 = 0; s1 < cols; s1 += F * blocksize) {
    const int64_t s2 = std::min<int64_t>(s1 + F * blocksize, cols);
    for (int64_t i1 = s1; i1 < s2; i1 += blocksize) {
      const int64_t i2 = std::min<int64_t>(i1 + blocksize, cols);
      if (gs > 0 && !fuse) {
        const int64_t g_first = cdiv(i1, gs);
        const int64_t g_end = cdiv(i2, gs);  // groups whose start lies in [i1, i2)
        if (g_end > g_first) {
          const int64_t g_count = g_end - g_first;
          const unsigned blocks = static_cast<unsigned>(cdiv(rows * g_count, 4));
          hipLaunchKernelGGL(sweep_params, dim3(blocks), dim3(256), 0, st, psrc, cols, rows, cols, gs, maxq,
                             ref ? 1 : 0, g_first, g_count, scale, zero, ngroups);
          if ((rc = check_launch("sweep_params"))) return rc;
        }
      }
      for (int64_t j1 = i1; j1 < i2; j1 += kSub) {
        const int64_t j2 = std::min<int64_t>(j1 + kSub, i2);
        const int n = static_cast<int>(j2 - j1);
        const int64_t e_off = trailing ? j1 - s1 : 0;
        SubArgs a;
        a.W = W; a.T = T; a.ldt = ldt; a.cols = cols; a.rows = rows; a.j1 = j1; a.n = n; a.gs = gs; a.maxq = maxq;
        a.ref = ref ? 1 : 0; a.scale = scale; a.zero = zero; a.ngroups = ngroups;
        a.g_lo = gs > 0 ? j1 / gs : 0;
        a.G = gs > 0 ? static_cast<int>((j2 - 1) / gs - j1 / gs + 1) : 1;
        a.fuse = fuse ? 1 : 0;
        a.out_cols = defer ? nullptr : out_cols; a.codes = codes; a.dq = dequant; a.dq_dtype = dequant_dtype;
        a.err_sq = err_sq; a.losses = losses; a.Err = Err; a.lde = lde; a.e_off = e_off;
        if ((rc = launch_r16(st, a))) return rc;
        // the columns swept next: the rest of the run (trailing) or of the block
        const int64_t end = trailing ? s2 : i2;
        if (j2 < end) {
          rc = launch_gemm_f32(st, rows, end - j2, n, -1.0f, Err + e_off, lde, false, T + j1 * ldt + j2, ldt, false,
                               1.0f, W + j2, cols, 0);
          if (rc) return rc;
        }
      }
    }
    // the run's errors, all at once, into every later column
    if (trailing && s2 < cols) {
      rc = launch_gemm_f32(st, rows, cols - s2, s2 - s1, -1.0f, Err, lde, false, T + s1 * ldt + s2, ldt, false, 1.0f,
                           W + s2, cols, 0);
      if (rc) return rc;
    }
  }
  if (defer) {
    hipLaunchKernelGGL(unpermute_rows, dim3(static_cast<unsigned>(rows)), dim3(256), sizeof(float) * cols, st, codes,
                       dequant, dequant ? dtype_size(dequant_dtype) : 0, losses, out_cols, cols);
    if ((rc = check_launch("unpermute_rows"))) return rc;
  }
  return GPTQ_OK;
}
