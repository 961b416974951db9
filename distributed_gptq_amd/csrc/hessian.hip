// Hessian accumulation H += X^T X on gfx950 MFMA (one triangle).
//
// Work decomposition
//   * H is cut into 256 x 256 tiles; only tiles (I, J) with J <= I are
//     computed.  A tile is one workgroup of 8 waves in a 2 x 4 grid, each
//     wave owning a 128 x 64 block = 4 x 2 MFMA 32x32 blocks (128 fp32
//     accumulators per lane).
//   * The tokens are cut into S contiguous splits.  Workgroup b works on
//     split b % S of tile b / S; since consecutive workgroups are dispatched
//     round-robin over the 8 XCDs and S is a multiple of 8, every XCD streams
//     its own token range of X exactly once through its L2.
//   * Each (split, tile) writes an fp32 partial tile to the workspace; a
//     reduce kernel adds the S partials in fixed order (deterministic) to the
//     lower triangle of H and mirrors them to the upper triangle.
//
// Operands.  The Gram matrix needs, per lane, 8 consecutive tokens of one
// feature (the k-run of v_mfma_f32_32x32x16_{bf16,f16}); X is stored token-
// major, so every thread loads an 8 token x 8 feature block with eight
// 128-bit loads, transposes it in registers and writes eight 128-bit feature
// runs to LDS.  The LDS slot of feature f is f ^ ((f >> 4) & 15), which keeps
// both the transposed writes and the MFMA-fragment reads free of 16-byte
// bank-group collisions.  fp32 inputs use v_mfma_f32_32x32x2_f32 with a
// token-major LDS tile (no transpose needed).
#include "common.hpp"

namespace gptq {
namespace {

constexpr int kTile = 256;
constexpr int kThreads = 512;
constexpr int kWaveRows = 128;
constexpr int kWaveCols = 64;

__device__ __forceinline__ void tile_coords(int t, int& I, int& J) {
  int i = static_cast<int>((sqrtf(8.0f * static_cast<float>(t) + 1.0f) - 1.0f) * 0.5f);
  while ((i + 1) * (i + 2) / 2 <= t) ++i;
  while (i * (i + 1) / 2 > t) --i;
  I = i;
  J = t - i * (i + 1) / 2;
}

__device__ __forceinline__ int swz(int f) { return f ^ ((f >> 4) & 15); }

// ------------------------------------------------------- 16-bit inputs ----
// LDS: [buffer][operand][token-octet (8)][slot (256)] x 16 B  (8 tokens of a feature)
// 64 tokens per stage; 512 loader threads = 2 operands x 8 token-octets x 32
// feature-octets, one 8x8 block each.
template <bool kBF16, bool kVec>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void hessian_tile16(const uint16_t* __restrict__ X, int64_t n, int K, int64_t ldx,
                    int S, int64_t tok_per_split, int ntiles, float* __restrict__ partial) {
  constexpr int kBK = 64;
  __shared__ u32x4 lds[2][2][kBK / 8][kTile];  // [buffer][operand][token-octet][slot]

  const int s = blockIdx.x % S;
  const int tile = blockIdx.x / S;
  int I, J;
  tile_coords(tile, I, J);
  const bool diag = (I == J);
  const int64_t t_begin = static_cast<int64_t>(s) * tok_per_split;
  const int64_t t_end = min(n, t_begin + tok_per_split);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 2) * kWaveRows;
  const int wn = (wave & 3) * kWaveCols;
  // waves whose block lies strictly above the diagonal of a diagonal tile
  const bool wave_idle = diag && (wn >= wm + kWaveRows);

  // loader role
  const int op = tid >> 8;
  const int fo = tid & 31;
  const int to = (tid >> 5) & 7;
  const bool loader = !(diag && op == 1);
  const int feat0 = (op == 0 ? I : J) * kTile + fo * 8;

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  u32x4 pre[8];
  auto load_stage = [&](int64_t t0) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int64_t tok = t0 + to * 8 + r;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (loader && tok < t_end && feat0 < K) {
        const uint16_t* src = X + tok * ldx + feat0;
        if constexpr (kVec) {
          v = *reinterpret_cast<const u32x4*>(src);
        } else {
          uint32_t h[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) h[e] = (feat0 + e < K) ? src[e] : 0u;
          v = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
        }
      }
      pre[r] = v;
    }
  };
  auto store_stage = [&](int bsel) {
    if (!loader) return;
#pragma unroll
    for (int f = 0; f < 8; ++f) {
      u32x4 o;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint32_t a = pre[2 * d][f >> 1];
        const uint32_t b = pre[2 * d + 1][f >> 1];
        o[d] = (f & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
      }
      lds[bsel][op][to][swz(fo * 8 + f)] = o;
    }
  };

  // LDS ping-pong: stage s is multiplied out of buffer s & 1 while stage s + 1
  // is written to the other buffer and stage s + 2 is being fetched; one
  // barrier per stage.
  const int bop = diag ? 0 : 1;
  int buf = 0;
  if (t_begin < t_end) {
    load_stage(t_begin);
    store_stage(0);
    if (t_begin + kBK < t_end) load_stage(t_begin + kBK);
  }
  __syncthreads();
  for (int64_t t0 = t_begin; t0 < t_end; t0 += kBK) {
    if (!wave_idle) {
#pragma unroll
      for (int ks = 0; ks < kBK / 16; ++ks) {
        const int tko = ks * 2 + (lane >> 5);
        u32x4 a[4], b[2];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = lds[buf][0][tko][swz(wm + i * 32 + (lane & 31))];
#pragma unroll
        for (int j = 0; j < 2; ++j) b[j] = lds[buf][bop][tko][swz(wn + j * 32 + (lane & 31))];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            if constexpr (kBF16) {
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                  __builtin_bit_cast(bf16x8, a[i]), __builtin_bit_cast(bf16x8, b[j]), acc[i][j], 0, 0, 0);
            } else {
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                  __builtin_bit_cast(f16x8, a[i]), __builtin_bit_cast(f16x8, b[j]), acc[i][j], 0, 0, 0);
            }
          }
      }
    }
    if (t0 + kBK < t_end) {
      store_stage(buf ^ 1);
      if (t0 + 2 * kBK < t_end) load_stage(t0 + 2 * kBK);
    }
    __syncthreads();
    buf ^= 1;
  }

  // 32x32 accumulator layout: lane l, register v -> row 8*(v/4) + 4*(l/32) + v%4, col l%32
  if (wave_idle) return;
  float* out = partial + (static_cast<int64_t>(s) * ntiles + tile) * (kTile * kTile);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = wm + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        const int col = wn + j * 32 + (lane & 31);
        out[row * kTile + col] = acc[i][j][v];
      }
}

// --------------------------------------------------------- fp32 inputs ----
// LDS: [operand][token (16)][feature (256)] fp32; lane l of a
// v_mfma_f32_32x32x2_f32 takes token l/32 of feature l%32.
template <bool kVec>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void hessian_tile32(const float* __restrict__ X, int64_t n, int K, int64_t ldx, int S,
                    int64_t tok_per_split, int ntiles, float* __restrict__ partial) {
  constexpr int kBK = 16;
  __shared__ f32x4 lds[2][kBK][kTile / 4];

  const int s = blockIdx.x % S;
  const int tile = blockIdx.x / S;
  int I, J;
  tile_coords(tile, I, J);
  const bool diag = (I == J);
  const int64_t t_begin = static_cast<int64_t>(s) * tok_per_split;
  const int64_t t_end = min(n, t_begin + tok_per_split);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 2) * kWaveRows;
  const int wn = (wave & 3) * kWaveCols;
  const bool wave_idle = diag && (wn >= wm + kWaveRows);

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // per stage: 2 operands x 16 tokens x 64 float4 = 2048 float4, 4 per thread
  constexpr int kPer = 2 * kBK * (kTile / 4) / kThreads;
  f32x4 pre[kPer];
  auto load_stage = [&](int64_t t0) {
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int idx = q * kThreads + tid;
      const int op = idx >> 10;
      const int tok_l = (idx >> 6) & 15;
      const int f4 = idx & 63;
      const int64_t tok = t0 + tok_l;
      const int feat = (op == 0 ? I : J) * kTile + f4 * 4;
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (!(diag && op == 1) && tok < t_end && feat < K) {
        const float* src = X + tok * ldx + feat;
        if constexpr (kVec) {
          v = *reinterpret_cast<const f32x4*>(src);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (feat + e < K) ? src[e] : 0.0f;
        }
      }
      pre[q] = v;
    }
  };
  auto store_stage = [&]() {
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int idx = q * kThreads + tid;
      const int op = idx >> 10;
      if (diag && op == 1) continue;
      lds[op][(idx >> 6) & 15][idx & 63] = pre[q];
    }
  };

  const int bop = diag ? 0 : 1;
  const float* ldsf = reinterpret_cast<const float*>(&lds[0][0][0]);
  if (t_begin < t_end) load_stage(t_begin);
  for (int64_t t0 = t_begin; t0 < t_end; t0 += kBK) {
    __syncthreads();
    store_stage();
    __syncthreads();
    if (t0 + kBK < t_end) load_stage(t0 + kBK);
    if (!wave_idle) {
#pragma unroll
      for (int kk = 0; kk < kBK / 2; ++kk) {
        const int tok = kk * 2 + (lane >> 5);
        float a[4], b[2];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = ldsf[(0 * kBK + tok) * kTile + wm + i * 32 + (lane & 31)];
#pragma unroll
        for (int j = 0; j < 2; ++j) b[j] = ldsf[(bop * kBK + tok) * kTile + wn + j * 32 + (lane & 31)];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
      }
    }
  }

  if (wave_idle) return;
  float* out = partial + (static_cast<int64_t>(s) * ntiles + tile) * (kTile * kTile);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = wm + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        const int col = wn + j * 32 + (lane & 31);
        out[row * kTile + col] = acc[i][j][v];
      }
}

// ------------------------------------------------------------- reduce ----
// One workgroup per 32 x 32 sub-block of a lower tile.  H[gi][gj] (gi >= gj
// within diagonal sub-blocks) += sum_s partial[s]; the sum is mirrored to
// H[gj][gi] through an LDS transpose so H stays exactly symmetric.
__global__ __launch_bounds__(256) void hessian_reduce(float* __restrict__ H, int K, const float* __restrict__ partial,
                                                      int S, int ntiles) {
  __shared__ float t[32][33];
  const int tile = blockIdx.x >> 6;
  const int sb = blockIdx.x & 63;
  const int sr = sb >> 3, sc = sb & 7;
  int I, J;
  tile_coords(tile, I, J);
  if (I == J && sc > sr) return;
  const bool diag_sb = (I == J) && (sr == sc);
  const int tid = threadIdx.x;
  const int row = tid >> 3;
  const int col0 = (tid & 7) * 4;
  const int64_t gi = static_cast<int64_t>(I) * kTile + sr * 32 + row;
  const int64_t tstride = static_cast<int64_t>(ntiles) * kTile * kTile;
  const float* p = partial + static_cast<int64_t>(tile) * kTile * kTile + (sr * 32 + row) * kTile + sc * 32 + col0;
  f32x4 v = *reinterpret_cast<const f32x4*>(p);
  for (int s = 1; s < S; ++s) {
    const f32x4 w = *reinterpret_cast<const f32x4*>(p + s * tstride);
    v += w;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t gj = static_cast<int64_t>(J) * kTile + sc * 32 + col0 + e;
    float val = v[e];
    if (gi < K && gj < K) {
      val += H[gi * K + gj];
      if (!diag_sb || gi >= gj) H[gi * K + gj] = val;
    }
    t[row][col0 + e] = val;
  }
  __syncthreads();
  // mirror: H[J*256 + sc*32 + r][I*256 + sr*32 + c] = t[c][r]
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int r = row;            // row of the mirrored block (column of t)
    const int c = col0 + e;       // column of the mirrored block (row of t)
    const int64_t mi = static_cast<int64_t>(J) * kTile + sc * 32 + r;
    const int64_t mj = static_cast<int64_t>(I) * kTile + sr * 32 + c;
    // source element is (gi', gj') = (mj, mi); mirror strictly-lower sources only
    if (mi < K && mj < K && (!diag_sb || mj > mi)) H[mi * K + mj] = t[c][r];
  }
}

int choose_splits(int64_t n, int ntiles) {
  constexpr int kTargetWG = 2048;  // ~8 workgroups per CU on 256 CUs
  int64_t s = 8 * cdiv(kTargetWG, 8LL * ntiles);
  s = std::min<int64_t>(s, 64);
  // keep at least 512 tokens per split
  s = std::min<int64_t>(s, std::max<int64_t>(1, n / 512));
  if (s >= 8) s -= s % 8;
  return static_cast<int>(std::max<int64_t>(s, 1));
}

}  // namespace
}  // namespace gptq

using namespace gptq;

extern "C" size_t gptq_hessian_workspace_size(int64_t n, int64_t K) {
  if (n <= 0 || K <= 0) return 0;
  const int64_t T = cdiv(K, kTile);
  const int ntiles = static_cast<int>(T * (T + 1) / 2);
  const int S = choose_splits(n, ntiles);
  return static_cast<size_t>(S) * ntiles * kTile * kTile * sizeof(float);
}

extern "C" int gptq_hessian_accumulate(float* H, const void* X, int64_t n, int64_t K, int64_t ldx, int dtype,
                                       void* workspace, size_t workspace_bytes, gptq_stream_t stream) {
  clear_error();
  GPTQ_REQUIRE(H && (X || n == 0), GPTQ_ERR_ARG, "hessian_accumulate: null pointer");
  GPTQ_REQUIRE(K > 0 && K <= (1 << 20) && n >= 0 && ldx >= K, GPTQ_ERR_SHAPE,
               "hessian_accumulate: bad shape n=%lld K=%lld ldx=%lld", (long long)n, (long long)K, (long long)ldx);
  GPTQ_REQUIRE(valid_dtype(dtype), GPTQ_ERR_DTYPE, "hessian_accumulate: bad dtype %d", dtype);
  if (n == 0) return GPTQ_OK;
  const int64_t T = cdiv(K, kTile);
  const int ntiles = static_cast<int>(T * (T + 1) / 2);
  const int S = choose_splits(n, ntiles);
  const size_t need = static_cast<size_t>(S) * ntiles * kTile * kTile * sizeof(float);
  GPTQ_REQUIRE(workspace && workspace_bytes >= need, GPTQ_ERR_WORKSPACE,
               "hessian_accumulate: workspace %zu < %zu bytes", workspace_bytes, need);
  const int64_t per = cdiv(cdiv(n, S), 32) * 32;
  float* part = static_cast<float*>(workspace);
  hipStream_t st = as_hip(stream);
  const dim3 grid(static_cast<unsigned>(S) * ntiles);
  const int esz = dtype_size(dtype);
  const bool vec = (ldx * esz) % 16 == 0 && (reinterpret_cast<uintptr_t>(X) % 16) == 0 && (K * esz) % 16 == 0;
  if (dtype == GPTQ_F32) {
    const float* x = static_cast<const float*>(X);
    if (vec)
      hipLaunchKernelGGL((hessian_tile32<true>), grid, dim3(kThreads), 0, st, x, n, (int)K, ldx, S, per, ntiles, part);
    else
      hipLaunchKernelGGL((hessian_tile32<false>), grid, dim3(kThreads), 0, st, x, n, (int)K, ldx, S, per, ntiles, part);
  } else {
    const uint16_t* x = static_cast<const uint16_t*>(X);
    if (dtype == GPTQ_BF16) {
      if (vec)
        hipLaunchKernelGGL((hessian_tile16<true, true>), grid, dim3(kThreads), 0, st, x, n, (int)K, ldx, S, per, ntiles, part);
      else
        hipLaunchKernelGGL((hessian_tile16<true, false>), grid, dim3(kThreads), 0, st, x, n, (int)K, ldx, S, per, ntiles, part);
    } else {
      if (vec)
        hipLaunchKernelGGL((hessian_tile16<false, true>), grid, dim3(kThreads), 0, st, x, n, (int)K, ldx, S, per, ntiles, part);
      else
        hipLaunchKernelGGL((hessian_tile16<false, false>), grid, dim3(kThreads), 0, st, x, n, (int)K, ldx, S, per, ntiles, part);
    }
  }
  int rc = check_launch("hessian_tile");
  if (rc) return rc;
  hipLaunchKernelGGL(hessian_reduce, dim3(static_cast<unsigned>(ntiles) * 64), dim3(256), 0, st, H, (int)K, part, S, ntiles);
  return check_launch("hessian_reduce");
}
