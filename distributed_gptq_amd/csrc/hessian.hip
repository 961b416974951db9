// Hessian accumulation H += X^T X on gfx950 MFMA (one triangle).
//
// Work decomposition
//   * H is cut into 256 x 256 tiles; only tiles (I, J) with J <= I are
//     computed.  A tile is one workgroup of 8 waves in a 2 x 4 grid, each
//     wave owning a 128 x 64 block = 4 x 2 MFMA 32x32 blocks (128 fp32
//     accumulators per lane).
//   * The tokens are cut into S contiguous splits (choose_splits: at most
//     16384 tokens each).  Workgroup b works on the (split, tile) pair that
//     split_tile maps it to: split-major, tiles in band order, each round of
//     256 workgroups permuted so that every XCD runs 32 neighbouring tiles.
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
#include <type_traits>

#include "common.hpp"

namespace gptq {
namespace {

constexpr int kTile = 256;
constexpr int kThreads = 512;
constexpr int kWaveRows = 128;
constexpr int kWaveCols = 64;

__host__ __device__ __forceinline__ void tile_coords(int t, int& I, int& J) {
  int i = static_cast<int>((sqrtf(8.0f * static_cast<float>(t) + 1.0f) - 1.0f) * 0.5f);
  while ((i + 1) * (i + 2) / 2 <= t) ++i;
  while (i * (i + 1) / 2 > t) --i;
  I = i;
  J = t - i * (i + 1) / 2;
}

// Tile t of the lower triangle (I >= J) of a T x T tile grid in band order:
// bands of 4 tile rows, each walked column by column (4 tiles per column left
// of the diagonal, then the band's own triangle), so that 32 consecutive
// tiles span 4 row panels and 8 column panels of X.  Bands before band c
// hold 8c^2 + 2c tiles (only the last band can have fewer than 4 rows).
__host__ __device__ __forceinline__ void band_coords(int t, int T, int& I, int& J) {
  int c = static_cast<int>((sqrtf(32.0f * static_cast<float>(t) + 4.0f) - 2.0f) * 0.0625f);
  while (8 * (c + 1) * (c + 1) + 2 * (c + 1) <= t) ++c;
  while (8 * c * c + 2 * c > t) --c;
  const int r0 = 4 * c, h = (T - r0 < 4) ? T - r0 : 4;
  int u = t - (8 * c * c + 2 * c);
  if (u < r0 * h) {
    J = u / h;
    I = r0 + u % h;
    return;
  }
  u -= r0 * h;
  int k = 0, len = h;
  while (u >= len) {
    u -= len;
    ++k;
    --len;
  }
  J = r0 + k;
  I = r0 + k + u;
}

// LDS slot of feature f: bits 0-2 are XORed with bits 4-6 and with bit 3
// moved to bit 2.  MFMA-fragment reads take 8 or 16 consecutive slots per LDS
// pass and the transposed stores take slots 8 apart (one per feature-octet);
// both land on distinct 16-byte bank groups whether a pass serves 8 lanes
// (32 banks) or 16 lanes (64 banks).
__device__ __forceinline__ int swz(int f) { return f ^ (((f >> 4) ^ ((f >> 1) & 4)) & 7); }

// Workgroup b -> (split, tile).  Workgroups are dispatched round-robin over
// the 8 XCDs, so XCD x runs b = x, x + 8, ...; with S a multiple of 8 it
// walks every tile of split x, then of split x + 8, ...: the workgroups
// resident on one XCD at a time share one token range and neighbouring
// feature blocks, which its L2 then serves.
template <int kMap = 0>
__host__ __device__ __forceinline__ void split_tile(int b, int S, int ntiles, int& s, int& tile) {
  if (kMap == 1) {  // split-major: all XCDs on the same split
    s = b / ntiles;
    tile = b % ntiles;
    return;
  }
  if (kMap == 2) {
    // split-major over band-ordered tiles, with every round of 256
    // workgroups (8 XCDs x 32 CUs) permuted so that XCD x runs 32 consecutive
    // entries of that order: b = 8q + x -> entry 32 (8 (q / 32) + x) + q % 32.
    // The last partial round keeps b itself.
    int idx = b;
    if (b < ((S * ntiles) & ~255)) {
      const int x = b & 7, q = b >> 3;
      idx = (((q >> 5) << 3) + x) * 32 + (q & 31);
    }
    s = idx / ntiles;
    tile = idx % ntiles;
    return;
  }
  if (S % 8 == 0) {
    const int x = b & 7, q = b >> 3;
    s = x + 8 * (q / ntiles);
    tile = q % ntiles;
  } else {
    s = b % S;
    tile = b / S;
  }
}

// ------------------------------------------------------- 16-bit inputs ----
// One workgroup of 4 waves (one per SIMD) per (split, tile); wave w owns the
// 128 x 128 block (w / 2, w % 2) of the 256 x 256 tile as 4 x 4 MFMA 32x32
// blocks, 256 fp32 accumulators per lane (AGPRs).  Per 16 tokens a wave
// reads 8 fragments from LDS for 16 MFMAs.
// LDS: [buffer][operand][token-octet (8)][slot (256)] x 16 B  (8 tokens of a feature)
// 64 tokens per stage; each of the 256 threads loads and transposes the 8x8
// (token x feature) block (to, fo) of both operands.
constexpr int kThreads16 = 256;

template <bool kBF16, bool kVec>
__global__ __launch_bounds__(kThreads16) __attribute__((amdgpu_waves_per_eu(1, 1)))
void hessian_tile16(const uint16_t* __restrict__ X, int64_t n, int K, int64_t ldx,
                    int S, int64_t tok_per_split, int ntiles, float* __restrict__ partial) {
  constexpr int kBK = 64;
  __shared__ u32x4 lds[2][2][kBK / 8][kTile];  // [buffer][operand][token-octet][slot]

  int s, tile;
  split_tile(blockIdx.x, S, ntiles, s, tile);
  int I, J;
  tile_coords(tile, I, J);
  const bool diag = (I == J);
  const int64_t t_begin = static_cast<int64_t>(s) * tok_per_split;
  const int64_t t_end = min(n, t_begin + tok_per_split);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 1) * 128;
  const int wn = (wave & 1) * 128;
  // the wave above the diagonal of a diagonal tile has nothing to do
  const bool wave_idle = diag && (wn > wm);

  // loader role: token-octet `to`, feature-octet `fo`, both operands
  const int fo = tid & 31;
  const int to = tid >> 5;
  const int nops = diag ? 1 : 2;

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // 8 rows of 16 bytes per operand: with 16-byte aligned rows they are
  // buffer loads from a per-stage descriptor (row offsets in one vector
  // register; tokens past the split read zeros); otherwise element loads
  const int64_t rowb = ldx * 2;
  uint32_t voff[2];
  bool fok[2];
#pragma unroll
  for (int op = 0; op < 2; ++op) {
    fok[op] = (op == 0 ? I : J) * kTile + fo * 8 < K;
    voff[op] = fok[op] ? static_cast<uint32_t>(to * 8 * rowb + fo * 16) : 0x80000000u;
  }
  u32x4 pre[2][8];
  auto load_stage = [&](int64_t t0) {
#pragma unroll
    for (int op = 0; op < 2; ++op) {
      const int fblk = (op == 0 ? I : J) * kTile;
      if constexpr (kVec) {
        const int64_t left = t_end - t0;  // rows of this stage that exist (the stage reads at most kBK)
        const uint32_t nrec = static_cast<uint32_t>((left < kBK ? left : kBK) * rowb);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(X + t0 * ldx + fblk), static_cast<short>(0), static_cast<int>(op < nops ? nrec : 0u),
            0x00020000);
#pragma unroll
        for (int r = 0; r < 8; ++r)
          pre[op][r] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff[op] + static_cast<uint32_t>(r * rowb), 0, 0);
      } else {
        const int feat0 = fblk + fo * 8;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const int64_t tok = t0 + to * 8 + r;
          u32x4 v = {0u, 0u, 0u, 0u};
          if (op < nops && tok < t_end && feat0 < K) {
            const uint16_t* src = X + tok * ldx + feat0;
            uint32_t h[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = (feat0 + e < K) ? src[e] : 0u;
            v = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
          }
          pre[op][r] = v;
        }
      }
    }
  };
  auto store_stage = [&](int bsel) {
#pragma unroll
    for (int op = 0; op < 2; ++op) {
      if (op >= nops) break;
#pragma unroll
      for (int f = 0; f < 8; ++f) {
        u32x4 o;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t a = pre[op][2 * d][f >> 1];
          const uint32_t b = pre[op][2 * d + 1][f >> 1];
          o[d] = (f & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
        }
        lds[bsel][op][to][swz(fo * 8 + f)] = o;
      }
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
      // fragments of k-step ks + 1 are read while the 16 MFMAs of ks run
      auto read_frags = [&](int ks, u32x4 (&a)[4], u32x4 (&b)[4]) {
        const int tko = ks * 2 + (lane >> 5);
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = lds[buf][0][tko][swz(wm + i * 32 + (lane & 31))];
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = lds[buf][bop][tko][swz(wn + j * 32 + (lane & 31))];
      };
      u32x4 a[4], b[4];
      read_frags(0, a, b);
#pragma unroll 1
      for (int ks = 0; ks < kBK / 16; ++ks) {
        u32x4 an[4], bn[4];
        read_frags((ks + 1) & (kBK / 16 - 1), an, bn);  // the last step re-reads step 0 (unused)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if constexpr (kBF16) {
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                  __builtin_bit_cast(bf16x8, a[i]), __builtin_bit_cast(bf16x8, b[j]), acc[i][j], 0, 0, 0);
            } else {
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                  __builtin_bit_cast(f16x8, a[i]), __builtin_bit_cast(f16x8, b[j]), acc[i][j], 0, 0, 0);
            }
          }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a[i] = an[i];
          b[i] = bn[i];
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
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = wm + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        const int col = wn + j * 32 + (lane & 31);
        out[row * kTile + col] = acc[i][j][v];
      }
}

// ------------------------------------------- 16-bit inputs, LDS DMA path ----
// For 16-byte aligned rows.  Per stage of 64 tokens, each operand's slab
// (64 tokens x 256 features, token-major, 32 KB) is copied into LDS by
// buffer_load_dwordx4 ... lds (one instruction = 1 KB = 2 token rows; tokens
// past the split and features past K read as zeros) -- no registers, no
// transposes.  MFMA fragments (8 consecutive tokens of one feature per lane)
// are then read with ds_read_b64_tr_b16: in each 16-lane group, lane 4r + q
// addresses token r, features 4q..4q+3 of a 4 x 16 block and lane i receives
// feature i of the 4 tokens.  The 16-byte slots of token row t are XOR-
// swizzled by dma_sig(t & 3) so that these reads hit distinct banks whether an
// LDS pass serves 16 or 32 lanes.  Waves form a (256 / WM) x (256 / WN) grid of
// WM x WN blocks; one barrier per stage, the next stage's copy is in flight
// during the current stage's MFMAs.
constexpr int kRowB = 512;          // one token row of a slab
constexpr int kSlabB = 64 * kRowB;  // one operand, one stage

__device__ __forceinline__ int dma_sig(int r) { return 10 * (r & 1) + 4 * ((r >> 1) & 1); }

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ u32x4 tr_frag(const uint8_t* p) {
  // (generic -> LDS address-space casts have to be C-style)
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 4 * kRowB));
  const uint2 a = __builtin_bit_cast(uint2, lo), b = __builtin_bit_cast(uint2, hi);
  return u32x4{a.x, a.y, b.x, b.y};
}

// Stages of kDmaBK = 48 tokens rotate through three buffers (144 KB): the
// copies of two stages are in flight while a third is multiplied out.  The
// buffers are distinct LDS variables and the stage loop is unrolled by three,
// so the compiler can tell the buffers being copied into from the one being
// read and does not wait for the copies before the reads.
constexpr int kDmaBK = 48;
constexpr int kStageB = kDmaBK * kRowB;  // one operand, one stage
__shared__ __attribute__((aligned(1024))) uint8_t g_hslab0[2][kStageB];
__shared__ __attribute__((aligned(1024))) uint8_t g_hslab1[2][kStageB];
__shared__ __attribute__((aligned(1024))) uint8_t g_hslab2[2][kStageB];

template <int B>
__device__ __forceinline__ uint8_t* hslab(int op) {
  return B == 0 ? &g_hslab0[op][0] : B == 1 ? &g_hslab1[op][0] : &g_hslab2[op][0];
}

// s_waitcnt for "at most N vector-memory operations outstanding" (gfx9
// encoding: vmcnt low bits 3:0, expcnt 6:4 and lgkmcnt 11:8 left at "no wait")
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N < 16, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

template <bool kBF16, int WM, int WN, int kMap = 0>
__global__ __launch_bounds__((256 / WM) * (256 / WN) * 64) __attribute__((amdgpu_waves_per_eu(1, 2)))
void hessian_dma16(const uint16_t* __restrict__ X, int64_t n, int K, int64_t ldx, int S, int64_t tok_per_split,
                   int ntiles, float* __restrict__ partial) {
  // 128 x 128 blocks keep their 256 accumulators per lane in AGPRs: an AGPR
  // clobber makes the compiler select the AGPR form of the MFMAs
  if constexpr (WM * WN > 128 * 64) asm volatile("" ::: "a0");
  constexpr int kW = (256 / WM) * (256 / WN);
  constexpr int FM = WM / 32, FN = WN / 32;
  constexpr int kBK = kDmaBK;
  constexpr int kChunks = kBK / 2;             // 1 KB copies per operand and stage
  constexpr int kPerWave = 2 * kChunks / kW;   // copies per wave and stage, both operands
  static_assert((2 * kChunks) % kW == 0 && kChunks % kW == 0, "copies split evenly over the waves");

  int s, tile;
  int I, J;
  split_tile<kMap>(blockIdx.x, S, ntiles, s, tile);
  if constexpr (kMap == 2)
    band_coords(tile, static_cast<int>(cdiv(static_cast<int64_t>(K), kTile)), I, J);
  else
    tile_coords(tile, I, J);
  const bool diag = (I == J);
  const int nops = diag ? 1 : 2;
  const int bop = diag ? 0 : 1;
  const int64_t t_begin = static_cast<int64_t>(s) * tok_per_split;
  const int64_t t_end = min(n, t_begin + tok_per_split);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave / (256 / WN)) * WM;
  const int wn = (wave % (256 / WN)) * WN;
  const bool wave_idle = diag && (wn >= wm + WM);

  // copy role: chunk c of an operand holds token rows 2c, 2c + 1; lane l
  // lands on row 2c + l / 32, slot l % 32, and fetches octet slot ^ sig(row)
  const int64_t rowb = ldx * 2;
  uint32_t vl[2][2];  // [operand][chunk parity]
#pragma unroll
  for (int op = 0; op < 2; ++op)
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int row = 2 * par + (lane >> 5);
      const int oct = (lane & 31) ^ dma_sig(row);
      const bool ok = (op == 0 ? I : J) * kTile + oct * 8 < K;
      vl[op][par] = ok ? static_cast<uint32_t>((lane >> 5) * rowb + oct * 16) : 0x80000000u;
    }
  auto issue = [&](int64_t t0, auto bsel) {
    constexpr int B = decltype(bsel)::value;
    const int64_t left = t_end - t0;
    const uint32_t nrec = static_cast<uint32_t>((left < kBK ? left : kBK) * rowb);
#pragma unroll
    for (int k = 0; k < kPerWave; ++k) {
      const int id = wave + kW * k;  // chunk id over both operands
      const int op = id / kChunks, c = id % kChunks;
      if (op < nops) {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(X + t0 * ldx + (op == 0 ? I : J) * kTile), static_cast<short>(0),
            static_cast<int>(nrec), 0x00020000);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(hslab<B>(op) + c * 1024), 16,
                                                 vl[op][c & 1] + static_cast<uint32_t>(2 * c * rowb), 0, 0, 0);
      }
    }
  };

  // fragment role: lane (g, r, q) reads token 8 (g / 2) + r (+4 for the second
  // half), octet ob + 2 (g % 2) + q / 2, 8-byte half q % 2
  const int g = lane >> 4, r = (lane >> 2) & 3, q = lane & 3;
  uint32_t aoff[FM], boff[FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
    aoff[i] = (8 * (g >> 1) + r) * kRowB + ((((wm + 32 * i) >> 3) + 2 * (g & 1) + (q >> 1)) ^ dma_sig(r)) * 16 +
              (q & 1) * 8;
#pragma unroll
  for (int j = 0; j < FN; ++j)
    boff[j] = (8 * (g >> 1) + r) * kRowB + ((((wn + 32 * j) >> 3) + 2 * (g & 1) + (q >> 1)) ^ dma_sig(r)) * 16 +
              (q & 1) * 8;

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  auto compute = [&](const uint8_t* la, const uint8_t* lb) {
    u32x4 fa[2][FM], fb[2][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) fa[0][i] = tr_frag(la + aoff[i]);
#pragma unroll
    for (int j = 0; j < FN; ++j) fb[0][j] = tr_frag(lb + boff[j]);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < kBK / 16) {
#pragma unroll
        for (int i = 0; i < FM; ++i) fa[cur ^ 1][i] = tr_frag(la + aoff[i] + (ks + 1) * 16 * kRowB);
#pragma unroll
        for (int j = 0; j < FN; ++j) fb[cur ^ 1][j] = tr_frag(lb + boff[j] + (ks + 1) * 16 * kRowB);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          if constexpr (kBF16) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(bf16x8, fa[cur][i]), __builtin_bit_cast(bf16x8, fb[cur][j]), acc[i][j], 0, 0, 0);
          } else {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                __builtin_bit_cast(f16x8, fa[cur][i]), __builtin_bit_cast(f16x8, fb[cur][j]), acc[i][j], 0, 0, 0);
          }
        }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // one stage out of buffer B: wait until this wave's copies into B have
  // landed (those of the next stage, in flight, may stay outstanding); after
  // the barrier every wave's have, and no wave still reads buffer B + 2 (the
  // previous stage's), which the copy of stage + 2 then fills
  auto stage = [&](int64_t t0, auto bsel) {
    constexpr int B = decltype(bsel)::value;
    if (t0 + kBK >= t_end) wait_vm<0>();
    else if (diag) wait_vm<kPerWave / 2>();
    else wait_vm<kPerWave>();
    __syncthreads();
    if (t0 + 2 * kBK < t_end) issue(t0 + 2 * kBK, std::integral_constant<int, (B + 2) % 3>{});
    if (!wave_idle) compute(hslab<B>(0), hslab<B>(bop));
  };

  if (t_begin < t_end) {
    issue(t_begin, std::integral_constant<int, 0>{});
    if (t_begin + kBK < t_end) issue(t_begin + kBK, std::integral_constant<int, 1>{});
    for (int64_t t0 = t_begin;;) {
      stage(t0, std::integral_constant<int, 0>{});
      if ((t0 += kBK) >= t_end) break;
      stage(t0, std::integral_constant<int, 1>{});
      if ((t0 += kBK) >= t_end) break;
      stage(t0, std::integral_constant<int, 2>{});
      if ((t0 += kBK) >= t_end) break;
    }
  }

  // 32x32 accumulator layout: lane l, register v -> row 8*(v/4) + 4*(l/32) + v%4, col l%32
  if (wave_idle) return;
  // partials are stored in the row-major triangle order the reduce reads
  const int slot = I * (I + 1) / 2 + J;
  float* out = partial + (static_cast<int64_t>(s) * ntiles + slot) * (kTile * kTile);
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
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

  int s, tile;
  split_tile(blockIdx.x, S, ntiles, s, tile);
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
  uint32_t ok = 0;  // bit 4 q + e: element e of pre[q] lies inside X
  static_assert(kPer <= 8, "validity bits");
  // branch-free loads (out-of-range elements read X[0][0] and are zeroed when
  // stored), so that the stage's loads stay in flight across the multiply
  auto load_stage = [&](int64_t t0) {
    ok = 0;
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int idx = q * kThreads + tid;
      const int op = idx >> 10;
      const int tok_l = (idx >> 6) & 15;
      const int f4 = idx & 63;
      const int64_t tok = t0 + tok_l;
      const int feat = (op == 0 ? I : J) * kTile + f4 * 4;
      const bool row_in = !(diag && op == 1) && tok < t_end;
      const int64_t off = tok * ldx + feat;
      if constexpr (kVec) {
        const bool in = row_in && feat < K;
        pre[q] = *reinterpret_cast<const f32x4*>(X + (in ? off : 0));
        ok |= in ? 0xFu << (4 * q) : 0u;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool in = row_in && feat + e < K;
          pre[q][e] = X[in ? off + e : 0];
          ok |= in ? 1u << (4 * q + e) : 0u;
        }
      }
    }
  };
  auto store_stage = [&]() {
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int idx = q * kThreads + tid;
      const int op = idx >> 10;
      if (diag && op == 1) continue;
      f32x4 v = pre[q];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (ok >> (4 * q + e)) & 1u ? v[e] : 0.0f;
      lds[op][(idx >> 6) & 15][idx & 63] = v;
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
  // partials summed in split order; eight loads are issued before their adds
  f32x4 v = *reinterpret_cast<const f32x4*>(p);
  int s = 1;
  for (; s + 8 <= S; s += 8) {
    f32x4 w[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) w[u] = *reinterpret_cast<const f32x4*>(p + (s + u) * tstride);
#pragma unroll
    for (int u = 0; u < 8; ++u) v += w[u];
  }
  for (; s < S; ++s) v += *reinterpret_cast<const f32x4*>(p + s * tstride);
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

}  // namespace
}  // namespace gptq

using namespace gptq;

namespace gptq {
namespace {

// H += X^T X for one run of tokens with S splits, partials in `part`
int accumulate_run(float* H, const void* X, int64_t n, int64_t K, int64_t ldx, int dtype, int S, float* part,
                   hipStream_t st) {
  const int64_t T = cdiv(K, kTile);
  const int ntiles = static_cast<int>(T * (T + 1) / 2);
  const int64_t per = cdiv(cdiv(n, S), 32) * 32;
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
    // aligned rows: LDS-DMA kernel, 8 waves of 128 x 64, split-major band order;
    // otherwise the register-staged kernel with element loads
    if (dtype == GPTQ_BF16) {
      if (vec)
        hipLaunchKernelGGL((hessian_dma16<true, 128, 64, 2>), grid, dim3(512), 0, st, x, n, (int)K, ldx, S, per, ntiles, part);
      else
        hipLaunchKernelGGL((hessian_tile16<true, false>), grid, dim3(kThreads16), 0, st, x, n, (int)K, ldx, S, per, ntiles, part);
    } else {
      if (vec)
        hipLaunchKernelGGL((hessian_dma16<false, 128, 64, 2>), grid, dim3(512), 0, st, x, n, (int)K, ldx, S, per, ntiles, part);
      else
        hipLaunchKernelGGL((hessian_tile16<false, false>), grid, dim3(kThreads16), 0, st, x, n, (int)K, ldx, S, per, ntiles, part);
    }
  }
  int rc = check_launch("hessian_tile");
  if (rc) return rc;
  hipLaunchKernelGGL(hessian_reduce, dim3(static_cast<unsigned>(ntiles) * 64), dim3(256), 0, st, H, (int)K, part, S, ntiles);
  return check_launch("hessian_reduce");
}

}  // namespace
}  // namespace gptq

extern "C" int gptq_hessian_accumulate(float* H, const void* X, int64_t n, int64_t K, int64_t ldx, int dtype,
                                       void* workspace, size_t workspace_bytes, gptq_stream_t stream) {
  clear_error();
  GPTQ_REQUIRE(H && (X || n == 0), GPTQ_ERR_ARG, "hessian_accumulate: null pointer");
  GPTQ_REQUIRE(K > 0 && K <= (1 << 20) && n >= 0 && ldx >= K, GPTQ_ERR_SHAPE,
               "hessian_accumulate: bad shape n=%lld K=%lld ldx=%lld", (long long)n, (long long)K, (long long)ldx);
  GPTQ_REQUIRE(valid_dtype(dtype), GPTQ_ERR_DTYPE, "hessian_accumulate: bad dtype %d", dtype);
  if (n == 0) return GPTQ_OK;
  const int ntiles = static_cast<int>(plan::hessian_tiles(K));
  const size_t split_bytes = plan::hessian_split_bytes(K);
  GPTQ_REQUIRE(workspace && workspace_bytes >= split_bytes, GPTQ_ERR_WORKSPACE,
               "hessian_accumulate: workspace %zu < %zu bytes (one split's partial tiles)", workspace_bytes,
               split_bytes);
  float* part = static_cast<float*>(workspace);
  hipStream_t st = as_hip(stream);
  const int S = plan::choose_splits(n, ntiles);
  if (static_cast<size_t>(S) * split_bytes <= workspace_bytes)
    return accumulate_run(H, X, n, K, ldx, dtype, S, part, st);
  // a smaller workspace: consecutive runs of tokens, each with as many splits
  // as the workspace holds, added to H one after the other (fixed order)
  const int64_t cap = static_cast<int64_t>(workspace_bytes / split_bytes);
  const int64_t run = plan::hessian_run_tokens(ntiles, cap);
  const int esz = dtype_size(dtype);
  for (int64_t t0 = 0; t0 < n; t0 += run) {
    const int64_t m = std::min<int64_t>(run, n - t0);
    const int Sm = static_cast<int>(std::min<int64_t>(plan::choose_splits(m, ntiles), cap));
    const int rc = accumulate_run(H, static_cast<const char*>(X) + t0 * ldx * esz, m, K, ldx, dtype, Sm, part, st);
    if (rc) return rc;
  }
  return GPTQ_OK;
}
