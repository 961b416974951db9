// Hessian accumulation H += X^T X on gfx950 MFMA (one triangle).
//
// Work decomposition
//   * H is cut into 256 x 256 tiles; only tiles (I, J) with J <= I are
//     computed.  A tile is one workgroup of 4 waves (one per SIMD) in a 2 x 2
//     grid, each wave owning a 128 x 128 block = 4 x 4 MFMA 32x32 blocks (256
//     fp32 accumulators per lane, in AGPRs).
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
// major.  With 16-byte aligned rows (hessian_gram16) token rows are copied
// into LDS as they are (direct-to-LDS buffer loads) and the fragments are
// read back transposed with ds_read_b64_tr_b16.  Otherwise (hessian_tile16)
// every thread loads an 8 token x 8 feature block with eight loads,
// transposes it in registers and writes eight 128-bit feature runs to LDS;
// there the LDS slot of feature f is swz(f) (below), which keeps both the
// transposed writes and the MFMA-fragment reads free of 16-byte bank-group
// collisions.  fp32 inputs use v_mfma_f32_32x32x2_f32 with a
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
// For 16-byte aligned rows.  Per stage of 48 tokens, each operand's slab
// (48 tokens x 256 features, token-major, 24 KB) is copied into LDS by
// buffer_load_dwordx4 ... lds (one instruction = 1 KB = 2 token rows; tokens
// past the split and features past K read as zeros) -- no registers, no
// transposes.  MFMA fragments (8 consecutive tokens of one feature per lane)
// are then read with ds_read_b64_tr_b16: in each 16-lane group, lane 4r + q
// addresses token r, features 4q..4q+3 of a 4 x 16 block and lane i receives
// feature i of the 4 tokens.  The 16-byte slots of token row t are XOR-
// swizzled by dma_sig(t & 3) so that these reads hit distinct banks whether an
// LDS pass serves 16 or 32 lanes.
//
// One workgroup of 4 waves (one per SIMD) per (split, tile); wave w owns the
// 128 x 128 block (w / 2, w % 2) of the 256 x 256 tile as 4 x 4 MFMA 32x32
// blocks, 256 fp32 accumulators per lane in AGPRs.  Per 16 tokens (a step) a
// wave reads 8 fragments (16 LDS reads) for 16 MFMAs.
//
// Schedule, per stage of three steps out of one of three LDS buffers:
//   * fragments are read one step ahead into three register sets (step q of
//     a stage uses set q), two LDS reads after each of a step's first 8 MFMAs;
//   * the stage barrier sits after the first 8 MFMAs of the last step: before
//     it a wave waits for its own copies of the next stage (those of the
//     stage after it stay in flight) and for its LDS reads of this stage;
//     after it the next stage's first fragments are read under the step's
//     last 8 MFMAs.  The barrier is a bare s_barrier: these waits are all it
//     needs, and the compiler's full wait before a barrier would also wait
//     for the copies still in flight;
//   * each wave issues 12 copies per stage, one after every fourth MFMA of
//     the first two steps (4 + 4 copies of the stage two ahead, into the
//     buffer freed at the previous stage's barrier) and after every second
//     MFMA of the last step's tail (4 copies of the stage three ahead, into
//     this stage's buffer).  Spread this way the copies cost 8-9% less time
//     than issued together after the barrier.
//   * the MFMAs are inline asm (accumulators pinned to AGPRs, fragments to
//     VGPRs; with the builtin the register allocator moved accumulators
//     through VGPRs and spilled).  volatile keeps them in program order with
//     the LDS reads and copies; the compiler still places the LDS waits
//     before each MFMA from its operands.
constexpr int kRowB = 512;  // one token row of a slab

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

// Three stage buffers (3 x 48 KB).  They are distinct LDS variables selected
// at compile time (the stage loop is unrolled by three), so the compiler can
// tell the buffers being copied into from the one being read and does not
// wait for the copies before the reads.
constexpr int kDmaBK = 48;
constexpr int kStageB = kDmaBK * kRowB;  // one operand, one stage
__shared__ __attribute__((aligned(1024))) uint8_t g_hslab0[2][kStageB];
__shared__ __attribute__((aligned(1024))) uint8_t g_hslab1[2][kStageB];
__shared__ __attribute__((aligned(1024))) uint8_t g_hslab2[2][kStageB];

template <int B>
__device__ __forceinline__ uint8_t* hslab(int op) {
  return B == 0 ? &g_hslab0[op][0] : B == 1 ? &g_hslab1[op][0] : &g_hslab2[op][0];
}

template <bool kBF16>
__device__ __forceinline__ void mfma32_asm(f32x16& acc, const u32x4& a, const u32x4& b) {
  if constexpr (kBF16)
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  else
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// A wave-uniform 64-bit value through readfirstlane, which takes and returns
// int: each half is widened as unsigned, so that a low half with bit 31 set
// does not sign-extend into the high half.
__device__ __forceinline__ uint64_t uniform_u64(uint64_t v) {
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(v))));
  const uint32_t hi =
      static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(v >> 32))));
  return static_cast<uint64_t>(hi) << 32 | lo;
}

// One 16-byte-per-lane copy into LDS from base + voff, zeros at and past nrec
// bytes.  base and nrec are wave-uniform (the descriptor stays in SGPRs).
// (Target builtins sit in a __device__ function, not in the kernel body: in
// the kernel body the host pass dropped the kernel's launch stub.)
__device__ __forceinline__ void lds_copy16(const uint16_t* base, uint32_t nrec, uint8_t* lds, uint32_t voff) {
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<uint16_t*>(uniform_u64(reinterpret_cast<uint64_t>(base))), static_cast<short>(0),
      __builtin_amdgcn_readfirstlane(static_cast<int>(nrec)), 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)lds, 16, voff, 0, 0, 0);
}

__device__ __forceinline__ void bare_barrier() { asm volatile("s_barrier" ::: "memory"); }

// s_waitcnt for "at most N vector-memory operations outstanding" (gfx9
// encoding: vmcnt bits 3:0 and 15:14; expcnt and lgkmcnt left at "no wait")
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N < 64, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// s_waitcnt for "at most N LDS / scalar-memory operations outstanding"
template <int N>
__device__ __forceinline__ void wait_lgkm() {
  static_assert(N < 16, "lgkmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0xC07F | (N << 8));
}

// copy slots: after which MFMA m of a step the step's j-th copy goes (-1:
// none), and after which MFMA m (8..15) of the last step's tail
constexpr int step_copy(int m) { return m % 4 == 1 ? m / 4 : -1; }
constexpr int tail_copy(int m) { return m % 2 == 1 ? (m - 9) / 2 : -1; }

template <bool kBF16>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void hessian_gram16(const uint16_t* __restrict__ X, int64_t n, int K, int64_t ldx, int S, int64_t tok_per_split,
                    int ntiles, float* __restrict__ partial) {
  constexpr int kBK = kDmaBK;
  constexpr int kPerWave = kBK / 4;  // 12 copies of 1 KB per wave and stage: 6 of each operand

  int s, tile, I, J;
  split_tile<2>(blockIdx.x, S, ntiles, s, tile);
  band_coords(tile, static_cast<int>(cdiv(static_cast<int64_t>(K), kTile)), I, J);
  const bool diag = (I == J);
  const int64_t tb = static_cast<int64_t>(uniform_u64(static_cast<uint64_t>(static_cast<int64_t>(s) * tok_per_split)));
  const int64_t te = static_cast<int64_t>(uniform_u64(static_cast<uint64_t>(min(n, tb + tok_per_split))));

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int wm = (wave >> 1) * 128, wn = (wave & 1) * 128;
  // the wave above the diagonal of a diagonal tile computes but stores nothing
  const bool wave_idle = diag && wn > wm;

  // copy role: chunk c of an operand holds token rows 2c, 2c + 1; copy k
  // (0..11) of this wave is chunk c = wave + 4 (k mod 6) of operand k / 6,
  // all of one row parity.  Lane l lands on row 2c + l / 32, slot l % 32, and
  // fetches octet slot ^ sig(row); features past K get an offset past every
  // record count (zeros).
  const int64_t rowb = ldx * 2;
  uint32_t voff[kPerWave];
#pragma unroll
  for (int k = 0; k < kPerWave; ++k) {
    const int op = k >= kPerWave / 2 ? 1 : 0;
    const int c = wave + 4 * (k - op * (kPerWave / 2));
    const int row = 2 * (wave & 1) + (lane >> 5);
    const int oct = (lane & 31) ^ dma_sig(row);
    const bool ok = (op == 0 ? I : J) * kTile + oct * 8 < K;
    voff[k] = ok ? static_cast<uint32_t>((lane >> 5) * rowb + oct * 16 + 2 * c * rowb) : 0x80000000u;
  }
  // the two operands' bases and record counts for the stage at t0: rows past
  // the split's end and the second operand of a diagonal tile are not fetched
  struct StageSrc {
    const uint16_t* base[2];
    uint32_t nrec[2];
  };
  auto stage_src = [&](int64_t t0) {
    const int rem = static_cast<int>(te - t0);
    const int rows = rem <= 0 ? 0 : rem < kBK ? rem : kBK;
    const uint32_t nrec = static_cast<uint32_t>(rows * rowb);
    StageSrc ss;
#pragma unroll
    for (int op = 0; op < 2; ++op) {
      ss.base[op] = X + t0 * ldx + (op == 0 ? I : J) * kTile;
      ss.nrec[op] = op == 1 && diag ? 0u : nrec;
    }
    return ss;
  };
  auto copy = [&](const StageSrc& ss, auto bsel, auto ksel) {
    constexpr int B = decltype(bsel)::value, k = decltype(ksel)::value;
    constexpr int op = k >= kPerWave / 2 ? 1 : 0;
    const int c = wave + 4 * (k - op * (kPerWave / 2));
    lds_copy16(ss.base[op], ss.nrec[op], hslab<B>(op) + c * 1024, voff[k]);
  };

  // fragment role: lane (g, r, q) reads token 8 (g / 2) + r (+4 for the second
  // half), octet ob + 2 (g % 2) + q / 2, 8-byte half q % 2
  const int g = lane >> 4, r = (lane >> 2) & 3, q = lane & 3;
  const int bop = diag ? 0 : 1;
  uint32_t aoff[4], boff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    aoff[i] = (8 * (g >> 1) + r) * kRowB + ((((wm + 32 * i) >> 3) + 2 * (g & 1) + (q >> 1)) ^ dma_sig(r)) * 16 +
              (q & 1) * 8;
    boff[i] = bop * kStageB + (8 * (g >> 1) + r) * kRowB +
              ((((wn + 32 * i) >> 3) + 2 * (g & 1) + (q >> 1)) ^ dma_sig(r)) * 16 + (q & 1) * 8;
  }

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  u32x4 fr[3][8];  // [set][A0..A3, B0..B3]
  // fragment f of step ks of buffer B into set St; read order A0, B0, B1, B2,
  // B3, A1, A2, A3 (the order the next step's MFMAs need them)
  auto read = [&](auto bsel, auto ssel, auto ksel, auto fsel) {
    constexpr int B = decltype(bsel)::value, St = decltype(ssel)::value;
    constexpr int ks = decltype(ksel)::value, f = decltype(fsel)::value;
    constexpr int idx = f == 0 ? 0 : f < 5 ? f + 3 : f - 4;
    const uint8_t* base = hslab<B>(0) + ks * 16 * kRowB;
    if constexpr (idx < 4)
      fr[St][idx] = tr_frag(base + aoff[idx]);
    else
      fr[St][idx] = tr_frag(base + boff[idx - 4]);
  };
  auto mfma = [&](auto ssel, auto msel) {
    constexpr int St = decltype(ssel)::value, m = decltype(msel)::value;
    mfma32_asm<kBF16>(acc[m >> 2][m & 3], fr[St][m >> 2], fr[St][4 + (m & 3)]);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;

  // one step on set St: 16 MFMAs; the next step's fragments (set Sn, step
  // ksn of buffer Bn) after the first 8, copies 4j.. of the stage two ahead
  // at the step's copy slots
  auto step = [&](auto ssel, auto bnsel, auto snsel, auto knsel, const StageSrc& ss, auto psel, auto k0sel) {
    sfor<0, 16>([&](auto mc) {
      constexpr int m = decltype(mc)::value;
      mfma(ssel, mc);
      if constexpr (m < 8) read(bnsel, snsel, knsel, mc);
      if constexpr (step_copy(m) >= 0)
        copy(ss, psel, std::integral_constant<int, decltype(k0sel)::value + step_copy(m)>{});
    });
    sfor<0, 16>([&](auto mc) {
      constexpr int m = decltype(mc)::value;
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                          // MFMA
      if constexpr (m < 8) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);      // LDS reads
      if constexpr (step_copy(m) >= 0) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // copy
    });
    __builtin_amdgcn_sched_barrier(0);
  };

  // stage at t0 out of buffer B, its step-0 fragments already in set 0.  The
  // tail after the barrier runs also after the split's last stage: its
  // copies then have zero records and its reads go unused.
  auto stage = [&](int64_t t0, auto bsel) {
    constexpr int B = decltype(bsel)::value;
    using Bn = std::integral_constant<int, (B + 1) % 3>;
    using Bp = std::integral_constant<int, (B + 2) % 3>;
    const StageSrc ahead2 = stage_src(t0 + 2 * kBK);
    step(I0{}, bsel, I1{}, I1{}, ahead2, Bp{}, std::integral_constant<int, 4>{});
    step(I1{}, bsel, I2{}, I2{}, ahead2, Bp{}, std::integral_constant<int, 8>{});
    sfor<0, 8>([&](auto mc) { mfma(I2{}, mc); });
    __builtin_amdgcn_sched_barrier(0);
    wait_vm<kPerWave>();
    wait_lgkm<0>();
    bare_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const StageSrc ahead3 = stage_src(t0 + 3 * kBK);
    sfor<8, 16>([&](auto mc) {
      constexpr int m = decltype(mc)::value;
      mfma(I2{}, mc);
      read(Bn{}, I0{}, I0{}, std::integral_constant<int, m - 8>{});
      if constexpr (tail_copy(m) >= 0) copy(ahead3, bsel, std::integral_constant<int, tail_copy(m)>{});
    });
    sfor<8, 16>([&](auto mc) {
      constexpr int m = decltype(mc)::value;
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      if constexpr (tail_copy(m) >= 0) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    });
    __builtin_amdgcn_sched_barrier(0);
  };

  if (tb < te) {
    // stages 0 and 1 whole, copies 0..3 of stage 2 (the first stage's steps
    // issue its copies 4..11)
    const StageSrc s0 = stage_src(tb), s1 = stage_src(tb + kBK), s2 = stage_src(tb + 2 * kBK);
    sfor<0, kPerWave>([&](auto kc) { copy(s0, I0{}, kc); });
    sfor<0, kPerWave>([&](auto kc) { copy(s1, I1{}, kc); });
    sfor<0, 4>([&](auto kc) { copy(s2, I2{}, kc); });
    wait_vm<kPerWave + 4>();
    bare_barrier();
    __builtin_amdgcn_sched_barrier(0);
    sfor<0, 8>([&](auto fc) { read(I0{}, I0{}, I0{}, fc); });
    // three stages per trip, one per buffer; stages past the split's end
    // multiply zeros, which leaves the sums unchanged (+0 added to a sum that
    // starts at +0)
    for (int64_t t0 = tb; t0 < te; t0 += 3 * kBK) {
      stage(t0, I0{});
      stage(t0 + kBK, I1{});
      stage(t0 + 2 * kBK, I2{});
    }
    // no copy may still be writing LDS when the workgroup ends
    wait_vm<0>();
    // the accumulators are read below: wait states after the last MFMA (the
    // compiler does not see the asm MFMAs' results as MFMA results)
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  }

  // 32x32 accumulator layout: lane l, register v -> row 8*(v/4) + 4*(l/32) + v%4, col l%32
  if (wave_idle) return;
  // partials are stored in the row-major triangle order the reduce reads
  const int slot = I * (I + 1) / 2 + J;
  float* out = partial + (static_cast<int64_t>(s) * ntiles + slot) * (kTile * kTile);
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
  // partials summed in split order; up to eight loads are issued before
  // their adds (the last < 8 as well: one at a time, each waited for, they
  // were a chain of round trips with 4 splits)
  f32x4 v = *reinterpret_cast<const f32x4*>(p);
  int s = 1;
  for (; s + 8 <= S; s += 8) {
    f32x4 w[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) w[u] = *reinterpret_cast<const f32x4*>(p + (s + u) * tstride);
#pragma unroll
    for (int u = 0; u < 8; ++u) v += w[u];
  }
  if (s < S) {
    f32x4 w[7];
#pragma unroll
    for (int u = 0; u < 7; ++u)
      if (s + u < S) w[u] = *reinterpret_cast<const f32x4*>(p + (s + u) * tstride);
#pragma unroll
    for (int u = 0; u < 7; ++u)
      if (s + u < S) v += w[u];
  }
  // H's four elements read together (one 16-byte load when the quad is in
  // bounds), before any is added or written
  const int64_t gj0 = static_cast<int64_t>(J) * kTile + sc * 32 + col0;
  f32x4 hv = f32x4{0.f, 0.f, 0.f, 0.f};
  if (gi < K && gj0 + 3 < K && (K & 3) == 0) {
    hv = *reinterpret_cast<const f32x4*>(H + gi * K + gj0);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (gi < K && gj0 + e < K) hv[e] = H[gi * K + gj0 + e];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t gj = gj0 + e;
    float val = v[e];
    if (gi < K && gj < K) {
      val += hv[e];
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
  // (the DMA kernel's 32-bit row offsets: 48 rows of at most 8 MB)
  const bool vec = (ldx * esz) % 16 == 0 && (reinterpret_cast<uintptr_t>(X) % 16) == 0 && (K * esz) % 16 == 0 &&
                   ldx * esz <= (int64_t(1) << 23);
  if (dtype == GPTQ_F32) {
    const float* x = static_cast<const float*>(X);
    if (vec)
      hipLaunchKernelGGL((hessian_tile32<true>), grid, dim3(kThreads), 0, st, x, n, (int)K, ldx, S, per, ntiles, part);
    else
      hipLaunchKernelGGL((hessian_tile32<false>), grid, dim3(kThreads), 0, st, x, n, (int)K, ldx, S, per, ntiles, part);
  } else {
    const uint16_t* x = static_cast<const uint16_t*>(X);
    // aligned rows: LDS-DMA kernel, 4 waves of 128 x 128, split-major band
    // order; otherwise the register-staged kernel with element loads
    if (dtype == GPTQ_BF16) {
      if (vec)
        hipLaunchKernelGGL((hessian_gram16<true>), grid, dim3(256), 0, st, x, n, (int)K, ldx, S, per, ntiles, part);
      else
        hipLaunchKernelGGL((hessian_tile16<true, false>), grid, dim3(kThreads16), 0, st, x, n, (int)K, ldx, S, per, ntiles, part);
    } else {
      if (vec)
        hipLaunchKernelGGL((hessian_gram16<false>), grid, dim3(256), 0, st, x, n, (int)K, ldx, S, per, ntiles, part);
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
