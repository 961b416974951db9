// fp32 GEMM on v_mfma_f32_32x32x2_f32 (gfx950).
//
// 128 x 128 output tile per workgroup of 4 waves (2 x 2, 64 x 64 each =
// 2 x 2 MFMA 32x32 blocks), 16-deep k stages staged in LDS as [row][k]
// (pitch 18 floats: the two k-rows a 32x32x2 fragment reads land in
// disjoint bank halves), next stage prefetched into registers while the
// current one is multiplied.  Triangular operands skip the k-tiles that are
// known to be zero; GEMM_C_LOWER skips tiles strictly above the diagonal.
#include "gemm.hpp"

namespace gptq {
namespace {

constexpr int kTM = 128;
constexpr int kTN = 128;
constexpr int kBK = 16;
constexpr int kPitch = kBK + 2;
constexpr int kThreads = 256;

struct Operand {
  const float* p;
  int64_t ld;
  bool trans;   // element (r, k) of the operand is p[k * ld + r] when trans
  int64_t rows; // extent along r
};

// Loads the stage (r0..r0+127, k0..k0+15) of an operand viewed as [r][k]
// into registers: 512 float4 per operand, 2 per thread.
template <bool kVec>
__device__ __forceinline__ void load_op(const Operand& o, int64_t r0, int64_t k0, int64_t Kd, int tid,
                                        f32x4 (&pre)[2]) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int idx = q * kThreads + tid;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (!o.trans) {
      // contiguous along k: 4 lanes per row
      const int64_t r = r0 + (idx >> 2);
      const int64_t k = k0 + (idx & 3) * 4;
      if (r < o.rows) {
        const float* src = o.p + r * o.ld + k;
        if (kVec && k + 3 < Kd) {
          v = *reinterpret_cast<const f32x4*>(src);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (k + e < Kd) ? src[e] : 0.0f;
        }
      }
    } else {
      // contiguous along r: 32 lanes per k-row
      const int64_t k = k0 + (idx >> 5);
      const int64_t r = r0 + (idx & 31) * 4;
      if (k < Kd) {
        const float* src = o.p + k * o.ld + r;
        if (kVec && r + 3 < o.rows) {
          v = *reinterpret_cast<const f32x4*>(src);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (r + e < o.rows) ? src[e] : 0.0f;
        }
      }
    }
    pre[q] = v;
  }
}

__device__ __forceinline__ void store_op(bool trans, float* s, int tid, const f32x4 (&pre)[2]) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int idx = q * kThreads + tid;
    if (!trans) {
      const int r = idx >> 2, k = (idx & 3) * 4;
      float2* d = reinterpret_cast<float2*>(s + r * kPitch + k);
      d[0] = make_float2(pre[q][0], pre[q][1]);
      d[1] = make_float2(pre[q][2], pre[q][3]);
    } else {
      const int k = idx >> 5, r = (idx & 31) * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) s[(r + e) * kPitch + k] = pre[q][e];
    }
  }
}

template <bool kVec>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(int64_t M, int64_t N, int64_t Kd, float alpha,
                                                           Operand a, Operand b, float beta, float* __restrict__ C,
                                                           int64_t ldc, int flags, int tiles_n) {
  __shared__ float sA[kTM * kPitch];
  __shared__ float sB[kTN * kPitch];
  const int tm = blockIdx.x / tiles_n;
  const int tn = blockIdx.x % tiles_n;
  const int64_t i0 = static_cast<int64_t>(tm) * kTM;
  const int64_t j0 = static_cast<int64_t>(tn) * kTN;
  if ((flags & GEMM_C_LOWER) && j0 > i0 + kTM - 1) return;

  int64_t kb = 0, ke = Kd;
  if (flags & GEMM_KLIM_A_LE_I) ke = std::min<int64_t>(ke, i0 + kTM);
  if (flags & GEMM_KLIM_B_LE_J) ke = std::min<int64_t>(ke, j0 + kTN);
  if (flags & GEMM_KLIM_A_GE_I) kb = std::max<int64_t>(kb, i0);
  if (flags & GEMM_KLIM_B_GE_J) kb = std::max<int64_t>(kb, j0);
  kb = (kb / kBK) * kBK;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 1) * 64;
  const int wn = (wave & 1) * 64;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  f32x4 pa[2], pb[2];
  if (kb < ke) {
    load_op<kVec>(a, i0, kb, Kd, tid, pa);
    load_op<kVec>(b, j0, kb, Kd, tid, pb);
  }
  for (int64_t k0 = kb; k0 < ke; k0 += kBK) {
    __syncthreads();
    store_op(a.trans, sA, tid, pa);
    store_op(b.trans, sB, tid, pb);
    __syncthreads();
    if (k0 + kBK < ke) {
      load_op<kVec>(a, i0, k0 + kBK, Kd, tid, pa);
      load_op<kVec>(b, j0, k0 + kBK, Kd, tid, pb);
    }
#pragma unroll
    for (int kk = 0; kk < kBK / 2; ++kk) {
      const int k = kk * 2 + (lane >> 5);
      float fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = sA[(wm + i * 32 + (lane & 31)) * kPitch + k];
#pragma unroll
      for (int j = 0; j < 2; ++j) fb[j] = sB[(wn + j * 32 + (lane & 31)) * kPitch + k];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i], fb[j], acc[i][j], 0, 0, 0);
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
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = cbase + j * 32;
      float* cp = C + (rbase + i * 32) * ldc + col;
      float cv[16];
      if (beta != 0.0f) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t row = rbase + i * 32 + 8 * (v >> 2) + (v & 3);
          cv[v] = (row < M && col < N) ? cp[(8 * (v >> 2) + (v & 3)) * ldc] : 0.0f;
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

}  // namespace

int launch_gemm_f32(hipStream_t st, int64_t M, int64_t N, int64_t Kd, float alpha, const float* A, int64_t lda,
                    bool transA, const float* B, int64_t ldb, bool transB, float beta, float* C, int64_t ldc,
                    int flags) {
  if (M <= 0 || N <= 0) return GPTQ_OK;
  const int tiles_m = static_cast<int>(cdiv(M, kTM));
  const int tiles_n = static_cast<int>(cdiv(N, kTN));
  Operand a{A, lda, transA, M};
  Operand b{B, ldb, !transB, N};  // operand B is viewed as [j][k]: B^T
  const bool vec = lda % 4 == 0 && ldb % 4 == 0 && (reinterpret_cast<uintptr_t>(A) % 16) == 0 &&
                   (reinterpret_cast<uintptr_t>(B) % 16) == 0;
  const dim3 grid(static_cast<unsigned>(tiles_m) * tiles_n);
  if (vec)
    hipLaunchKernelGGL(gemm_f32_kernel<true>, grid, dim3(kThreads), 0, st, M, N, Kd, alpha, a, b, beta, C, ldc,
                       flags, tiles_n);
  else
    hipLaunchKernelGGL(gemm_f32_kernel<false>, grid, dim3(kThreads), 0, st, M, N, Kd, alpha, a, b, beta, C, ldc,
                       flags, tiles_n);
  return check_launch("gemm_f32");
}

}  // namespace gptq
