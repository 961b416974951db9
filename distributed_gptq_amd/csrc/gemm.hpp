// fp32 MFMA GEMM used inside the library (factorisation and the sweep's
// lazy-batch trailing update):
//   C[i][j] = alpha * sum_k opA[i][k] opB[k][j] + beta * C[i][j]
// opA = A (M x Kd, row stride lda) or A^T; opB = B (Kd x N) or B^T.
// With beta == 0, C is not read.
#pragma once
#include "common.hpp"

namespace gptq {

enum GemmFlags {
  GEMM_KLIM_A_LE_I = 1,  // opA[i][k] == 0 for k > i (skip those k-tiles)
  GEMM_KLIM_A_GE_I = 2,  // opA[i][k] == 0 for k < i
  GEMM_KLIM_B_LE_J = 4,  // opB[k][j] == 0 for k > j
  GEMM_KLIM_B_GE_J = 8,  // opB[k][j] == 0 for k < j
  GEMM_C_LOWER = 16      // only C[i][j] with i >= j is computed and written
};

struct GemmCall {
  int64_t M, N, Kd;
  float alpha;
  const float* A;
  int64_t lda;
  bool transA;
  const float* B;
  int64_t ldb;
  bool transB;
  float beta;
  float* C;
  int64_t ldc;
  int flags;
};

int launch_gemm_f32(hipStream_t st, int64_t M, int64_t N, int64_t Kd, float alpha, const float* A,
                    int64_t lda, bool transA, const float* B, int64_t ldb, bool transB, float beta,
                    float* C, int64_t ldc, int flags);

// Two products that are independent (neither reads or writes what the other
// writes).  When both take 64 x 64 tiles they run as one grid, so that their
// tiles share the CUs and the pair pays one launch; otherwise p, then q.
int launch_gemm_f32_pair(hipStream_t st, const GemmCall& p, const GemmCall& q);

}  // namespace gptq
