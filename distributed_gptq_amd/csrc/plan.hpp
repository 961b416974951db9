// Host-side planning of libgptq_hip.so: how the entry points split their work
// (token splits, recursion splits, kernel plans) and how much workspace they
// need, and the argument checks of gptq::linear.  Pure integer functions with
// no HIP dependency, so that the launchers in the .hip files and a CPU build
// of this file under AddressSanitizer and UndefinedBehaviorSanitizer run the
// same code.
#pragma once

#include <cstddef>
#include <cstdint>

#include "status.hpp"

namespace gptq {

inline bool valid_dtype(int d) { return d == GPTQ_F32 || d == GPTQ_F16 || d == GPTQ_BF16; }
inline int dtype_size(int d) { return d == GPTQ_F32 ? 4 : 2; }

namespace plan {

// ceil(a / b) for a >= 0, b > 0, without the overflow of (a + b - 1) / b
inline int64_t ceil_div(int64_t a, int64_t b) { return a / b + (a % b != 0); }
// a * b and a + b, or SIZE_MAX where the result does not fit in size_t (a
// workspace no allocation can provide; the size queries report it as such)
inline size_t mul_sat(size_t a, size_t b) {
  size_t r;
  return __builtin_mul_overflow(a, b, &r) ? SIZE_MAX : r;
}
inline size_t add_sat(size_t a, size_t b) {
  size_t r;
  return __builtin_add_overflow(a, b, &r) ? SIZE_MAX : r;
}

// ------------------------------------------------------------- Hessian ----
constexpr int kHessTile = 256;  // H is computed in 256 x 256 tiles of its lower triangle

// tiles of the lower triangle (diagonal included) of a K x K Hessian
int64_t hessian_tiles(int64_t K);
// bytes of one token split's fp32 partial tiles
size_t hessian_split_bytes(int64_t K);
// token splits of one launch over n tokens (1..64)
int choose_splits(int64_t n, int64_t ntiles);
// tokens per run when the workspace holds only `cap` splits' partial tiles
// (fewer than choose_splits wants): runs are added to H one after the other
int64_t hessian_run_tokens(int64_t ntiles, int64_t cap);

// ------------------------------------------------------- factorisation ----
constexpr int kFactorLeaf = 128;  // the recursion's leaf (one workgroup)

// size of the left half of a recursion node of size m (whole leaves)
int64_t factor_split(int64_t m);
// scratch floats the recursion below a node of size m needs
int64_t factor_scratch_floats(int64_t m);

// ---------------------------------------------------------------- sweep ----
constexpr int kSweepSub = 128;     // columns per sweep sub-block
constexpr int64_t kSweepRun = 512;  // columns per run of the two-level lazy batch

// blocks of `blocksize` columns per run (at least kSweepRun columns)
int64_t sweep_run_blocks(int blocksize);

// --------------------------------------------------------------- linear ----
// the register-decoded dequant-GEMM's plan for 16 < M <= 384: K splits (0 =
// the kernel does not take the layer), compute waves per workgroup and weight
// rows per compute wave
struct RxPlan {
  int splits = 0;
  int waves = 8;
  int rows = 16;
};
RxPlan rx_plan(int64_t M, int64_t N, int64_t K, int64_t pitch, int bits, bool rows32 = true);
// K splits of the register path for 1 < M <= 16 on 4097-8191-row layers (0
// outside these shapes), on 8192-row layers and, for 8 < M <= 16 with
// K >= 10240, on 3072-4096-row layers (0 elsewhere)
int reg4_mid_splits(int64_t M, int64_t N, int64_t K);
int reg4_wide_splits(int64_t M, int64_t N, int64_t K);
int reg4_narrow_splits(int64_t M, int64_t N, int64_t K);
// split-K partial-sum bytes the register kernels use for this layer (0 when
// they do not split it)
size_t splitk_bytes(int64_t M, int64_t N, int64_t K, int bits, int group_size, int x_dtype);
size_t round256(size_t b);
// argument checks shared by the gptq_linear entry points (a gptq_status)
int check_linear_args(const void* x, int x_dtype, int64_t M, const void* packed, int bits, const void* scales,
                      const void* zeros, int sz_dtype, const int32_t* g_idx, int group_size, int64_t ngroups,
                      const void* bias, int bias_dtype, int64_t N, int64_t K, const void* y);

}  // namespace plan
}  // namespace gptq
