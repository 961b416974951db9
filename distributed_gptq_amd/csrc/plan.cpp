// Host-side planning of libgptq_hip.so (see plan.hpp): split counts, kernel
// plans, workspace sizes and the gptq::linear argument checks.
#include "plan.hpp"

#include <algorithm>

namespace gptq {
namespace plan {

// ------------------------------------------------------------- Hessian ----

int64_t hessian_tiles(int64_t K) {
  const int64_t T = ceil_div(K, kHessTile);
  return T * (T + 1) / 2;
}

size_t hessian_split_bytes(int64_t K) {
  return static_cast<size_t>(hessian_tiles(K)) * kHessTile * kHessTile * sizeof(float);
}

// Every split writes, and the reduce reads back, 512 KB per tile, so splits
// cost traffic once they are short: at most 16384 tokens per split (10240 for
// products of fewer than 512 tiles, K < 5888), and beyond that only as many
// splits as bring the launch to ~512 workgroups while each keeps >= 1024
// tokens; at most 64.  Measured on MI355X (fp16 X): (n, K) = (32768, 768) ->
// 32 splits, (32768, 3072) -> 7, (16384, 5120) -> 3, (16384, 13824) -> 1,
// (262144, 14336) -> 16, each within 5% of the best split count of a sweep
// over 1..64, and 1.2-1.5x faster than ~2048 workgroups for the short calls;
// bf16 at (262144, 4096): 16 / 24 / 32 splits 4.57 / 4.47 / 4.52 ms (26 now).
// With the 4-wave tile kernel, (262144, 14336) with 4 / 8 / 12 / 16 splits
// takes 41.6 / 41.8 / 42.6 / 42.9 ms, and the reduce reads 4x fewer partial
// tiles with 4: products of >= 1024 tiles (K >= 11265) therefore take at most
// 4 splits, or as many as keep each <= 65536 tokens (tile + reduce at
// (262144, 14336): 43.1 against 44.7 ms; workspace 1.7 against 6.7 GB).
// Shorter products keep the rule above: applied to every product, 65536
// tokens per split changed H's rounding where the sweeps were validated (the
// 27685-token Hessian at K = 13824 ran as 1 split instead of 2, and the 8-bit
// act-order codes then agreed with the fp32 oracle's to 0.99865, below 0.999).
int choose_splits(int64_t n, int64_t ntiles) {
  constexpr int64_t kTokMin = 1024, kMinWG = 512;
  if (n <= 0 || ntiles <= 0) return 1;
  const int64_t tok_max = ntiles < 512 ? 10240 : 16384;
  const int64_t fill = std::min<int64_t>(ceil_div(kMinWG, ntiles), std::max<int64_t>(1, n / kTokMin));
  int64_t s = std::max<int64_t>(ceil_div(n, tok_max), fill);
  // >= 1024 tiles: 4 splits already make >= 4096 workgroups (16 rounds of the
  // 256 CUs), so beyond 4 only as many as keep each split <= 65536 tokens
  if (ntiles >= 1024) s = std::max<int64_t>(std::min<int64_t>(s, 4), ceil_div(n, 65536));
  return static_cast<int>(std::min<int64_t>(std::max<int64_t>(s, 1), 64));
}

int64_t hessian_run_tokens(int64_t ntiles, int64_t cap) {
  int64_t run = std::max<int64_t>(cap, 1) * 16384;
  while (run > 1024 && choose_splits(run, ntiles) > cap) run /= 2;
  return run;
}

// ------------------------------------------------------- factorisation ----

int64_t factor_split(int64_t m) {
  const int64_t nb = ceil_div(m, kFactorLeaf);
  return ((nb + 1) / 2) * kFactorLeaf;
}

// 2 * m2 * m1 floats at this node + whatever the right child needs (the left
// child's scratch is reused)
int64_t factor_scratch_floats(int64_t m) {
  if (m <= kFactorLeaf) return 0;
  const int64_t m1 = factor_split(m), m2 = m - m1;
  return 2 * m2 * m1 + std::max(factor_scratch_floats(m1), factor_scratch_floats(m2));
}

// ---------------------------------------------------------------- sweep ----

int64_t sweep_run_blocks(int blocksize) { return std::max<int64_t>(1, ceil_div(kSweepRun, blocksize)); }

// --------------------------------------------------------------- linear ----

// Compute waves and K splits of the register-decoded kernel.  A workgroup
// has 8 or 7 compute waves (128 or 112 weight rows).  On layers of >= 192 x
// 128 rows it runs unsplit, on 7 waves when at most 256 workgroups of 112
// rows cover the layer.  Otherwise each wave count gets as many K splits as
// keep the grid within 256 workgroups, and the count with the larger grid
// wins (8 on a tie); that plan is unsplit when it has one split and still
// >= 128 workgroups.  Measured on MI355X (4-bit, M = 128 / 64 / 32, us):
// 28672 x 4096 70.4 / 44.4 / 39.2 -> 66.9 / 44.3 / 38.4; 22016 x 4096 93.9 /
// 52.3 / 50.8 (tile kernels) -> 60.6 / 40.5 / 35.4; 14336 x 4096 (2 splits)
// 45.3 / 30.4 / 26.2 -> 44.2 / 29.0 / 24.9.
RxPlan rx_plan(int64_t M, int64_t N, int64_t K, int64_t pitch, int bits, bool rows32) {
  RxPlan p;
  if (!((bits == 4 || bits == 3) && M > 16 && M <= 384 && (bits == 4 || pitch % 4 == 0))) return p;
  constexpr int64_t k24 = int64_t(1) << 24;
  if (M <= 32 && N <= k24 && K <= k24 && N * K <= k24) return p;
  const int64_t mt = ceil_div(M, 128);
  const int64_t nblk = K / 128, cols8 = ceil_div(N, 128) * mt, cols7 = ceil_div(N, 112) * mt;
  if (nblk <= 0) return p;
  auto splits_for = [&](int64_t cols) {
    const int64_t sp = std::min<int64_t>(nblk, std::max<int64_t>(1, 256 / cols));
    return ceil_div(nblk, ceil_div(nblk, sp));  // no empty split
  };
  int64_t grid = 0;
  if (cols8 >= 192) {
    p.splits = 1;
    p.waves = cols7 <= 256 || cols8 > 256 ? 7 : 8;
    grid = p.waves == 7 ? cols7 : cols8;
  } else {
    const int64_t s8 = splits_for(cols8), s7 = splits_for(cols7);
    const bool w7 = cols7 * s7 > cols8 * s8;
    const int64_t sp = w7 ? s7 : s8;
    grid = w7 ? cols7 * s7 : cols8 * s8;
    if ((sp > 1 && N % 4 != 0) || (sp == 1 && grid < 128)) return p;
    p.splits = static_cast<int>(sp);
    p.waves = w7 ? 7 : 8;
  }
  // 64 < M <= 128: 32 rows per compute wave (7 compute waves, 224 rows per
  // workgroup) read each X fragment for two row blocks, where its grid is at
  // least as large with at most 8 splits (measured, 4-bit M = 128, us: 28672 x
  // 4096 68.3 -> 66.2, 14336 x 4096 44.0 -> 41.9, 13824 x 5120 50.1 -> 46.2,
  // 22016 x 4096 63.2 -> 59.1, 11008 x 4096 40.7 -> 38.8; where its grid is
  // smaller, slower: 16384 x 4096 47.5 -> 48.7, 8192 x 8192 49.6 -> 52.7)
  if (rows32 && M > 64 && M <= 128) {
    const int64_t cols32 = ceil_div(N, 224), s32 = splits_for(cols32);
    if (s32 <= 8 && cols32 * s32 >= grid && (s32 == 1 || N % 4 == 0)) {
      p.splits = static_cast<int>(s32);
      p.waves = 7;
      p.rows = 32;
    }
  }
  return p;
}

// 1 < M <= 16 on layers of 4097-8191 rows: 32-row workgroups (160-255 of
// them; 16-row ones would leave 64-127 CUs with two), and for K >= 8192 K
// split in 3 when that keeps the grid within two workgroups per CU.
// Measured on MI355X, 4-bit M = 16 (M = 8; M = 2): 5120 x 5120 12.9 (11.1;
// 10.2) us against 16.0 (11.9; 11.6) with 16-row workgroups, 5120 x 13824
// split 24.5 (21.2; 20.0) against 37.2 (27.2; 22.1), 6144 x 4096 11.0 (9.7;
// 9.1) against 13.4 (10.2; 9.7).
int reg4_mid_splits(int64_t M, int64_t N, int64_t K) {
  if (!(M > 1 && M <= 16 && N > 4096 && N < 8192)) return 0;
  return K >= 8192 && 3 * ceil_div(N, 32) <= 512 && N % 4 == 0 ? 3 : 1;
}

// 1 < M <= 16 on 8192-row layers: 128 workgroups of 64 rows, so K split in
// 2 (measured on MI355X, 4-bit 8192 x 8192, M = 16 / 4: 21.5 / 19.2 us
// against 26.0 / 22.2 unsplit; on 11008-14336 rows, where the unsplit grid
// is 172-224 workgroups, splitting measured 15-40% slower).
int reg4_wide_splits(int64_t M, int64_t N, int64_t K) {
  return M > 1 && M <= 16 && N >= 8192 && ceil_div(N, 64) * 2 <= 256 && N % 4 == 0 && K >= 256 ? 2 : 0;
}

// 8 < M <= 16 on layers of 3072-4096 rows with K >= 10240: 96-128 workgroups
// of 32 rows (16 waves), K split in 2.  Measured on MI355X (graph-timed, us,
// against 16-row workgroups of 8 waves unsplit): 4-bit M = 16 / 12 at 4096 x
// 14336 16.6 / 15.3 against 19.5 / 17.4, 4096 x 11008 M = 16 14.3 against
// 16.2, 3584 x 14336 16.6 against 19.8; 3-bit at 4096 x 14336 18.8 / 17.9
// against 19.7 / 18.2.  At K = 8192 and at M <= 8 it was no faster than the
// unsplit 16-wave workgroups.
int reg4_narrow_splits(int64_t M, int64_t N, int64_t K) {
  return M > 8 && M <= 16 && N >= 3072 && N <= 4096 && N % 4 == 0 && K >= 10240 ? 2 : 0;
}

size_t round256(size_t b) { return b > SIZE_MAX - 255 ? SIZE_MAX : (b + 255) / 256 * 256; }

size_t splitk_bytes(int64_t M, int64_t N, int64_t K, int bits, int group_size, int x_dtype) {
  if (M <= 0 || N <= 0 || K <= 0 || x_dtype == GPTQ_F32 || K % 128 != 0 || group_size <= 0 || group_size % 32 != 0)
    return 0;
  if (K > INT32_MAX / 8) return 0;  // gptq::linear refuses such K
  const int64_t pitch = (K * bits + 7) / 8;
  // M <= 16: the register path stages <= 128 groups per row
  const int sp = M > 16 ? rx_plan(M, N, K, pitch, bits).splits
                        : (bits == 4 || bits == 3) && ceil_div(K, group_size) <= 128
                              ? std::max({reg4_mid_splits(M, N, K), reg4_wide_splits(M, N, K),
                                          reg4_narrow_splits(M, N, K)})
                              : 0;
  return sp > 1 ? mul_sat(mul_sat(static_cast<size_t>(sp) * sizeof(float), static_cast<size_t>(M)),
                          static_cast<size_t>(N))
                : 0;
}

int check_linear_args(const void* x, int x_dtype, int64_t M, const void* packed, int bits, const void* scales,
                      const void* zeros, int sz_dtype, const int32_t* g_idx, int group_size, int64_t ngroups,
                      const void* bias, int bias_dtype, int64_t N, int64_t K, const void* y) {
  GPTQ_REQUIRE(x && packed && scales && zeros && y, GPTQ_ERR_ARG, "linear: null pointer");
  GPTQ_REQUIRE(bits == 0 || bits == 2 || bits == 3 || bits == 4 || bits == 8, GPTQ_ERR_ARG, "linear: bits=%d", bits);
  GPTQ_REQUIRE(valid_dtype(x_dtype) && valid_dtype(sz_dtype) && (!bias || valid_dtype(bias_dtype)), GPTQ_ERR_DTYPE,
               "linear: bad dtype");
  GPTQ_REQUIRE(M >= 0 && N > 0 && K > 0 && ngroups > 0 && (g_idx || group_size > 0), GPTQ_ERR_SHAPE,
               "linear: bad shape");
  GPTQ_REQUIRE(g_idx || ceil_div(K, group_size) <= ngroups, GPTQ_ERR_SHAPE, "linear: too few groups");
  GPTQ_REQUIRE(K <= INT32_MAX / 8, GPTQ_ERR_SHAPE, "linear: K=%lld too large", static_cast<long long>(K));
  return GPTQ_OK;
}

}  // namespace plan
}  // namespace gptq

using namespace gptq;

// ----------------------------------------------------- workspace queries ----

extern "C" size_t gptq_hessian_workspace_size(int64_t n, int64_t K) {
  if (n <= 0 || K <= 0 || K > (1 << 20)) return 0;
  const int64_t ntiles = plan::hessian_tiles(K);
  return static_cast<size_t>(plan::choose_splits(n, ntiles)) * plan::hessian_split_bytes(K);
}

extern "C" size_t gptq_hessian_workspace_min(int64_t K) {
  if (K <= 0 || K > (1 << 20)) return 0;
  return plan::hessian_split_bytes(K);
}

extern "C" size_t gptq_factor_workspace_size(int64_t K) {
  if (K <= 0 || K > (1 << 17)) return 0;
  // [lambda pad 64 floats][A K*K][scratch]
  return (64 + static_cast<size_t>(K) * K + static_cast<size_t>(plan::factor_scratch_floats(K))) * sizeof(float);
}

extern "C" size_t gptq_sweep_workspace_size(int64_t rows, int64_t cols, int blocksize) {
  (void)cols;
  if (rows <= 0 || blocksize <= 0) return 0;
  const int64_t width = std::max<int64_t>(plan::kSweepSub, plan::sweep_run_blocks(blocksize) * blocksize);
  return plan::mul_sat(static_cast<size_t>(rows), static_cast<size_t>(width) * sizeof(float));
}

extern "C" size_t gptq_linear_perm_workspace_size(int64_t M, int64_t K, int x_dtype) {
  if (M <= 0 || K <= 0 || !valid_dtype(x_dtype)) return 0;
  return plan::mul_sat(plan::mul_sat(static_cast<size_t>(M), static_cast<size_t>(K)),
                       static_cast<size_t>(dtype_size(x_dtype)));
}

extern "C" size_t gptq_linear_workspace_size(int64_t M, int64_t N, int64_t K, int bits, int group_size, int x_dtype,
                                             int has_perm) {
  if (M <= 0 || N <= 0 || K <= 0 || !valid_dtype(x_dtype)) return 0;
  const size_t g = has_perm ? gptq_linear_perm_workspace_size(M, K, x_dtype) : 0;
  const size_t gather = g == SIZE_MAX ? SIZE_MAX : plan::round256(g);
  return plan::add_sat(gather, plan::splitk_bytes(M, N, K, bits, group_size, x_dtype));
}
