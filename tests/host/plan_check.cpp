// Host-side checks of libgptq_hip.so's planning code (csrc/plan.cpp,
// csrc/status.cpp), built with g++ under AddressSanitizer and
// UndefinedBehaviorSanitizer by tests/test_host_sanitizer.py.  No GPU, no HIP.
//
// It walks the workspace queries and the internal plans (Hessian token
// splits and runs, factor recursion scratch, the register-decoded GEMM plan,
// the split-K rules, the gptq::linear argument checks) over grids of shapes
// including extreme sizes, checks the properties each must have, and prints
// every workspace query's result as "name args = value" so that the test can
// compare them with the shipped library's.  Exit status 0 = every check held.
#include <cinttypes>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../distributed_gptq_amd/csrc/plan.hpp"

using namespace gptq;

static int g_fail = 0;
#define CHECK(cond, ...)                                  \
  do {                                                    \
    if (!(cond)) {                                        \
      std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
      std::fprintf(stderr, __VA_ARGS__);                  \
      std::fprintf(stderr, "\n");                         \
      ++g_fail;                                           \
    }                                                     \
  } while (0)

static const int64_t kSizes[] = {1, 2, 3, 7, 31, 32, 33, 127, 128, 129, 255, 256, 257, 511, 512, 768, 1000, 1024,
                                 2048, 3072, 4096, 5120, 5888, 6144, 8192, 8229, 11008, 13824, 14336, 16384, 16389,
                                 22016, 24576, 28672, 32768, 65536, 131072, 262144, 524288, 1048576, 1048577,
                                 int64_t(1) << 31, int64_t(1) << 40, INT64_MAX / 4};

static void hessian_checks() {
  for (int64_t K : kSizes) {
    const size_t mn = gptq_hessian_workspace_min(K);
    std::printf("gptq_hessian_workspace_min %" PRId64 " = %zu\n", K, mn);
    if (K > (1 << 20)) {
      CHECK(mn == 0, "workspace_min(K=%" PRId64 ") = %zu beyond the supported K", K, mn);
      continue;
    }
    const int64_t nt = plan::hessian_tiles(K);
    const int64_t T = plan::ceil_div(K, plan::kHessTile);
    CHECK(nt == T * (T + 1) / 2 && nt >= 1, "tiles(K=%" PRId64 ") = %" PRId64, K, nt);
    CHECK(mn == static_cast<size_t>(nt) * 256 * 256 * 4, "workspace_min(K=%" PRId64 ")", K);
    for (int64_t n : kSizes) {
      const int S = plan::choose_splits(n, nt);
      CHECK(S >= 1 && S <= 64, "choose_splits(%" PRId64 ", %" PRId64 ") = %d", n, nt, S);
      // tokens per split: <= 10240 below 512 tiles, <= 16384 below 1024, and
      // from 1024 tiles on <= 65536 with at least 4 splits of > 16384
      const int64_t tok_max = nt < 512 ? 10240 : nt < 1024 ? 16384 : 65536;
      CHECK(S == 64 || S >= plan::ceil_div(n, tok_max), "too few splits for n=%" PRId64, n);
      if (nt >= 1024) {
        CHECK(S == 64 || S >= std::min<int64_t>(4, plan::ceil_div(n, 16384)), "too few splits for n=%" PRId64, n);
        CHECK(S <= std::max<int64_t>(4, plan::ceil_div(n, 65536)), "too many splits for n=%" PRId64, n);
      }
      const size_t ws = gptq_hessian_workspace_size(n, K);
      std::printf("gptq_hessian_workspace_size %" PRId64 " %" PRId64 " = %zu\n", n, K, ws);
      CHECK(ws == static_cast<size_t>(S) * mn, "workspace_size(%" PRId64 ", %" PRId64 ")", n, K);
    }
    // runs with a workspace of `cap` splits: every run fits, and they cover n
    for (int64_t cap = 1; cap <= 64; cap = cap * 2 + 1) {
      const int64_t run = plan::hessian_run_tokens(nt, cap);
      CHECK(run >= 1024 && (plan::choose_splits(run, nt) <= cap || run <= 1024), "run(%" PRId64 ", cap %" PRId64
            ") = %" PRId64, nt, cap, run);
      const int64_t n = 262144 + 37;
      int64_t covered = 0, runs = 0;
      for (int64_t t0 = 0; t0 < n; t0 += run, ++runs) covered += (n - t0 < run ? n - t0 : run);
      CHECK(covered == n && runs == plan::ceil_div(n, run), "runs do not cover n");
    }
  }
}

static void factor_sweep_checks() {
  for (int64_t K : kSizes) {
    const size_t ws = gptq_factor_workspace_size(K);
    std::printf("gptq_factor_workspace_size %" PRId64 " = %zu\n", K, ws);
    if (K > (1 << 17)) {
      CHECK(ws == 0, "factor workspace beyond the supported K");
      continue;
    }
    // the recursion: halves of whole leaves; the scratch of a node of size m
    // is m^2 / 2 at most plus its right child's, so at most 2 K^2 / 3 (+ the
    // uneven halves' slack)
    const int64_t m1 = plan::factor_split(K);
    CHECK(K <= plan::kFactorLeaf || (m1 % plan::kFactorLeaf == 0 && m1 > 0 && m1 < K), "split(%" PRId64 ")", K);
    const int64_t sc = plan::factor_scratch_floats(K);
    CHECK(sc >= 0 && 3 * sc <= 2 * K * K + 3 * plan::kFactorLeaf * K, "scratch(%" PRId64 ") = %" PRId64, K, sc);
    CHECK(ws == (64 + static_cast<size_t>(K) * K + static_cast<size_t>(sc)) * 4, "factor workspace");
    for (int bs : {1, 32, 64, 127, 128, 256, 512, 1024, 4096}) {
      const size_t sw = gptq_sweep_workspace_size(K, K, bs);
      std::printf("gptq_sweep_workspace_size %" PRId64 " %" PRId64 " %d = %zu\n", K, K, bs, sw);
      const int64_t fb = plan::sweep_run_blocks(bs);
      CHECK(fb * bs >= plan::kSweepRun || fb == 1, "run blocks(%d) = %" PRId64, bs, fb);
      CHECK(sw >= static_cast<size_t>(K) * plan::kSweepSub * 4, "sweep workspace too small");
    }
  }
  CHECK(gptq_sweep_workspace_size(0, 10, 128) == 0 && gptq_sweep_workspace_size(10, 10, 0) == 0, "empty sweep");
  // sizes past what size_t holds saturate instead of wrapping
  CHECK(gptq_sweep_workspace_size(INT64_MAX, 1, 128) == SIZE_MAX, "sweep size does not saturate");
  CHECK(gptq_sweep_workspace_size(INT64_MAX / 8, 1, 1 << 30) == SIZE_MAX, "sweep size does not saturate");
  CHECK(gptq_hessian_workspace_size(INT64_MAX, 4096) == 64 * gptq_hessian_workspace_min(4096), "hessian at n max");
  CHECK(plan::ceil_div(INT64_MAX, 2) == INT64_MAX / 2 + 1 && plan::ceil_div(10, 5) == 2, "ceil_div");
}

static void linear_checks() {
  const int64_t Ms[] = {0, 1, 2, 3, 4, 5, 16, 17, 24, 32, 33, 40, 64, 65, 96, 100, 128, 129, 150, 192, 256, 300,
                        384, 385, 16384, int64_t(1) << 31, int64_t(1) << 40};
  for (int64_t M : Ms)
    for (int64_t N : kSizes)
      for (int64_t K : {int64_t(128), int64_t(256), int64_t(1000), int64_t(1024), int64_t(4096), int64_t(5120),
                        int64_t(13824), int64_t(14336), int64_t(17408), int64_t(1) << 20, int64_t(1) << 31,
                        int64_t(1) << 40})
        for (int bits : {0, 2, 3, 4, 8})
          for (int gs : {-1, 32, 64, 128, 1000}) {
            const int64_t pitch = (K * (bits ? bits : 8) + 7) / 8;
            const plan::RxPlan p = plan::rx_plan(M, N, K, pitch, bits);
            if (p.splits > 0) {
              const int64_t nblk = K / 128;
              CHECK((bits == 4 || bits == 3) && M > 16 && M <= 384, "rx plan outside its shapes");
              CHECK(p.waves == 7 || p.waves == 8, "waves %d", p.waves);
              CHECK(p.rows == 16 || (p.rows == 32 && p.waves == 7 && M > 64 && M <= 128), "rows %d", p.rows);
              CHECK(p.splits <= nblk, "more splits than blocks");
              const int64_t per = plan::ceil_div(nblk, p.splits);
              CHECK((p.splits - 1) * per < nblk, "empty split: %d splits of %" PRId64 " blocks", p.splits, nblk);
              CHECK(p.splits == 1 || N % 4 == 0, "split with N %% 4 != 0");
            }
            const int mid = plan::reg4_mid_splits(M, N, K), wide = plan::reg4_wide_splits(M, N, K);
            CHECK(mid >= 0 && mid <= 3 && wide >= 0 && wide <= 2, "reg4 splits %d %d", mid, wide);
            for (int dt : {int(GPTQ_F32), int(GPTQ_F16), int(GPTQ_BF16)}) {
              const size_t sk = plan::splitk_bytes(M, N, K, bits, gs, dt);
              CHECK(sk == 0 || (dt != GPTQ_F32 && K % 128 == 0), "split-K for a layout the kernels do not take");
              for (int perm = 0; perm < 2; ++perm) {
                const size_t ws = gptq_linear_workspace_size(M, N, K, bits, gs, dt, perm);
                if (M > 0 && N > 0 && bits == 4 && (gs == 128 || gs == -1) && K <= (int64_t(1) << 20) &&
                    N <= 32768 && M <= 16384)
                  std::printf("gptq_linear_workspace_size %" PRId64 " %" PRId64 " %" PRId64 " %d %d %d %d = %zu\n",
                              M, N, K, bits, gs, dt, perm, ws);
              }
            }
          }
  for (int64_t M : Ms)
    for (int64_t K : kSizes)
      for (int dt : {int(GPTQ_F32), int(GPTQ_F16), int(GPTQ_BF16), 7}) {
        const size_t ws = gptq_linear_perm_workspace_size(M, K, dt);
        CHECK((M > 0 && K > 0 && dt != 7) || ws == 0, "perm workspace for an empty or bad input");
      }
  CHECK(gptq_linear_perm_workspace_size(INT64_MAX, INT64_MAX, GPTQ_F16) == SIZE_MAX, "perm size does not saturate");
  CHECK(gptq_linear_workspace_size(INT64_MAX, 4096, 4096, 4, 128, GPTQ_F16, 1) == SIZE_MAX, "linear size saturates");
  CHECK(gptq_linear_workspace_size(128, INT64_MAX, INT64_MAX, 4, 128, GPTQ_F16, 0) == 0, "linear size for bad K");
  // argument checks: every failure is reported with the right status
  int dummy = 0;
  const void* p = &dummy;
  const int32_t gi[1] = {0};
  struct Case {
    int want;
    const void *x, *packed, *scales, *zeros, *y;
    int x_dtype, bits, sz_dtype, gs;
    const int32_t* g_idx;
    int64_t M, N, K, ngroups;
  } cases[] = {
      {GPTQ_OK, p, p, p, p, p, GPTQ_F16, 4, GPTQ_F16, 128, nullptr, 1, 4096, 4096, 32},
      {GPTQ_OK, p, p, p, p, p, GPTQ_BF16, 3, GPTQ_F32, 64, nullptr, 0, 8, 128, 2},
      {GPTQ_OK, p, p, p, p, p, GPTQ_F32, 0, GPTQ_BF16, 0, gi, 5, 3, 200, 4},
      {GPTQ_ERR_ARG, nullptr, p, p, p, p, GPTQ_F16, 4, GPTQ_F16, 128, nullptr, 1, 16, 128, 1},
      {GPTQ_ERR_ARG, p, p, p, p, nullptr, GPTQ_F16, 4, GPTQ_F16, 128, nullptr, 1, 16, 128, 1},
      {GPTQ_ERR_ARG, p, p, p, p, p, GPTQ_F16, 5, GPTQ_F16, 128, nullptr, 1, 16, 128, 1},
      {GPTQ_ERR_DTYPE, p, p, p, p, p, 9, 4, GPTQ_F16, 128, nullptr, 1, 16, 128, 1},
      {GPTQ_ERR_DTYPE, p, p, p, p, p, GPTQ_F16, 4, -1, 128, nullptr, 1, 16, 128, 1},
      {GPTQ_ERR_SHAPE, p, p, p, p, p, GPTQ_F16, 4, GPTQ_F16, 128, nullptr, -1, 16, 128, 1},
      {GPTQ_ERR_SHAPE, p, p, p, p, p, GPTQ_F16, 4, GPTQ_F16, 128, nullptr, 1, 0, 128, 1},
      {GPTQ_ERR_SHAPE, p, p, p, p, p, GPTQ_F16, 4, GPTQ_F16, 0, nullptr, 1, 16, 128, 1},
      {GPTQ_ERR_SHAPE, p, p, p, p, p, GPTQ_F16, 4, GPTQ_F16, 64, nullptr, 1, 16, 256, 3},
      {GPTQ_ERR_SHAPE, p, p, p, p, p, GPTQ_F16, 4, GPTQ_F16, 128, nullptr, 1, 16, int64_t(1) << 40, int64_t(1) << 40},
      {GPTQ_ERR_SHAPE, p, p, p, p, p, GPTQ_F16, 4, GPTQ_F16, 128, nullptr, 1, 16, INT64_MAX, INT64_MAX},
  };
  for (const Case& c : cases) {
    clear_error();
    const int rc = plan::check_linear_args(c.x, c.x_dtype, c.M, c.packed, c.bits, c.scales, c.zeros, c.sz_dtype,
                                           c.g_idx, c.gs, c.ngroups, nullptr, 0, c.N, c.K, c.y);
    CHECK(rc == c.want, "check_linear_args: %d, expected %d (%s)", rc, c.want, gptq_last_error());
    CHECK((rc == GPTQ_OK) == (gptq_last_error()[0] == '\0'), "an error without a message, or the reverse");
  }
}

int main() {
  hessian_checks();
  factor_sweep_checks();
  linear_checks();
  std::fprintf(stderr, "%d check(s) failed\n", g_fail);
  return g_fail ? 1 : 0;
}
