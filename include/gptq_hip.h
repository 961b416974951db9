/*
 * gptq_hip.h -- C ABI of the MI355X (gfx950) GPTQ hot-path library
 * (libgptq_hip.so).
 *
 * Plain pointers and sizes only.  Every buffer is a device pointer that the
 * caller allocated and owns; the library never allocates device memory: the
 * scratch it needs comes in through a caller-sized workspace (see the
 * *_workspace_size queries).  Every entry point enqueues on the given HIP
 * stream, returns a gptq_status, and never synchronises the device.  The
 * message of the last failure on the calling thread is gptq_last_error().
 *
 * Matrices are row-major and contiguous unless a leading dimension is given.
 * Each entry point names the reference interface it replaces
 * (kambojvikram/Distributed_GPTQ, paths under src/distributed_gptq/).
 */
#ifndef GPTQ_HIP_H
#define GPTQ_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* gptq_stream_t; /* == hipStream_t */

typedef enum {
  GPTQ_OK = 0,
  GPTQ_ERR_ARG = 1,       /* null pointer, bad enum, bad size          */
  GPTQ_ERR_SHAPE = 2,     /* shapes that the algorithm does not define  */
  GPTQ_ERR_DTYPE = 3,     /* unsupported element type                   */
  GPTQ_ERR_WORKSPACE = 4, /* workspace too small                        */
  GPTQ_ERR_LAUNCH = 5,    /* a kernel launch failed                     */
  GPTQ_ERR_DEVICE = 6     /* no gfx950 device current                   */
} gptq_status;

typedef enum { GPTQ_F32 = 0, GPTQ_F16 = 1, GPTQ_BF16 = 2 } gptq_dtype;

/* Message describing the last error returned on this thread ("" if none). */
const char* gptq_last_error(void);
/* ABI version of this header (bumped on incompatible change). */
int gptq_abi_version(void);

/* ---------------------------------------------------------------- Hessian --
 * H (K x K, fp32, row-major, symmetric) += X^T X, X = n tokens x K features
 * (row stride ldx elements) in fp32, fp16 or bf16.  Only the lower triangle is
 * computed (MFMA tiles); the result is mirrored so H stays a full symmetric
 * matrix.  Products of fp16/bf16 inputs are exact in fp32; fp32 inputs use
 * fp32 MFMA.
 * Replaces GPTQ.add_batch, core/gptq.py:63-89 (H += inp @ inp.t(), :88-89).
 */
size_t gptq_hessian_workspace_size(int64_t n, int64_t K);
int gptq_hessian_accumulate(float* H, const void* X, int64_t n, int64_t K,
                            int64_t ldx, int dtype, void* workspace,
                            size_t workspace_bytes, gptq_stream_t stream);

/* The smallest workspace gptq_hessian_accumulate takes: one token split's
 * partial tiles (ceil(K/256) (ceil(K/256) + 1) / 2 x 256 KB).  With less than
 * gptq_hessian_workspace_size(n, K) the tokens are processed in consecutive
 * runs, each with as many splits as the workspace holds, added to H in token
 * order (deterministic; a little slower).  No counterpart in the reference
 * (its add_batch allocates nothing beyond H); for callers short of memory. */
size_t gptq_hessian_workspace_min(int64_t K);

/* ------------------------------------------------------- damp + factorise --
 * Hd = scale * H[perm][:, perm] (perm may be NULL); if dead_cols is non-NULL,
 * every i with Hd[i][i] == 0 gets Hd[i][i] = 1 and dead_cols[i] = 1 (else 0);
 * then Hd += percdamp * mean(diag(Hd)) * I.  Then, in fp32:
 *   mode GPTQ_FACTOR_FULL_INVERSE: out = Hd^-1 (full, symmetric)
 *     -- replaces core/gptq.py:112-122 (H /= nsamples; damping;
 *        cholesky_inverse(cholesky(H))), with scale = 1/nsamples;
 *   mode GPTQ_FACTOR_UPPER_CHOL_INV: out = U, upper triangular with positive
 *     diagonal and U^T U = Hd^-1 (strict lower part of out is zeroed)
 *     -- the canonical GPTQ factor (fasterquant: chol, cholesky_inverse,
 *        chol(upper)), formed as U = J chol(J Hd J)^-1 J.
 * *info (device int) is set to 0 on success, or to 1 + the first column whose
 * pivot was not positive (H not positive definite after damping).
 * Hd may be NULL if the damped matrix is not wanted.
 */
enum { GPTQ_FACTOR_FULL_INVERSE = 0, GPTQ_FACTOR_UPPER_CHOL_INV = 1 };
size_t gptq_factor_workspace_size(int64_t K);
int gptq_damp_factor(const float* H, int64_t K, float scale, float percdamp,
                     const int32_t* perm, int mode, float* Hd, float* out,
                     int32_t* dead_cols, int32_t* info, void* workspace,
                     size_t workspace_bytes, gptq_stream_t stream);

/* ------------------------------------------------------------ the sweep --
 * Column-blocked quantise-and-propagate over W (rows x cols, fp32, modified
 * in place) with the propagation matrix T (cols x cols fp32, row stride ldt,
 * upper triangle used: U in canonical mode, the leading cols x cols block of
 * the full inverse in reference mode).  Rows are
 * independent.  For each block [i1, i2) of `blocksize` columns, for each
 * column c: q = codes of W[:, c]; e = (W[:, c] - dequant(q)) / T[c][c];
 * W[:, c+1:i2] -= e T[c, c+1:i2]; then, with GPTQ_SWEEP_TRAILING,
 * W[:, i2:] -= E T[i1:i2, i2:] (lazy-batch update, fp32 MFMA).
 * Group parameters (asymmetric min-max) of the group starting at column c
 * are taken, at the start of the block holding c, over columns
 * [c, c + group_size) of W (or of W0 with GPTQ_SWEEP_GROUPS_FROM_W0).
 * group_size <= 0 means one group per row whose parameters are given in
 * scale/zero on entry.
 * Flags:
 *   GPTQ_SWEEP_TRAILING          lazy-batch trailing update (canonical)
 *   GPTQ_SWEEP_REF_QUANTIZER     q = clamp(round(w/s + z)); s, z from raw
 *                                min/max (core/gptq.py:165-175); else the
 *                                canonical q = clamp(round(w/s) + z) with 0
 *                                forced into [min, max] and a zero-range
 *                                guard
 *   GPTQ_SWEEP_GROUPS_FROM_W0    group statistics from W0 (core/gptq.py:162)
 * Outputs (any may be NULL except codes): codes (rows x cols uint8),
 * dequant (rows x cols, dequant_dtype), scale/zero (rows x ngroups fp32),
 * err_sq (rows, fp32: sum over the row of e^2) and losses (rows x cols fp32,
 * (w - dequant)^2 / T[c][c]^2 / 2).  If out_cols is non-NULL, column c of
 * the sweep is stored at column out_cols[c] of codes/dequant/losses (act-order
 * un-permutation); scale/zero stay in sweep order.  out_cols must then be a
 * permutation of [0, cols).
 * Workspace: gptq_sweep_workspace_size(rows, cols, blocksize) bytes (the
 * errors of one run of blocks spanning >= 512 columns: trailing updates are
 * applied per run, an exact re-association of the per-block updates).
 * Replaces GPTQ.quantize, core/gptq.py:91-214 (column loop :132-194), and the
 * canonical fasterquant loop.
 */
enum {
  GPTQ_SWEEP_TRAILING = 1,
  GPTQ_SWEEP_REF_QUANTIZER = 2,
  GPTQ_SWEEP_GROUPS_FROM_W0 = 4
};
size_t gptq_sweep_workspace_size(int64_t rows, int64_t cols, int blocksize);
int gptq_quantize_sweep(float* W, const float* W0, const float* T,
                        int64_t ldt, int64_t rows, int64_t cols, int bits,
                        int group_size,
                        int blocksize, int flags, const int32_t* out_cols,
                        uint8_t* codes, void* dequant, int dequant_dtype,
                        float* scale, float* zero, float* err_sq,
                        float* losses, void* workspace, size_t workspace_bytes,
                        gptq_stream_t stream);

/* Min-max quantisation parameters per row and group of `src` (rows x cols,
 * row stride ld): group g covers columns [g*group_size, (g+1)*group_size)
 * (group_size <= 0: the whole row).  flags: GPTQ_SWEEP_REF_QUANTIZER for the
 * reference formula (core/gptq.py:165-169), else the canonical asymmetric
 * Quantizer.find_params; GPTQ_PARAMS_SYM for the canonical symmetric form
 * (xmax = max(|xmin|, xmax), z = (maxq + 1) / 2).  scale/zero are
 * (rows x ngroups) fp32.
 * Replaces the group statistics block core/gptq.py:159-169. */
enum { GPTQ_PARAMS_SYM = 8 };
int gptq_minmax_params(const float* src, int64_t rows, int64_t cols,
                       int64_t ld, int bits, int group_size, int flags,
                       float* scale, float* zero, gptq_stream_t stream);

/* Quantise rows with given parameters: codes[r][c] = clamp(round(x/s + z))
 * (GPTQ_SWEEP_REF_QUANTIZER, core/gptq.py:175) or clamp(round(x/s) + z),
 * dequant[r][c] = s * (codes - z) (core/gptq.py:179), group of column c =
 * c / group_size (group_size <= 0: one group).  codes and dequant may each be
 * NULL.  x, dequant: (rows x cols) fp32. */
int gptq_quantize_rows(const float* x, int64_t rows, int64_t cols, int bits,
                       int group_size, int flags, const float* scale,
                       const float* zero, uint8_t* codes, float* dequant,
                       gptq_stream_t stream);

/* Convert a layer weight to fp32 in sweep order:
 * out[r][c] = w[r][perm[c]] (transpose == 0; w is rows x cols, row stride
 * ldw) or out[r][c] = w[perm[c]][r] (transpose != 0; w is cols x rows, the
 * reference orientation W = weight.t()), perm may be NULL, and columns whose
 * dead_cols entry (indexed by the original column) is non-zero are set to 0.
 * Replaces W = layer.weight.data.clone().float(); W = W.t()
 * (core/gptq.py:101-108) and the canonical dead-column / act-order
 * preparation. */
int gptq_prepare_weight(const void* w, int dtype, int64_t rows, int64_t cols,
                        int64_t ldw, const int32_t* perm,
                        const int32_t* dead_cols, int transpose, float* out,
                        gptq_stream_t stream);

/* ------------------------------------------------------- packing formats --
 * Native packed layout: each row of (N x K) codes is an LSB-first bit stream
 * of `bits`-bit fields, ceil(K*bits/8) bytes per row (unused high bits of a
 * row's last byte are 0).  For 4-bit
 * this is QuantizedLinear.pack_weights (models/layers.py:67-96: byte =
 * w[:, i] | w[:, i+1] << 4); for 2/4/8-bit, read as little-endian int32 it is
 * pack_weights_kernel (kernels/triton_kernels.py:186-222).  3-bit: 32 codes
 * per three 32-bit words.  bits in {2,3,4,8}.
 */
int gptq_pack(const uint8_t* codes, int64_t N, int64_t K, int bits,
              uint8_t* packed, gptq_stream_t stream);
int gptq_unpack(const uint8_t* packed, int64_t N, int64_t K, int bits,
                uint8_t* codes, gptq_stream_t stream);

/* GPTQ.pack_weights layout (core/gptq.py:216-266) from codes (N x K): works
 * on W = codes^T (K x N).  bits 4: out (K x N/2) byte = 16*W[:, 2i] +
 * W[:, 2i+1]; bits 2: out (K x N/4) with weights 64,16,4,1; bits 3 and 8:
 * out (K x N) = W cast to uint8 (the int8 view of 8-bit wraps at 128). */
int gptq_pack_reference_layout(const uint8_t* codes, int64_t N, int64_t K,
                               int bits, uint8_t* out, gptq_stream_t stream);

/* W[n][k] = (q[n][k] - zeros[n][g]) * scales[n][g] in fp32 (no FMA), with
 * g = g_idx[k] (g_idx NULL: g = k / group_size).  q comes from `packed` in
 * the native layout of `bits`, or, with bits == 0, one code per byte (N x K
 * uint8, the reference's unpacked storage).  scales/zeros: (N x ngroups) in
 * sz_dtype (fp16 in QuantizedLinear, fp32 elsewhere).
 * Replaces QuantizedLinear.unpack_weights (models/layers.py:98-138),
 * GPTQDequantizer.dequantize_weight (core/dequantizer.py:31-66). */
int gptq_dequant(const uint8_t* packed, int bits, const void* scales,
                 const void* zeros, int sz_dtype, const int32_t* g_idx,
                 int group_size, int64_t ngroups, int64_t N, int64_t K,
                 float* out, gptq_stream_t stream);

/* gptq_dequant with W stored in out_dtype (GPTQ_F32, GPTQ_F16 or
 * GPTQ_BF16): the fp32 value above rounded once to the output type, i.e. the
 * weight the reference's fallback F.linear(x, unpack_weights(), bias)
 * multiplies in x's dtype (models/layers.py:155-157).  Serves gptq::linear
 * for many rows of x as this dequantisation plus a library GEMM. */
int gptq_dequant_to(const uint8_t* packed, int bits, const void* scales,
                    const void* zeros, int sz_dtype, const int32_t* g_idx,
                    int group_size, int64_t ngroups, int64_t N, int64_t K,
                    void* out, int out_dtype, gptq_stream_t stream);

/* ------------------------------------------------ dequant GEMV / GEMM --
 * y[M x N] = x[M x K] @ W^T (+ bias), W as in gptq_dequant, fp32
 * accumulation, x/y in x_dtype (fp16, bf16 or fp32), bias (N) in bias_dtype
 * or NULL.  Weights are streamed once per 16 rows of x with 128-bit loads.
 * Replaces torch.ops.gptq.linear, the call at models/layers.py:151-153 whose
 * semantics are F.linear(x, unpack_weights(), bias) (:155-157), and
 * quantized_matmul_kernel (kernels/triton_kernels.py:126-183). */
int gptq_linear(const void* x, int x_dtype, int64_t M, const uint8_t* packed,
                int bits, const void* scales, const void* zeros, int sz_dtype,
                const int32_t* g_idx, int group_size, int64_t ngroups,
                const void* bias, int bias_dtype, int64_t N, int64_t K,
                void* y, gptq_stream_t stream);

/* gptq_linear with a caller workspace (perm may be NULL): with perm, x is
 * gathered through it into the workspace first (as gptq_linear_perm); the
 * rest of the workspace (from its first 256-byte boundary) lets the kernels
 * for 1 < M <= 384 split K over more workgroups on narrower layers, their
 * fp32 partial sums reduced in split order (deterministic).
 * gptq_linear_workspace_size gives the bytes for both (has_perm: 0 or 1);
 * with less, the layer runs as gptq_linear would.
 * Same semantics as gptq_linear; no counterpart in the reference beyond
 * torch.ops.gptq.linear (models/layers.py:151-157). */
size_t gptq_linear_workspace_size(int64_t M, int64_t N, int64_t K, int bits,
                                  int group_size, int x_dtype, int has_perm);
int gptq_linear_ws(const void* x, int x_dtype, int64_t M, const int32_t* perm,
                   const uint8_t* packed, int bits, const void* scales,
                   const void* zeros, int sz_dtype, const int32_t* g_idx,
                   int group_size, int64_t ngroups, const void* bias,
                   int bias_dtype, int64_t N, int64_t K, void* y,
                   void* workspace, size_t workspace_bytes,
                   gptq_stream_t stream);

/* y = x[:, perm] @ W^T (+ bias), W and the other arguments as in
 * gptq_linear: the act-order serving layout, where weight column j holds
 * input column perm[j] (perm: K int32, a permutation of [0, K); entries
 * outside [0, K) are clamped) so that groups are contiguous in the stored
 * order and the fast kernels serve the layer.  The gathered x
 * (gptq_linear_perm_workspace_size bytes) is written to the workspace first,
 * by one small kernel, then the kernels of gptq_linear read it.
 * Replaces torch.ops.gptq.linear (models/layers.py:151-153) for GPTQ
 * act-order output, whose g_idx (:60) maps input columns to groups out of
 * order; semantics F.linear(x, unpack_weights(), bias) (:155-157). */
size_t gptq_linear_perm_workspace_size(int64_t M, int64_t K, int x_dtype);
int gptq_linear_perm(const void* x, int x_dtype, int64_t M, const int32_t* perm,
                     const uint8_t* packed, int bits, const void* scales,
                     const void* zeros, int sz_dtype, const int32_t* g_idx,
                     int group_size, int64_t ngroups, const void* bias,
                     int bias_dtype, int64_t N, int64_t K, void* y,
                     void* workspace, size_t workspace_bytes,
                     gptq_stream_t stream);

/* gptq_linear_perm without a workspace: for callers that cannot allocate
 * (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  The gathered activations go
 * to a static device array of gptq_linear_perm_noalloc_max_bytes() bytes
 * (4 MiB) that each GPU holds until the process ends; M * K * sizeof(x
 * element) above that is refused with GPTQ_ERR_WORKSPACE.  Nothing is
 * allocated or freed.  All calls on one GPU share that array: calls that
 * overlap on one GPU (different streams, no ordering between them) race.
 * Otherwise as gptq_linear_perm. */
size_t gptq_linear_perm_noalloc_max_bytes(void);
int gptq_linear_perm_noalloc(const void* x, int x_dtype, int64_t M,
                             const int32_t* perm, const uint8_t* packed,
                             int bits, const void* scales, const void* zeros,
                             int sz_dtype, const int32_t* g_idx,
                             int group_size, int64_t ngroups, const void* bias,
                             int bias_dtype, int64_t N, int64_t K, void* y,
                             gptq_stream_t stream);

/* ------------------------------------------------- elementwise quantise --
 * Flat groups of group_size consecutive elements (the tensor API of
 * kernels/triton_kernels.py:377-481): per group s = (max - min) / maxq,
 * z = -min / s (not rounded, :410-411), then
 * q = clamp(round(x / s + z), 0, maxq) (quantize_kernel, :34-79; round half
 * away from zero) stored as the low byte in int8; and the inverse
 * (q - z) * s with q read as int8 (dequantize_kernel, :82-123).
 * flags & GPTQ_TENSOR_PARAMS_GIVEN: scales/zeros are inputs and only the
 * elementwise pass runs (TritonQuantizedLinear.quantize_weights, :299-308).
 */
enum { GPTQ_TENSOR_PARAMS_GIVEN = 1 };
int gptq_quantize_tensor(const void* x, int dtype, int64_t n, int bits,
                         int group_size, int flags, int8_t* q, float* scales,
                         float* zeros, gptq_stream_t stream);
int gptq_dequantize_tensor(const int8_t* q, int64_t n, int group_size,
                           const float* scales, const float* zeros, float* out,
                           gptq_stream_t stream);

/* ------------------------------------------------------- measurement aid --
 * No counterpart in the reference: a read-only streaming kernel for the
 * benchmark.  It reads `bytes` bytes of `buf` (both multiples of 16 bytes)
 * with 16-byte non-temporal loads in a grid-stride loop of `blocks`
 * workgroups of 256 threads, `unroll` (1, 2, 4 or 8) loads in flight per
 * thread, and writes *flag = 1 only if a thread's XOR of its data equals a
 * fixed value (so the reads are kept).  Timed at a GEMV's byte count it
 * gives what one launch can read: the ceiling the M = 1 GEMV is compared
 * with. */
int gptq_stream_read(const void* buf, size_t bytes, int blocks, int unroll,
                     uint32_t* flag, gptq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* GPTQ_HIP_H */
