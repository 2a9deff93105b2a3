/*
 * locomp_amd C ABI: int4 / int8 weight-only dequantize and dequant-matmul on
 * AMD Instinct MI355X (gfx950).
 *
 * This is the drop-in boundary for locomp's quantized-inference path.  In the
 * reference (Zyora-Dev/locomp v1.0.0) every kernel launch reaches the GPU
 * through a per-kernel generated shared object exporting
 *     extern "C" void locomp_launch_<name>(int grid_x, int grid_y,
 *                                          int block_x, int block_y,
 *                                          void** args);
 * (locomp/backends/rocm_codegen.py:304-340), bound with ctypes in
 * locomp/api.py:949-990, with the kernel's integer constexprs baked into the
 * generated source.  Each entry point below replaces one such generated
 * launcher: it takes the same pointer arguments in the same order, then the
 * same integer arguments in the same order (now run-time values), then the
 * grid extent (rows N), then the extensions the reference lacks (activation
 * rows M, element dtypes, a HIP stream).
 *
 * Conventions
 *   - All pointers are device pointers.  The library allocates only
 *     grow-only workspaces per (device, stream): on the first prefill that
 *     splits K, on the first SiLU * mul call without a fused kernel, and on
 *     the first fp32-activation call (its bf16 part rows: 24 K bytes at
 *     M <= 4; at M > 4 2 M K x 2 bytes, plus the parts' fp32 products,
 *     2 M N x 4 bytes, where 2 M <= 64; each at most 256 MB, larger M in
 *     row blocks); they
 *     are held until the process ends or locomp_amd_release_workspaces.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = default stream) and
 *     is asynchronous: the caller synchronises.
 *   - Return value: 0 on success; a negative LQ_ERR_* for invalid arguments
 *     (nothing is launched); a positive hipError_t if the launch failed.
 *   - Layouts (locomp examples/38_quantized_matmul.py:30-134,
 *     examples/52_dequantize.py:27-74):
 *       int4 W: uint8 [N, K/2], byte j of row n = (q[n,2j+1] << 4) | q[n,2j],
 *               value (q - 8) * s
 *       int8 W: int8  [N, K],   value q * s
 *       scales: [N, K/G] row-major, s[n, k / G]  (G = K: per output channel)
 *       X: [M, K] row-major;  O: [M, N] row-major;  O = X @ dequant(W)^T
 *   - Dequantised values are float32(q - 8) * float32(s), rounded once to
 *     the output dtype (bit-exact with the reference's NumPy path).
 */
#ifndef LOCOMP_AMD_H_
#define LOCOMP_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LOCOMP_AMD_ABI_VERSION 5

/* Element dtype codes. */
enum {
  LQ_F32 = 0,  /* locomp.Tensor (float32)           */
  LQ_F16 = 1,  /* locomp.Float16                    */
  LQ_BF16 = 2  /* locomp.BFloat16 (stored as 16 bits) */
};

/* Error codes (negative; positive values are hipError_t). */
enum {
  LQ_OK = 0,
  LQ_ERR_SHAPE = -1,   /* inconsistent or unsupported sizes           */
  LQ_ERR_DTYPE = -2,   /* unknown dtype code                          */
  LQ_ERR_NULL = -3,    /* null pointer with a non-empty problem        */
  LQ_ERR_POLICY = -4,  /* unknown kernel policy                        */
  LQ_ERR_SCRATCH = -5, /* needs scratch that is not available: more than the
                          fixed buffer holds, or a workspace that cannot be
                          allocated during stream capture */
  LQ_ERR_NAME = -6     /* unknown kernel name (locomp_amd_launch)        */
};

/* Quantizer variants (locomp_amd_quantize_int4). */
enum {
  LQ_QUANT_EX38 = 0,  /* quantize_int4, examples/38_quantized_matmul.py:248-271 */
  LQ_QUANT_EX52 = 1   /* quantize_int4_ref, examples/52_dequantize.py:110-126 */
};

/* Kernel policies (locomp_amd_set_policy). */
enum {
  LQ_POLICY_AUTO = 0,    /* fastest applicable kernel (default)          */
  LQ_POLICY_GENERIC = 1  /* always the shape-generic kernels (for tests)  */
};

/* ABI version of the loaded library (== LOCOMP_AMD_ABI_VERSION). */
int locomp_amd_abi_version(void);

/* Static description of an error code (never NULL). */
const char* locomp_amd_strerror(int code);

/* Select the kernel policy for subsequent calls from this process.
 * No counterpart in the reference (it has one generated kernel per shape);
 * used by tests to run the shape-generic kernels on the same inputs. */
int locomp_amd_set_policy(int policy);
int locomp_amd_get_policy(void);

/* Frees the fp32 workspaces the library keeps for `stream` on the current
 * device (all streams of the device if all_streams != 0), including buffers
 * superseded when a workspace grew; waits for the device to be idle first.
 * The next call that needs a workspace allocates it again.  A HIP graph
 * captured before the release that names one of them must not be replayed,
 * and no other library call may run on that device concurrently with the
 * release (a call on another host thread may already hold a workspace
 * pointer that the release frees).  No counterpart in the reference (which
 * allocates nothing across calls). */
int locomp_amd_release_workspaces(void* stream, int all_streams);

/* Dequantize int4 -> OUT [N, K].
 * Replaces locomp_launch_dequant_int4 generated for
 * examples/52_dequantize.py:27-53 (args W, SCALES, OUT, K, HALF_K,
 * NUM_SCALES, GROUP_SIZE; grid (N,), launched at examples/52_dequantize.py:90). */
int locomp_amd_dequant_int4(const void* W, const void* SCALES, void* OUT,
                            int64_t K, int64_t HALF_K, int64_t NUM_SCALES,
                            int64_t GROUP_SIZE, int64_t N,
                            int scale_dtype, int out_dtype, void* stream);

/* Dequantize int8 -> OUT [N, K].
 * Replaces locomp_launch_dequant_int8 generated for
 * examples/52_dequantize.py:60-74 (args W, SCALES, OUT, K, NUM_SCALES,
 * GROUP_SIZE; grid (N,), launched at examples/52_dequantize.py:104). */
int locomp_amd_dequant_int8(const void* W, const void* SCALES, void* OUT,
                            int64_t K, int64_t NUM_SCALES, int64_t GROUP_SIZE,
                            int64_t N, int scale_dtype, int out_dtype,
                            void* stream);

/* O [M, N] = X [M, K] @ dequant_int4(W)^T, fp32 accumulation.
 * Replaces locomp_launch_dequant_matvec_int4 generated for
 * examples/38_quantized_matmul.py:30-87 (args X, W, scales, O, K_dim, HALF_K,
 * NUM_SCALES, GROUP_SIZE; grid (N,), launched at
 * examples/38_quantized_matmul.py:154).  M = 1 is the reference's matvec;
 * M <= 64 runs the decode (skinny) kernel, larger M the prefill MFMA GEMM.
 * Activations may be fp16, bf16 or fp32 (the reference's dtype): fp16 and
 * bf16 run on fp16 / bf16 matrix cores at every M (the row kernel at
 * M <= 2 with G % 32: bf16 dot products); fp32 at M <= 4 runs on bf16
 * matrix cores: at M = 1 on the segment kernel (K >= 2048, G % 128 == 0) as
 * two round-to-nearest bf16 parts (|x - hi - lo| <= 2^-16 |x|), at
 * 2 <= M <= 4 (and M = 1 where the segment kernel does not apply) as three
 * exact bf16 parts (split once per call into a workspace, or inside the
 * kernel on a capturing stream that has none yet and on small matrices),
 * except M = 1 with K <= 4096 where the segment kernel does not apply
 * (K < 2048 or G % 128 != 0), which takes fp32 FMAs on the row kernel;
 * fp32 at M > 4 is split into two round-to-nearest parts, 2 M bf16 rows
 * (row 2i + p = part p of row i) that take the bf16 kernels (2 M <= 64 the
 * decode kernels, else the MFMA GEMM, G % 32 == 0), whose stores add each
 * row's two part products (error at most 2^-16 sum_k |x_k w_nk| beyond
 * fp32 summation).  int4 scale groups G % 16 == 0 but G % 32 != 0 at
 * M <= 2 (fp32: M = 1, K <= 4096) take the row kernel with a scale per 16 k;
 * other scale groups G % 32 != 0 (G % 8 == 0; int8 G % 4),
 * operands aligned to 4 but not 16 bytes, fp32 shapes below 2^24
 * multiply-adds and a capture on a stream without the part-row workspace
 * take a VALU kernel with fp32 FMAs (fp16 / bf16: exact dot2 products);
 * anything else a generic kernel.  The MFMA kernels need X and W 16-byte
 * aligned and the scales 4-byte aligned.
 * A prefill GEMM with fewer output tiles than CUs splits K and keeps an fp32
 * workspace per (device, stream), allocated on first use and held until the
 * process ends (int4 and int8 alike). */
int locomp_amd_dequant_matvec_int4(const void* X, const void* W,
                                   const void* scales, void* O,
                                   int64_t K_dim, int64_t HALF_K,
                                   int64_t NUM_SCALES, int64_t GROUP_SIZE,
                                   int64_t N, int64_t M, int x_dtype,
                                   int scale_dtype, int out_dtype,
                                   void* stream);

/* As locomp_amd_dequant_matvec_int4, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  Same kernels; the
 * split-K prefill's fp32 partials (and the bf16 part rows of fp32 activations
 * at M <= 4) go to a fixed 32 MiB array in the library's device memory (one
 * per GPU, held until the process ends) instead of the per-stream workspaces,
 * and the call allocates nothing.  Where the allocating entry would split K
 * only for speed and the partials (M x N x 4 bytes x splits) exceed the
 * array, this entry runs the unsplit GEMM instead (same results to the
 * matmul tolerance, not bit for bit).  It returns LQ_ERR_SCRATCH, launching
 * nothing, only when a split is required and does not fit: bf16 activations
 * whose groups per split exceed what the GEMM stages (more than 64 scale
 * groups in K, e.g. K = 8192 with G = 32 at M x N > 2 M outputs).  All calls
 * on one GPU share its array: calls that overlap in time on one GPU (several
 * streams or threads) race and must be serialised by the caller. */
int locomp_amd_dequant_matvec_int4_noalloc(const void* X, const void* W,
                                           const void* scales, void* O,
                                           int64_t K_dim, int64_t HALF_K,
                                           int64_t NUM_SCALES, int64_t GROUP_SIZE,
                                           int64_t N, int64_t M, int x_dtype,
                                           int scale_dtype, int out_dtype,
                                           void* stream);

/* O [M, N] = X [M, K] @ dequant_int8(W)^T, fp32 accumulation.
 * Replaces locomp_launch_dequant_matvec_int8 generated for
 * examples/38_quantized_matmul.py:94-134 (args X, W, scales, O, K_dim,
 * NUM_SCALES, GROUP_SIZE; grid (N,), launched at
 * examples/38_quantized_matmul.py:170) and its copy quant_matvec_int8 in
 * examples/58_benchmark_suite.py:241-264. */
int locomp_amd_dequant_matvec_int8(const void* X, const void* W,
                                   const void* scales, void* O,
                                   int64_t K_dim, int64_t NUM_SCALES,
                                   int64_t GROUP_SIZE, int64_t N, int64_t M,
                                   int x_dtype, int scale_dtype,
                                   int out_dtype, void* stream);

/* SmolLM2-style MLP front half in one launch: W holds the int4 gate and up
 * projections with their rows interleaved (row 2i = gate_i, row 2i + 1 =
 * up_i; uint8 [2I, K/2], scales [2I, K/G]) and
 *     O[m, i] = silu(g) * u,  g = X[m] . deq(W[2i]),  u = X[m] . deq(W[2i + 1]),
 *     silu(g) = g / (1 + exp(-g)),  O: [M, I].
 * Replaces two dequant_matvec_int4 launches plus silu_mul_kernel
 * (examples/54_smollm2_inference.py:113-120, 545-548); arguments as
 * locomp_amd_dequant_matvec_int4 with I = intermediate size (half the rows).
 * One launch where a fused kernel covers the shape (fp32 activations: a
 * split into two bf16 part rows per row, in the stream's workspace, then
 * one fused launch); otherwise the matvec is staged in an fp32
 * per-(device, stream) buffer held until the process ends (M x 2I x 4
 * bytes) and an epilogue kernel follows. */
int locomp_amd_dequant_matvec_int4_silu_mul(const void* X, const void* W, const void* scales,
                                            void* O, int64_t K_dim, int64_t HALF_K,
                                            int64_t NUM_SCALES, int64_t GROUP_SIZE, int64_t I,
                                            int64_t M, int x_dtype, int scale_dtype, int out_dtype,
                                            void* stream);

/* One entry for every kernel above, in the reference's generated-launcher
 * convention: locomp_launch_<name>(grid_x, grid_y, block_x, block_y,
 * void** args) (locomp/backends/rocm_codegen.py:304-340, called from
 * locomp/api.py:985-990) takes args[i] = the device pointer of the i-th
 * pointer parameter in signature order and bakes the integer parameters into
 * the generated code; here the kernel is chosen by `name` and the integer
 * parameters are passed as values, in signature order:
 *   "dequant_int4"         (W, SCALES, OUT; K, HALF_K, NUM_SCALES, GROUP_SIZE)
 *                          examples/52_dequantize.py:27-53
 *   "dequant_int8"         (W, SCALES, OUT; K, NUM_SCALES, GROUP_SIZE)
 *                          examples/52_dequantize.py:60-74
 *   "dequant_matvec_int4"  (X, W, scales, O; K_dim, HALF_K, NUM_SCALES, GROUP_SIZE)
 *                          examples/38_quantized_matmul.py:30-87
 *   "dequant_matvec_int8", "quant_matvec_int8"
 *                          (X, W, scales, O; K_dim, NUM_SCALES, GROUP_SIZE)
 *                          examples/38_quantized_matmul.py:94-134,
 *                          examples/58_benchmark_suite.py:241-264
 * grid_x = N (the reference's grid (N,)); grid_y must be 1 and the block at
 * most 1024 threads (the kernels pick their own geometry).  dtypes[i] = the
 * element dtype code of pointer parameter i (ignored for the weights); m =
 * activation rows of X (1 for the reference's matvec).  Returns what the
 * matching entry point returns, LQ_ERR_NAME for an unknown name. */
int locomp_amd_launch(const char* name, int grid_x, int grid_y, int block_x, int block_y,
                      void** args, const int64_t* constexprs, int n_constexprs,
                      const int* dtypes, int64_t m, void* stream);

/* Quantize float weights W [N, K] (in_dtype fp32 / fp16 / bf16) on the GPU
 * into PACKED uint8 [N, K/2] (byte j = q[2j] | q[2j+1] << 4) and float32
 * SCALES [N, K/GROUP_SIZE], bit-exact with the reference's NumPy producers:
 *   variant LQ_QUANT_EX38: quantize_int4, examples/38_quantized_matmul.py:248-271
 *     s = amax > 0 ? amax / 7 : 1;  q = clip(round(w / s) + 8, 0, 15)
 *   variant LQ_QUANT_EX52: quantize_int4_ref, examples/52_dequantize.py:110-126
 *     s = max(amax, 1e-10) / 7;     q = clip(round(w / (s + 1e-10)) + 8, 0, 15)
 * (float32 arithmetic, round half to even).  GROUP_SIZE must divide K and be
 * even.  The reference runs these on the host as weight producers; here they
 * are one HBM-bound launch. */
int locomp_amd_quantize_int4(const void* W, void* PACKED, float* SCALES, int64_t N, int64_t K,
                             int64_t GROUP_SIZE, int variant, int in_dtype, void* stream);

/* Quantize to int8 Q [N, K] and float32 SCALES [N, K/GROUP_SIZE], bit-exact
 * with quantize_int8, examples/38_quantized_matmul.py:274-291:
 *   s = amax > 0 ? amax / 127 : 1;  q = clip(round(w / s), -128, 127). */
int locomp_amd_quantize_int8(const void* W, void* Q, float* SCALES, int64_t N, int64_t K,
                             int64_t GROUP_SIZE, int in_dtype, void* stream);

/* Measurement helper, no counterpart in the reference: stream-read `bytes`
 * (a multiple of 1024, below 2^31) of device memory at `buf` and discard it
 * (`sink`: 4 bytes of device memory, written only on a value random data does
 * not produce).  The achievable HBM read rate for a buffer of that size, the
 * ceiling the bandwidth-bound kernels above are compared against. */
int locomp_amd_stream_read(const void* buf, int64_t bytes, void* sink, void* stream);

/* Residual add + RMSNorm between the quantized linears of a decode step:
 * for each of the M rows of K elements, H += R (when R is not null; H is
 * updated in place), then Y = H * rsqrt(sum(H^2) / K + eps) * gamma.
 * Replaces locomp_launch_rms_norm_kernel generated for
 * examples/54_smollm2_inference.py:40-73 (args X, W, O, N, EPS_X1000 =
 * eps * 1e6; grid (rows,), launched at :488-489) fused with
 * locomp_launch_add_inplace_kernel (:164-167, the residual adds at :538 and
 * :554).  H, R, gamma and Y share one dtype (LQ_F16, LQ_BF16 or LQ_F32);
 * fp32 arithmetic; Y may not alias H or R. */
int locomp_amd_rms_norm(void* H, const void* R, const void* gamma, void* Y, int64_t M, int64_t K,
                        float eps, int dtype, void* stream);

/* One decode-step link in one launch: the dequant-matmul of
 * locomp_amd_dequant_matvec_int4 (N = weight rows) with
 *   norm_weight != NULL: X is the hidden state and the matmul takes
 *       rmsnorm(X[m]) = X[m] * rsqrt(sum(X[m]^2) / K + norm_eps) * norm_weight
 *       (norm_weight [K] of X's dtype; each normalized activation rounded
 *       to X's dtype, as locomp_amd_rms_norm would store it);
 *   residual != NULL: O = X W^T + residual (residual [M, N] of O's dtype;
 *       it may be O itself, the residual stream updated in place);
 *   silu_mul != 0: gate|up rows interleaved as for
 *       locomp_amd_dequant_matvec_int4_silu_mul, O [M, N / 2] (not with a
 *       residual).
 * Replaces, in examples/54_smollm2_inference.py's decode step (:494-554),
 * rms_norm_kernel (:40-73) before a matvec and add_inplace_kernel
 * (:164-167) after one: the layer's chain becomes norm+q|k|v, o+residual,
 * norm+gate|up(SiLU * mul), down+residual.  No counterpart in the
 * reference: it launches those kernels separately.  One launch on the row
 * kernel for M = 1, K <= 4096, G % 32 == 0, 16-byte aligned X, W and
 * norm_weight; otherwise staged through per-(device, stream) workspaces
 * (the normalized activations, M x K; the fp32 product before a residual
 * add, M x N x 4 bytes), held until the process ends; a capture on a stream
 * without them returns LQ_ERR_SCRATCH. */
int locomp_amd_dequant_matvec_int4_fused(const void* X, const void* W, const void* scales, void* O,
                                         int64_t K_dim, int64_t HALF_K, int64_t NUM_SCALES,
                                         int64_t GROUP_SIZE, int64_t N, int64_t M, int x_dtype,
                                         int scale_dtype, int out_dtype, const void* norm_weight,
                                         float norm_eps, const void* residual, int silu_mul,
                                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LOCOMP_AMD_H_ */
