/*
 * intentir_hip.h — C-ABI of libintentir_hip.so, the MI355X (gfx950) execution
 * backend for IntentIR.
 *
 * The reference selects a GPU backend by importing its Python module and, per
 * kernel, builds a torch extension whose pybind ``launch(*args)`` is the only
 * host->device boundary (frontends/cuda/runtime.py:621-808, called at
 * :1021-1026; lowering entry backends/cuda/codegen/intentir_to_cuda.py:2047).
 * This library replaces those per-kernel generated extensions with fixed,
 * precompiled gfx950 kernels behind plain C functions, one per kernel family
 * the lowering emits.  Each declaration cites the reference lowering it replaces.
 *
 * Conventions
 *  - Pointers are device pointers; sizes are element counts (int64); matrices
 *    are row-major and contiguous.  16-bit floats (f16, bf16) are passed as
 *    uint16_t bit patterns; bool outputs are one byte (0/1) per element.
 *  - ``stream`` is a hipStream_t passed as void* (NULL = the default stream).
 *    Work is enqueued on it; nothing synchronises the host.
 *  - The caller owns every buffer.  The library allocates no device memory.  Its only
 *    state is a thread-local error message and, for element-wise programs, a cache of
 *    compiled code behind a mutex; it is re-entrant.
 *  - Return: IHIP_OK (0); a negative IHIP_ERR_* for rejected arguments; or a
 *    positive hipError_t value when the launch itself failed.  On failure
 *    ihip_last_error() describes it (thread-local, valid until the next call).
 */
#ifndef INTENTIR_HIP_H_
#define INTENTIR_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IHIP_ABI_VERSION 3

#define IHIP_OK 0
#define IHIP_ERR_INVALID_ARG (-1)

#define IHIP_REDUCE_SUM 0
#define IHIP_REDUCE_MAX 1

/* ABI version of the loaded library (IHIP_ABI_VERSION it was built with). */
int ihip_abi_version(void);

/* Message of the calling thread's last failed call ("" after a success). */
const char* ihip_last_error(void);

/* out[m] = any(x[m, :] != cmp_value) for x f32 [M, N]; numpy semantics (NaN != c
 * is true, -0.0 == 0.0).  Replaces the CUDA any-dim lowering of `reduce_any`
 * and `const, ne, reduce_any` (backends/cuda/codegen/intentir_to_cuda.py:1693-1776,
 * dispatched at :2161-2162). */
int ihip_reduce_any_rows_f32(const float* x, uint8_t* out, int64_t M, int64_t N, float cmp_value, void* stream);

/* out[m] = any(x[m, :] != 0) for a bool/u8 matrix [M, N] (reduce_any on an i1
 * tensor, verify/interpreter.py:489-494). */
int ihip_reduce_any_rows_u8(const uint8_t* x, uint8_t* out, int64_t M, int64_t N, void* stream);

/* out[m] = sum(x[m, :]) (kind IHIP_REDUCE_SUM) or max(x[m, :]) (IHIP_REDUCE_MAX,
 * NaN-propagating) for x f32 [M, N].  Replaces the row reductions of
 * backends/cuda/codegen/intentir_to_cuda.py:1553-1690. */
int ihip_reduce_rows_f32(const float* x, float* out, int64_t M, int64_t N, int kind, void* stream);

/* Bytes of workspace ihip_reduce_rows_f32_ws uses for an [M, N] reduction: M * S floats when
 * rows are too few to fill the GPU (M < 256) and long enough to split into S <= 64 segments
 * of at least 64 KiB each, else 0 (the rows are not split).  Depends on M and N only. */
int64_t ihip_reduce_rows_f32_workspace_size(int64_t M, int64_t N);

/* ihip_reduce_rows_f32 with a caller-owned device workspace (the library still allocates
 * nothing): when ihip_reduce_rows_f32_workspace_size(M, N) > 0, each row is split over S
 * workgroups whose partial results go to the workspace and a second kernel folds them in a
 * fixed order (results are reproducible; a sum's rounding order differs from the unsplit
 * form).  workspace may be NULL (no split, exactly ihip_reduce_rows_f32); otherwise it must
 * hold at least workspace_size bytes, 4-byte aligned, and stay untouched until the work on
 * `stream` completes.  Same semantics as ihip_reduce_rows_f32 (verify/interpreter.py:478-500). */
int ihip_reduce_rows_f32_ws(const float* x, float* out, int64_t M, int64_t N, int kind, void* workspace,
                            int64_t workspace_bytes, void* stream);

/* ihip_reduce_rows_f32_ws with a result scale: out[m] = reduce(x[m, :]) * scale, one f32
 * multiply of the row's result (scale 1.0 is ihip_reduce_rows_f32_ws exactly).  The
 * interpreter's reduce_sum{scale} (verify/interpreter.py:478-488, :646-673), e.g. a row mean
 * written as sum * (1/N) (pipeline/cuda/core.py:509-511). */
int ihip_reduce_rows_f32_ex(const float* x, float* out, int64_t M, int64_t N, int kind, float scale, void* workspace,
                            int64_t workspace_bytes, void* stream);

/* ihip_reduce_rows_f32_ws without a workspace argument and without any allocation: no
 * counterpart in the reference; it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The row-split partials go
 * to a fixed 64 KiB scratch array in device memory that each GPU holds until the process
 * ends; every call on one GPU shares it, so calls that overlap on one GPU (concurrent
 * streams, threads) race and must be serialised by the caller.  Shapes whose split needs
 * more than 64 KiB are rejected (IHIP_ERR_INVALID_ARG); the split rule keeps every shape
 * within it.  Results are identical to ihip_reduce_rows_f32_ws. */
int ihip_reduce_rows_f32_noalloc(const float* x, float* out, int64_t M, int64_t N, int kind, void* stream);

/* y = softmax(x) over the last axis, x and y f32 [M, N] (y may not alias x).
 * Replaces _kernel_softmax_2d_last_f32 (backends/cuda/codegen/intentir_to_cuda.py:1103-1247)
 * and its device templates (backends/cuda/runtime/kernels/softmax.cuh:92-663). */
int ihip_softmax_rows_f32(const float* x, float* y, int64_t M, int64_t N, void* stream);

/* The same with a launch-shape knob, the role of the reference's SOFTMAX_THREADS binding
 * (backends/cuda/codegen/intentir_to_cuda.py:1175-1200): rows_per_wg = 0 chooses
 * automatically (rows of exactly 1024 floats: 8 per workgroup, two per wave; at most 256: 4, two
 * per wave; other rows of at most 1024 floats: 2, one per wave; longer: 4, one per wave); 1, 2 or 4 sets
 * how many rows (one wave each; 4 rows of at most 1024 floats: two waves of two) share a
 * workgroup.  Only the
 * one-wave-per-row form (N % 4 == 0, N <= 4096, 16-byte aligned x and y) has that choice;
 * for other shapes rows_per_wg must be 0 or 1 (IHIP_ERR_INVALID_ARG otherwise).  Results do
 * not depend on rows_per_wg. */
int ihip_softmax_rows_f32_ex(const float* x, float* y, int64_t M, int64_t N, int rows_per_wg, void* stream);

/* Bytes of workspace ihip_softmax_rows_f32_ws uses for an [M, N] softmax: 2 * M * S floats
 * when rows are longer than 65536 floats (vocabulary-width rows) and too few for a workgroup
 * per row to fill the GPU (fewer than 192, or a last round of at most 160 rows after one or
 * two full rounds of 256), split into S segments each; else 0 (the rows are not split).
 * Depends on M and N only.  Same softmax as ihip_softmax_rows_f32, whose long-row kernel it
 * speeds up on such shapes (the reference lowers every N through
 * _kernel_softmax_2d_last_f32, backends/cuda/codegen/intentir_to_cuda.py:1103-1247). */
int64_t ihip_softmax_rows_f32_workspace_size(int64_t M, int64_t N);

/* ihip_softmax_rows_f32 with a caller-owned device workspace (the library still allocates
 * nothing): when ihip_softmax_rows_f32_workspace_size(M, N) > 0 and the rows of x and y start
 * at the same offset modulo 16 bytes (4-byte aligned), each row is split over S workgroups;
 * one kernel writes each segment's maximum and sum of exponentials to the workspace and a
 * second folds a row's S partials in a fixed order and writes y.  Results are
 * reproducible; the sum's rounding order differs from the unsplit form.  workspace may be
 * NULL (exactly ihip_softmax_rows_f32); otherwise it must hold at least workspace_size
 * bytes, 8-byte aligned, and stay untouched until the work on `stream` completes. */
int ihip_softmax_rows_f32_ws(const float* x, float* y, int64_t M, int64_t N, void* workspace, int64_t workspace_bytes,
                             void* stream);

/* ihip_softmax_rows_f32_ws that also writes each row's statistics: row_max[m] = max(x[m, :])
 * (NaN-propagating) and row_sum[m] = sum(exp(x[m, :] - row_max[m])), the values the softmax
 * divides by, from the same launch (no second pass over x).  Either pointer may be NULL (not
 * written).  Rows of length 0 have no maximum: N == 0 with a non-NULL statistic is
 * IHIP_ERR_INVALID_ARG.  The reference's softmax IR with those outputs
 * (pipeline/cuda/core.py:453-493, softmax_inner: output_ptr, row_max_ptr, row_sum_ptr). */
int ihip_softmax_rows_f32_stats(const float* x, float* y, float* row_max, float* row_sum, int64_t M, int64_t N,
                                void* workspace, int64_t workspace_bytes, void* stream);

/* LayerNorm forward over the last axis with f16 data: x, y f16 [M, N]; w, b f16 [N];
 * mean, rstd f32 [M] (either may be NULL: that statistic is then not written);
 * f32 statistics, rstd = 1/sqrt(var + eps), y rounded to f16.  The reference has no f16
 * LayerNorm kernel (its CUDA lowering types f32 only, intentir_to_cuda.py:159-175); this
 * entry runs the reference LayerNorm IR (pipeline/tilelang/core.py:1322-1384) when it
 * declares x, w, b, y as f16, with the op order of ihip_layernorm_rows_f32. */
int ihip_layernorm_rows_f16(const uint16_t* x, const uint16_t* w, const uint16_t* b, uint16_t* y, float* mean,
                            float* rstd, int64_t M, int64_t N, float eps, void* stream);

/* LayerNorm forward in f32: x, y f32 [M, N]; w, b f32 [N]; mean, rstd f32 [M] (either may
 * be NULL: not written).  mean = sum(x)/N, d = x - mean, var = sum(d*d)/N,
 * rstd = 1/sqrt(var + eps), y = ((d*rstd)*w) + b, each step a separately rounded f32
 * operation.  Any N and alignment; M < 2^31.  Replaces _kernel_layernorm_2d_f32
 * (backends/cuda/codegen/intentir_to_cuda.py:1250-1338, dispatched at :2163-2164;
 * backends/cuda/runtime/kernels/layernorm.cuh:11-98). */
int ihip_layernorm_rows_f32(const float* x, const float* w, const float* b, float* y, float* mean, float* rstd,
                            int64_t M, int64_t N, float eps, void* stream);

/* y = alpha * gelu_tanh(x + bias[col]) + x for x, y bf16 [M, N], bias bf16 [N],
 * f32 arithmetic, one pass.  Replaces the fused element-wise lowering
 * (backends/cuda/codegen/intentir_to_cuda.py:229-534, dispatched at :2170-2199)
 * for the bias + GELU + axpy chain, which that lowering cannot type (bf16). */
int ihip_bias_gelu_tanh_axpy_bf16(const uint16_t* x, const uint16_t* bias, uint16_t* y, int64_t M, int64_t N,
                                  float alpha, void* stream);

/* out[i] = inp[row_idx[i], col_idx[i]] for i < L, with inp f32 [M, N], row_idx and col_idx
 * int32 [L], out f32 [L]; an index pair outside [0, M) x [0, N) (negative indices included)
 * gives other_value.  Replaces _kernel_gather2d_f32
 * (backends/cuda/codegen/intentir_to_cuda.py:1779-1832, dispatched at :2155-2156), with the
 * out-of-range rule its test pins (tests/backends/cuda/test_cuda_backend_smoke.py:292-336).
 * inp may be NULL when M * N == 0 (every index is then out of range). */
int ihip_gather2d_f32(const float* inp, const int32_t* row_idx, const int32_t* col_idx, float* out, int64_t M,
                      int64_t N, int64_t L, float other_value, void* stream);

/* C = act(A @ B + bias) with A bf16 [M, K], B bf16 [K, N], bias f32 [N] or NULL,
 * act = ReLU when relu != 0 else identity; f32 accumulation on MFMA, C bf16
 * (round to nearest even).  The reference lowers f32 matmul only, as a lone op
 * (backends/cuda/codegen/intentir_to_cuda.py:537-985, :2137-2140); this entry runs the
 * reference matmul IR (pipeline/tilelang/core.py:886-910, with its bias + ReLU epilogue)
 * when A, B and C are declared bf16.  The f32 IR runs on ihip_gemm_f32_bias_relu.
 * Any shape: rows that all start 16-byte aligned
 * (N % 8 == 0, K % 8 == 0, 16-byte aligned A, B, C) run the tiled MFMA kernel at any
 * M, N, K; other shapes a slower guarded kernel with the same accumulation order. */
int ihip_gemm_bf16_bias_relu(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                             int64_t N, int64_t K, int relu, void* stream);

/* C = act(op(A) @ op(B) + bias) in f32: A f32 [M, K] (or [K, M] when transpose_a), B f32
 * [K, N] (or [N, K] when transpose_b), bias f32 [N] or NULL, C f32 [M, N]; act = ReLU
 * (numpy's maximum(x, 0): NaN and -0.0 pass through) when relu != 0.  Exact f32 products
 * and f32 accumulation on the fp32 matrix cores (no reduced-precision inputs, so the
 * reference's opt-in ALLOW_TF32 is never needed).  Any M, N, K and alignment.  tile = 0
 * chooses automatically (128x128 C tiles, 64x64 when fewer than 256 tiles of 128x128 would
 * run); 64 or 128 fixes it; C does not depend on tile.  Replaces _kernel_matmul_f32 and
 * its device code (backends/cuda/codegen/intentir_to_cuda.py:537-985, dispatched at
 * :2137-2140; backends/cuda/runtime/kernels/matmul_fallback.cuh:8-73,
 * wmma_matmul.cuh:124-565), and also takes the bias + ReLU epilogue the reference's
 * builders emit (pipeline/tilelang/core.py:886-910) in the same launch. */
int ihip_gemm_f32_bias_relu(const float* A, const float* B, const float* bias, float* C, int64_t M, int64_t N,
                            int64_t K, int transpose_a, int transpose_b, int relu, int tile, void* stream);

/* The same with matmul's transpose flags (verify/interpreter.py:507-520): when transpose_a,
 * A is given as [K, M] and the product uses its transpose; when transpose_b, B is given as
 * [N, K].  Every layout runs the same MFMA schedule and accumulates in the same order, so a
 * transposed operand gives bit-identical C.  With B given as [N, K] the tiled kernel takes
 * any N (K % 8 == 0): C rows that are not 16-byte aligned are written with 2-byte stores. */
int ihip_gemm_bf16_bias_relu_t(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                               int64_t N, int64_t K, int transpose_a, int transpose_b, int relu, void* stream);

/* The same with a tile knob, the role of the reference's WMMA_* tile bindings and schedule
 * tile_m / tile_n (backends/cuda/codegen/intentir_to_cuda.py:659-664, 2074-2097): tile = 0
 * chooses automatically (256x256 C tiles, 128x128 when at most 128 tiles of 256x256 would
 * run); 128 or 256 fixes the tile extent, of the tiled and of the guarded kernel alike.  Every
 * tile extent accumulates in the same order, so C does not depend on tile (the workspace
 * entries below may split a 128 x 128 grid along K, which changes the f32 summation order). */
int ihip_gemm_bf16_bias_relu_ex(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                                int64_t N, int64_t K, int transpose_a, int transpose_b, int relu, int tile,
                                void* stream);

/* Workspace bytes ihip_gemm_bf16_bias_relu_ws needs for this shape (0: none), 256-byte
 * aligned pieces in this order:
 *  - K-contiguous copies, K rounded up to 8, of the operands whose rows cannot start 16-byte
 *    aligned (K % 8 != 0, N % 8 != 0 with B given as [K, N], M % 8 != 0 with A given as
 *    [K, M]);
 *  - split-K partials, S x M x (N rounded up to 4) floats, when the split rule cuts K into
 *    S > 1 segments: only grids of 128 x 128 tiles (the automatic choice when at most 128
 *    tiles of 256 x 256 would be busy) are split, into the S (segments of whole 64-k steps, at
 *    least 512 k each, at most 512 workgroups) of least estimated time on K8 = K rounded up
 *    to 8 (gemm_pack.hip split_plan).
 * Same shapes and layouts as the entries above (the reference allocates nothing for matmul:
 * its kernels take any shape in place, intentir_to_cuda.py:537-985). */
int64_t ihip_gemm_workspace_size(int64_t M, int64_t N, int64_t K, int transpose_a, int transpose_b);

/* ihip_gemm_bf16_bias_relu_ex with a caller workspace (256-byte aligned, workspace_bytes
 * long; NULL / 0 allowed):
 *  - operands the tiled kernel cannot read in place are copied into it as K-contiguous rows
 *    of K rounded up to 8 elements (zeros past K) and the tiled kernel runs on the copies;
 *    C rows that are not 16-byte aligned are written with 2-byte stores.  Unsplit, results
 *    are bit-identical to the guarded kernel's (the same zeros in the same k slots, the same
 *    MFMA order), which runs when the workspace is too small for the copies;
 *  - a grid of too few tiles (ihip_gemm_workspace_size) is split along K: each segment's
 *    f32 sums go to the workspace and a second kernel adds the segments in order, then bias
 *    and activation.  Deterministic; it differs from the unsplit result only by f32
 *    summation order.  Without room for the partials the launch is unsplit, and so is a
 *    launch with tile = 256 (the rule splits 128 x 128 tiles only).
 * The workspace must stay untouched until the launch completes on the stream. */
int ihip_gemm_bf16_bias_relu_ws(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                                int64_t N, int64_t K, int transpose_a, int transpose_b, int relu, int tile,
                                void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes of a split into `splits` K segments (0: the split rule of
 * ihip_gemm_workspace_size; 1: none), for operands read in place. */
int64_t ihip_gemm_splitk_workspace_size(int64_t M, int64_t N, int64_t K, int splits);

/* ihip_gemm_bf16_bias_relu_ex split into `splits` K segments (0: the split rule, which leaves
 * 256 x 256 tiles unsplit; 1: unsplit;
 * at most one per 64 k and at most 1024), for operands the tiled kernel reads in place (K % 8 == 0, M % 8 == 0
 * with A given as [K, M], N % 8 == 0 with B given as [K, N], A and B 16-byte aligned; any C
 * alignment), K > 0; IHIP_ERR_INVALID_ARG otherwise or when the workspace (256-byte aligned)
 * is smaller than ihip_gemm_splitk_workspace_size.  Each segment is a whole number of 64-k
 * steps.  The split count is a tuning knob with no counterpart in the reference
 * (intentir_to_cuda.py:537-985 runs one kernel per matmul). */
int ihip_gemm_bf16_bias_relu_splitk(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                                    int64_t N, int64_t K, int transpose_a, int transpose_b, int relu, int tile,
                                    int splits, void* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Generic element-wise program: any chain of element-wise ops over inputs that
 * broadcast, transpose or repeat along the axes of one iteration space (rank <= 4).
 * Replaces the reference's fused element-wise lowering, which generates and
 * compiles one CUDA kernel per chain (backends/cuda/codegen/intentir_to_cuda.py:229-534;
 * C++ emitter intentir_cuda_codegen.cpp:4057-4195).  Here one precompiled kernel runs a
 * short register program that the host passes by value: every wave executes the
 * same instruction stream (uniform branches), on 4 consecutive elements per lane.
 * Values are f32 inside the program; bool is 0.0 / 1.0.
 * ------------------------------------------------------------------------- */
/* Limits of the interpreter kernel (a fixed register file and instruction buffer). */
#define IHIP_EW_MAX_CODE 64
#define IHIP_EW_MAX_REGS 8
#define IHIP_EW_MAX_INPUTS 8
#define IHIP_EW_MAX_OUTPUTS 4
#define IHIP_EW_MAX_RANK 4
/* Limits of the native (hiprtc-compiled, straight-line) form, where registers are plain
 * variables and the instruction list becomes code: a program within the interpreter limits
 * above runs in every mode; a larger one, up to these, runs only as native code (modes AUTO
 * and NATIVE), and in INTERP mode or when its compilation fails the call returns an error
 * instead of falling back to the interpreter.  The reference generates one kernel per chain
 * with no such limits (backends/cuda/codegen/intentir_to_cuda.py:229-534). */
#define IHIP_EW_NATIVE_MAX_CODE 1024
#define IHIP_EW_NATIVE_MAX_REGS 255
#define IHIP_EW_NATIVE_MAX_INPUTS 32
#define IHIP_EW_NATIVE_MAX_OUTPUTS 8

/* Operand element types. */
#define IHIP_DT_F32 0
#define IHIP_DT_F16 1  /* IEEE half, 16-bit pattern */
#define IHIP_DT_BF16 2 /* bfloat16, 16-bit pattern */
#define IHIP_DT_BOOL 3 /* one byte; stored as 0/1, read as non-zero */
#define IHIP_DT_I32 4  /* exact while |x| < 2^24 inside the program */

/* Opcodes.  r[x] is register x; numpy float32 semantics (NaN propagates through
 * max/min/relu; comparisons with NaN are false except ne). */
#define IHIP_EW_LOAD 1       /* r[dst] = input[a] at the current coordinates */
#define IHIP_EW_IMM 2        /* r[dst] = imm */
#define IHIP_EW_IOTA 3       /* r[dst] = coordinate along axis a (0 = outermost of rank 4) */
#define IHIP_EW_STORE 4      /* output[b] = r[a], converted to the output type (RNE) */
#define IHIP_EW_MOV 5        /* r[dst] = r[a] */
#define IHIP_EW_ADD 10       /* binary: r[dst] = r[a] op r[b] */
#define IHIP_EW_SUB 11
#define IHIP_EW_MUL 12
#define IHIP_EW_DIV 13       /* IEEE division */
#define IHIP_EW_MAX 14       /* np.maximum */
#define IHIP_EW_MIN 15       /* np.minimum */
#define IHIP_EW_NE 20        /* comparisons give 0.0 / 1.0 */
#define IHIP_EW_LT 21
#define IHIP_EW_LE 22
#define IHIP_EW_GT 23
#define IHIP_EW_GE 24
#define IHIP_EW_EQ 25
#define IHIP_EW_AND 30       /* logical, operands tested != 0 */
#define IHIP_EW_OR 31
#define IHIP_EW_NOT 32       /* unary: r[dst] = op(r[a]) */
#define IHIP_EW_RELU 40      /* np.maximum(x, 0) */
#define IHIP_EW_EXP 41
#define IHIP_EW_RSQRT 42     /* 1 / sqrt(x), both correctly rounded */
#define IHIP_EW_ABS 43
#define IHIP_EW_FLOOR 44
#define IHIP_EW_NEG 45
#define IHIP_EW_WHERE 50     /* r[dst] = r[a] != 0 ? r[b] : r[c] */
#define IHIP_EW_CAST_F16 60  /* round to f16 (RNE) and back */
#define IHIP_EW_CAST_BF16 61 /* round to bf16 (RNE) and back */
#define IHIP_EW_CAST_BOOL 62 /* x != 0 */
#define IHIP_EW_CAST_I32 63  /* truncate toward zero */

typedef struct ihip_ew_instr {
  uint8_t op, dst, a, b, c;
  uint8_t reserved[3];
  float imm;
} ihip_ew_instr;

/* One input or output.  Inputs: element stride per axis of the rank-4 iteration
 * space (0 = broadcast along that axis); any strides are accepted.  Outputs are
 * dense row-major tensors of the iteration shape (strides ignored). */
typedef struct ihip_ew_operand {
  const void* ptr;
  int32_t dtype;
  int32_t reserved;
  int64_t stride[IHIP_EW_MAX_RANK];
} ihip_ew_operand;

/* Run `code` (host memory, copied into the launch) over the iteration space
 * `shape[0..rank-1]` (rank 0..4).  The program is checked before launch: known
 * opcodes, registers and operand indices in range, every register written before
 * it is read, every output stored exactly once. */
int ihip_elementwise_program(const ihip_ew_instr* code, int32_t n_code, const ihip_ew_operand* inputs,
                             int32_t n_inputs, const ihip_ew_operand* outputs, int32_t n_outputs,
                             const int64_t* shape, int32_t rank, void* stream);

/* The HIP C++ source that ihip_elementwise_program compiles for exactly this launch (same
 * arguments, without the stream): the role of the reference lowering's cuda_src
 * (backends/cuda/codegen/intentir_to_cuda.py:27-35).  Needs no device: pointers are only
 * inspected for their alignment.  *src_len (when not NULL) receives the source length in
 * bytes; when buf_len > 0 the source is copied to buf, truncated to buf_len - 1 bytes and
 * NUL-terminated.  Returns IHIP_OK or an argument error as ihip_elementwise_program. */
int ihip_elementwise_source(const ihip_ew_instr* code, int32_t n_code, const ihip_ew_operand* inputs,
                            int32_t n_inputs, const ihip_ew_operand* outputs, int32_t n_outputs, const int64_t* shape,
                            int32_t rank, char* buf, int64_t buf_len, int64_t* src_len);

/* How ihip_elementwise_program executes a program (process-wide):
 *  AUTO   - native code specialised for the program and its operand types, compiled with
 *           hiprtc on first use and cached (per device) for the life of the process; the
 *           interpreter kernel when that compilation fails.  The default.
 *  INTERP - always the interpreter kernel (no compilation).
 *  NATIVE - specialised code only; a failed compilation is returned as an error.
 * The first call of a new program in AUTO/NATIVE mode blocks the host for the compile
 * (~0.3-3 s); later calls only launch. */
#define IHIP_EW_MODE_AUTO 0
#define IHIP_EW_MODE_INTERP 1
#define IHIP_EW_MODE_NATIVE 2

/* Set the mode when mode >= 0; return the previous mode (-1 for an unknown mode, unchanged). */
int ihip_elementwise_mode(int mode);

/* Compile the native code of a program for the given operand types ahead of its first launch
 * (for example before capturing a graph).  Needs no device.  Checks the program like
 * ihip_elementwise_program; returns IHIP_OK, or an error whose message holds the compiler log.
 * The generated code fixes each operand's access form, so this prepares the form that dense
 * operands select: every input and output 16-byte aligned, read and written in full vectors
 * (inner size a multiple of 8 elements when all operands are 16-bit or narrower, else of 4).
 * Other layouts (broadcast scalars and [M,1] columns, strided or unaligned operands, operands
 * read across their unit-stride axis such as a transpose) compile on their first launch, or
 * ahead of it through ihip_elementwise_prepare_operands. */
int ihip_elementwise_prepare(const ihip_ew_instr* code, int32_t n_code, const int32_t* input_dtypes, int32_t n_inputs,
                             const int32_t* output_dtypes, int32_t n_outputs);

/* Compile exactly the native code that ihip_elementwise_program would run for these operands
 * and shape (same arguments, without the stream), ahead of the launch.  Needs no device:
 * the pointers are only inspected for their alignment.  Returns IHIP_OK, or an error as
 * ihip_elementwise_prepare. */
int ihip_elementwise_prepare_operands(const ihip_ew_instr* code, int32_t n_code, const ihip_ew_operand* inputs,
                                      int32_t n_inputs, const ihip_ew_operand* outputs, int32_t n_outputs,
                                      const int64_t* shape, int32_t rank);

#ifdef __cplusplus
}
#endif

#endif /* INTENTIR_HIP_H_ */
