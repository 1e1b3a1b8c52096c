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
 *  - The caller owns every buffer.  The library allocates nothing and keeps no
 *    state besides a thread-local error message; it is re-entrant.
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

#define IHIP_ABI_VERSION 1

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

/* y = softmax(x) over the last axis, x and y f32 [M, N] (y may not alias x).
 * Replaces _kernel_softmax_2d_last_f32 (backends/cuda/codegen/intentir_to_cuda.py:1103-1247)
 * and its device templates (backends/cuda/runtime/kernels/softmax.cuh:92-663). */
int ihip_softmax_rows_f32(const float* x, float* y, int64_t M, int64_t N, void* stream);

/* LayerNorm forward over the last axis: x, y f16 [M, N]; w, b f16 [N];
 * mean, rstd f32 [M]; f32 statistics, rstd = 1/sqrt(var + eps).  Replaces
 * _kernel_layernorm_2d_f32 (backends/cuda/codegen/intentir_to_cuda.py:1250-1338,
 * backends/cuda/runtime/kernels/layernorm.cuh:11-98), extended to f16 I/O. */
int ihip_layernorm_rows_f16(const uint16_t* x, const uint16_t* w, const uint16_t* b, uint16_t* y, float* mean,
                            float* rstd, int64_t M, int64_t N, float eps, void* stream);

/* y = alpha * gelu_tanh(x + bias[col]) + x for x, y bf16 [M, N], bias bf16 [N],
 * f32 arithmetic, one pass.  Replaces the fused element-wise lowering
 * (backends/cuda/codegen/intentir_to_cuda.py:229-534, dispatched at :2170-2199)
 * for the bias + GELU + axpy chain, which that lowering cannot type (bf16). */
int ihip_bias_gelu_tanh_axpy_bf16(const uint16_t* x, const uint16_t* bias, uint16_t* y, int64_t M, int64_t N,
                                  float alpha, void* stream);

/* C = act(A @ B + bias) with A bf16 [M, K], B bf16 [K, N], bias f32 [N] or NULL,
 * act = ReLU when relu != 0 else identity; f32 accumulation on MFMA, C bf16
 * (round to nearest even).  Replaces _kernel_matmul_f32 / wmma_matmul_f32_tf32
 * (backends/cuda/codegen/intentir_to_cuda.py:537-985,
 * backends/cuda/runtime/kernels/wmma_matmul.cuh:124-565), which lower matmul
 * only as a lone op (:2137-2140). */
int ihip_gemm_bf16_bias_relu(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                             int64_t N, int64_t K, int relu, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* INTENTIR_HIP_H_ */
