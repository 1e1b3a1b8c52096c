// C-ABI of libintentir_hip.so: the drop-in boundary of the HIP backend.
//
// Conventions (declared in include/intentir_hip.h):
//  * every entry point takes device pointers, int64 sizes, scalars and a HIP
//    stream passed as void*; the caller owns every buffer, the library never
//    allocates or frees;
//  * calls are stream-ordered and asynchronous: no host synchronisation inside;
//  * the return value is 0 on success, a negative IHIP_ERR_* code for a rejected
//    argument, or a positive hipError_t from the launch; ihip_last_error() gives
//    the message of the calling thread's last failure.
#include <stdarg.h>
#include <stdio.h>

#include "../../include/intentir_hip.h"
#include "common.hpp"

namespace ihip {
hipError_t launch_reduce_any_rows_f32(const float*, uint8_t*, int64_t, int64_t, float, hipStream_t);
hipError_t launch_reduce_any_rows_u8(const uint8_t*, uint8_t*, int64_t, int64_t, hipStream_t);
hipError_t launch_reduce_rows_f32(const float*, float*, int64_t, int64_t, int, hipStream_t);
hipError_t launch_softmax_rows_f32(const float*, float*, int64_t, int64_t, hipStream_t);
hipError_t launch_layernorm_rows_f16(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, float*, float*,
                                     int64_t, int64_t, float, hipStream_t);
hipError_t launch_bias_gelu_axpy_bf16(const uint16_t*, const uint16_t*, uint16_t*, int64_t, int64_t, float,
                                      hipStream_t);
hipError_t launch_gemm_bf16_bias_relu(const uint16_t*, const uint16_t*, const float*, uint16_t*, int64_t, int64_t,
                                      int64_t, int, hipStream_t);
}  // namespace ihip

namespace {

thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int finish(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(static_cast<int>(e), "%s: launch failed: %s", what, hipGetErrorString(e));
  g_last_error[0] = '\0';
  return IHIP_OK;
}

// Element count of an [a, b] matrix, or -1 when a dimension is negative or the product overflows.
int64_t numel2(int64_t a, int64_t b) {
  if (a < 0 || b < 0) return -1;
  if (a != 0 && b > INT64_MAX / a) return -1;
  return a * b;
}

#define IHIP_REQUIRE(cond, ...)                               \
  do {                                                        \
    if (!(cond)) return fail(IHIP_ERR_INVALID_ARG, __VA_ARGS__); \
  } while (0)

}  // namespace

extern "C" {

int ihip_abi_version(void) { return IHIP_ABI_VERSION; }

const char* ihip_last_error(void) { return g_last_error; }

int ihip_reduce_any_rows_f32(const float* x, uint8_t* out, int64_t M, int64_t N, float cmp_value, void* stream) {
  const int64_t n = numel2(M, N);
  IHIP_REQUIRE(n >= 0, "reduce_any_rows_f32: invalid shape [%lld, %lld]", (long long)M, (long long)N);
  IHIP_REQUIRE(M == 0 || out != nullptr, "reduce_any_rows_f32: out is null");
  IHIP_REQUIRE(n == 0 || x != nullptr, "reduce_any_rows_f32: x is null");
  return finish(ihip::launch_reduce_any_rows_f32(x, out, M, N, cmp_value, static_cast<hipStream_t>(stream)),
                "reduce_any_rows_f32");
}

int ihip_reduce_any_rows_u8(const uint8_t* x, uint8_t* out, int64_t M, int64_t N, void* stream) {
  const int64_t n = numel2(M, N);
  IHIP_REQUIRE(n >= 0, "reduce_any_rows_u8: invalid shape [%lld, %lld]", (long long)M, (long long)N);
  IHIP_REQUIRE(M == 0 || out != nullptr, "reduce_any_rows_u8: out is null");
  IHIP_REQUIRE(n == 0 || x != nullptr, "reduce_any_rows_u8: x is null");
  return finish(ihip::launch_reduce_any_rows_u8(x, out, M, N, static_cast<hipStream_t>(stream)), "reduce_any_rows_u8");
}

int ihip_reduce_rows_f32(const float* x, float* out, int64_t M, int64_t N, int kind, void* stream) {
  const int64_t n = numel2(M, N);
  IHIP_REQUIRE(n >= 0, "reduce_rows_f32: invalid shape [%lld, %lld]", (long long)M, (long long)N);
  IHIP_REQUIRE(kind == IHIP_REDUCE_SUM || kind == IHIP_REDUCE_MAX, "reduce_rows_f32: unknown kind %d", kind);
  IHIP_REQUIRE(!(kind == IHIP_REDUCE_MAX && N == 0 && M > 0),
               "reduce_rows_f32: max over an empty axis has no identity");
  IHIP_REQUIRE(M == 0 || out != nullptr, "reduce_rows_f32: out is null");
  IHIP_REQUIRE(n == 0 || x != nullptr, "reduce_rows_f32: x is null");
  return finish(ihip::launch_reduce_rows_f32(x, out, M, N, kind, static_cast<hipStream_t>(stream)), "reduce_rows_f32");
}

int ihip_softmax_rows_f32(const float* x, float* y, int64_t M, int64_t N, void* stream) {
  const int64_t n = numel2(M, N);
  IHIP_REQUIRE(n >= 0, "softmax_rows_f32: invalid shape [%lld, %lld]", (long long)M, (long long)N);
  IHIP_REQUIRE(n == 0 || (x != nullptr && y != nullptr), "softmax_rows_f32: null pointer");
  return finish(ihip::launch_softmax_rows_f32(x, y, M, N, static_cast<hipStream_t>(stream)), "softmax_rows_f32");
}

int ihip_layernorm_rows_f16(const uint16_t* x, const uint16_t* w, const uint16_t* b, uint16_t* y, float* mean,
                            float* rstd, int64_t M, int64_t N, float eps, void* stream) {
  const int64_t n = numel2(M, N);
  IHIP_REQUIRE(n >= 0, "layernorm_rows_f16: invalid shape [%lld, %lld]", (long long)M, (long long)N);
  IHIP_REQUIRE(M == 0 || (mean != nullptr && rstd != nullptr), "layernorm_rows_f16: null statistics pointer");
  IHIP_REQUIRE(n == 0 || (x != nullptr && y != nullptr && w != nullptr && b != nullptr),
               "layernorm_rows_f16: null pointer");
  return finish(ihip::launch_layernorm_rows_f16(x, w, b, y, mean, rstd, M, N, eps, static_cast<hipStream_t>(stream)),
                "layernorm_rows_f16");
}

int ihip_bias_gelu_tanh_axpy_bf16(const uint16_t* x, const uint16_t* bias, uint16_t* y, int64_t M, int64_t N,
                                  float alpha, void* stream) {
  const int64_t n = numel2(M, N);
  IHIP_REQUIRE(n >= 0, "bias_gelu_tanh_axpy_bf16: invalid shape [%lld, %lld]", (long long)M, (long long)N);
  IHIP_REQUIRE(n == 0 || (x != nullptr && bias != nullptr && y != nullptr), "bias_gelu_tanh_axpy_bf16: null pointer");
  return finish(ihip::launch_bias_gelu_axpy_bf16(x, bias, y, M, N, alpha, static_cast<hipStream_t>(stream)),
                "bias_gelu_tanh_axpy_bf16");
}

int ihip_gemm_bf16_bias_relu(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                             int64_t N, int64_t K, int relu, void* stream) {
  IHIP_REQUIRE(numel2(M, K) >= 0 && numel2(K, N) >= 0 && numel2(M, N) >= 0,
               "gemm_bf16_bias_relu: invalid shape M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  IHIP_REQUIRE(M == 0 || N == 0 || C != nullptr, "gemm_bf16_bias_relu: C is null");
  IHIP_REQUIRE(M == 0 || N == 0 || K == 0 || (A != nullptr && B != nullptr), "gemm_bf16_bias_relu: A or B is null");
  return finish(ihip::launch_gemm_bf16_bias_relu(A, B, bias, C, M, N, K, relu, static_cast<hipStream_t>(stream)),
                "gemm_bf16_bias_relu");
}

}  // extern "C"
