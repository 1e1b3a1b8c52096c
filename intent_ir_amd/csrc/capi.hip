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
#include <string.h>

#include <atomic>
#include <mutex>
#include <string>

#include "../../include/intentir_hip.h"
#include "common.hpp"

namespace ihip {
hipError_t launch_reduce_any_rows_f32(const float*, uint8_t*, int64_t, int64_t, float, hipStream_t);
hipError_t launch_reduce_any_rows_u8(const uint8_t*, uint8_t*, int64_t, int64_t, hipStream_t);
hipError_t launch_reduce_rows_f32(const float*, float*, int64_t, int64_t, int, float, float*, hipStream_t);
int reduce_rows_segments(int64_t, int64_t);
hipError_t launch_softmax_rows_f32(const float*, float*, int64_t, int64_t, int, hipStream_t, float*, float*, float*);
bool softmax_rows_per_wg_form(const float*, const float*, int64_t);
hipError_t launch_layernorm_rows_f16(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, float*, float*,
                                     int64_t, int64_t, float, hipStream_t);
hipError_t launch_layernorm_rows_f32(const float*, const float*, const float*, float*, float*, float*, int64_t, int64_t,
                                     float, hipStream_t);
hipError_t launch_gemm_f32_bias_relu(const float*, const float*, const float*, float*, int64_t, int64_t, int64_t, bool,
                                     bool, int, int, hipStream_t);
hipError_t launch_bias_gelu_axpy_bf16(const uint16_t*, const uint16_t*, uint16_t*, int64_t, int64_t, float,
                                      hipStream_t);
hipError_t launch_gather2d_f32(const float*, const int32_t*, const int32_t*, float*, int64_t, int64_t, int64_t, float,
                               hipStream_t);
hipError_t launch_gemm_bf16_bias_relu(const uint16_t*, const uint16_t*, const float*, uint16_t*, int64_t, int64_t,
                                      int64_t, bool, bool, int, int, hipStream_t);
hipError_t launch_gemm_bf16_bias_relu_ws(const uint16_t*, const uint16_t*, const float*, uint16_t*, int64_t, int64_t,
                                         int64_t, bool, bool, int, int, void*, int64_t, hipStream_t);
int64_t gemm_workspace_bytes(int64_t, int64_t, int64_t, bool, bool);
int64_t gemm_splitk_workspace_bytes(int64_t, int64_t, int64_t, int);
hipError_t launch_gemm_split(const uint16_t*, const uint16_t*, const float*, uint16_t*, int64_t, int64_t, int64_t,
                             bool, bool, int, int, int, void*, int64_t, hipStream_t);
hipError_t launch_elementwise_program(const ihip_ew_instr*, int, const ihip_ew_operand*, int, const ihip_ew_operand*,
                                      int, const int64_t (&)[4], hipStream_t);
hipError_t launch_elementwise_jit(const ihip_ew_instr*, int, const ihip_ew_operand*, int, const ihip_ew_operand*, int,
                                  const int64_t (&)[4], hipStream_t, std::string*);
bool prepare_elementwise_jit(const ihip_ew_instr*, int, int, const int*, int, const int*, std::string*);
bool prepare_elementwise_jit_operands(const ihip_ew_instr*, int, const ihip_ew_operand*, int, const ihip_ew_operand*,
                                      int, const int64_t (&)[4], std::string*);
std::string source_elementwise_jit_operands(const ihip_ew_instr*, int, const ihip_ew_operand*, int,
                                            const ihip_ew_operand*, int, const int64_t (&)[4]);
}  // namespace ihip

// Scratch of ihip_reduce_rows_f32_noalloc: the row-split partials (M * S floats; the split
// rule gives M < 256 and S <= 64, so at most 255 * 64).  Each GPU the library runs on holds
// its own copy until the process ends.  In host code `scratch` is only a symbol handle: its
// device address comes from hipGetSymbolAddress, per device, and only that address is ever
// passed to kernels.
static constexpr int64_t kScratchFloats = 256 * 64;
static __device__ __align__(256) float scratch[kScratchFloats];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch, resolved on the first call on that device.
hipError_t scratch_address(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

thread_local char g_last_error[512] = "";
std::atomic<int> g_ew_mode{IHIP_EW_MODE_AUTO};

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

// Operand shape of one element-wise program instruction: which fields name registers.
enum EwForm { kEwBad, kEwLoad, kEwImm, kEwIota, kEwStore, kEwUnary, kEwBinary, kEwWhere };

EwForm ew_form(int op) {
  switch (op) {
    case IHIP_EW_LOAD: return kEwLoad;
    case IHIP_EW_IMM: return kEwImm;
    case IHIP_EW_IOTA: return kEwIota;
    case IHIP_EW_STORE: return kEwStore;
    case IHIP_EW_MOV: case IHIP_EW_NOT: case IHIP_EW_RELU: case IHIP_EW_EXP: case IHIP_EW_RSQRT: case IHIP_EW_ABS:
    case IHIP_EW_FLOOR: case IHIP_EW_NEG: case IHIP_EW_CAST_F16: case IHIP_EW_CAST_BF16: case IHIP_EW_CAST_BOOL:
    case IHIP_EW_CAST_I32:
      return kEwUnary;
    case IHIP_EW_ADD: case IHIP_EW_SUB: case IHIP_EW_MUL: case IHIP_EW_DIV: case IHIP_EW_MAX: case IHIP_EW_MIN:
    case IHIP_EW_NE: case IHIP_EW_LT: case IHIP_EW_LE: case IHIP_EW_GT: case IHIP_EW_GE: case IHIP_EW_EQ:
    case IHIP_EW_AND: case IHIP_EW_OR:
      return kEwBinary;
    case IHIP_EW_WHERE: return kEwWhere;
    default: return kEwBad;
  }
}

bool ew_dtype_ok(int dt) { return dt >= IHIP_DT_F32 && dt <= IHIP_DT_I32; }

#define IHIP_REQUIRE(cond, ...)                               \
  do {                                                        \
    if (!(cond)) return fail(IHIP_ERR_INVALID_ARG, __VA_ARGS__); \
  } while (0)

// Data-flow check of an element-wise program: known opcodes, registers in range and written
// before read, operands in range, every output stored exactly once.  0 or a failure code.
int check_program(const ihip_ew_instr* code, int n_code, int n_inputs, int n_outputs) {
  bool written[IHIP_EW_NATIVE_MAX_REGS] = {};
  int stored[IHIP_EW_NATIVE_MAX_OUTPUTS] = {};
  for (int pc = 0; pc < n_code; ++pc) {
    const ihip_ew_instr& in = code[pc];
    const EwForm f = ew_form(in.op);
    IHIP_REQUIRE(f != kEwBad, "elementwise_program: instruction %d has unknown opcode %d", pc, (int)in.op);
    const auto reg_ok = [&](int r) { return r < IHIP_EW_NATIVE_MAX_REGS && written[r]; };
    switch (f) {
      case kEwLoad:
        IHIP_REQUIRE(in.a < n_inputs, "elementwise_program: instruction %d loads input %d of %d", pc, (int)in.a,
                     (int)n_inputs);
        break;
      case kEwIota:
        IHIP_REQUIRE(in.a < 4, "elementwise_program: instruction %d: iota axis %d outside 0..3", pc, (int)in.a);
        break;
      case kEwStore:
        IHIP_REQUIRE(reg_ok(in.a), "elementwise_program: instruction %d stores unwritten register %d", pc, (int)in.a);
        IHIP_REQUIRE(in.b < n_outputs, "elementwise_program: instruction %d stores output %d of %d", pc, (int)in.b,
                     (int)n_outputs);
        ++stored[in.b];
        break;
      case kEwWhere:
        IHIP_REQUIRE(reg_ok(in.c), "elementwise_program: instruction %d reads unwritten register %d", pc, (int)in.c);
        [[fallthrough]];
      case kEwBinary:
        IHIP_REQUIRE(reg_ok(in.b), "elementwise_program: instruction %d reads unwritten register %d", pc, (int)in.b);
        [[fallthrough]];
      case kEwUnary:
        IHIP_REQUIRE(reg_ok(in.a), "elementwise_program: instruction %d reads unwritten register %d", pc, (int)in.a);
        break;
      default:
        break;
    }
    if (f != kEwStore) {
      IHIP_REQUIRE(in.dst < IHIP_EW_NATIVE_MAX_REGS, "elementwise_program: instruction %d writes register %d of %d",
                   pc, (int)in.dst, IHIP_EW_NATIVE_MAX_REGS);
      written[in.dst] = true;
    }
  }
  for (int k = 0; k < n_outputs; ++k)
    IHIP_REQUIRE(stored[k] == 1, "elementwise_program: output %d is stored %d times (must be once)", k, stored[k]);
  return 0;
}

// True when a (checked) program fits the interpreter kernel: its instruction buffer, operand
// tables and register file.  Larger programs run only as native code.
bool fits_interpreter(const ihip_ew_instr* code, int n_code, int n_inputs, int n_outputs) {
  if (n_code > IHIP_EW_MAX_CODE || n_inputs > IHIP_EW_MAX_INPUTS || n_outputs > IHIP_EW_MAX_OUTPUTS) return false;
  for (int pc = 0; pc < n_code; ++pc) {
    const ihip_ew_instr& in = code[pc];
    const EwForm f = ew_form(in.op);
    if (f != kEwStore && in.dst >= IHIP_EW_MAX_REGS) return false;
    if ((f == kEwUnary || f == kEwBinary || f == kEwWhere || f == kEwStore) && in.a >= IHIP_EW_MAX_REGS) return false;
    if ((f == kEwBinary || f == kEwWhere) && in.b >= IHIP_EW_MAX_REGS) return false;
    if (f == kEwWhere && in.c >= IHIP_EW_MAX_REGS) return false;
  }
  return true;
}

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

int64_t ihip_reduce_rows_f32_workspace_size(int64_t M, int64_t N) {
  const int S = ihip::reduce_rows_segments(M, N);
  return S > 1 ? M * S * static_cast<int64_t>(sizeof(float)) : 0;
}

// Argument checks shared by the row-reduction entry points; 0 or a failure code.
static int check_reduce_rows(const char* who, const float* x, float* out, int64_t M, int64_t N, int kind) {
  const int64_t n = numel2(M, N);
  IHIP_REQUIRE(n >= 0, "%s: invalid shape [%lld, %lld]", who, (long long)M, (long long)N);
  IHIP_REQUIRE(kind == IHIP_REDUCE_SUM || kind == IHIP_REDUCE_MAX, "%s: unknown kind %d", who, kind);
  IHIP_REQUIRE(!(kind == IHIP_REDUCE_MAX && N == 0 && M > 0), "%s: max over an empty axis has no identity", who);
  IHIP_REQUIRE(M == 0 || out != nullptr, "%s: out is null", who);
  IHIP_REQUIRE(n == 0 || x != nullptr, "%s: x is null", who);
  return 0;
}

int ihip_reduce_rows_f32_ws(const float* x, float* out, int64_t M, int64_t N, int kind, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  return ihip_reduce_rows_f32_ex(x, out, M, N, kind, 1.0f, workspace, workspace_bytes, stream);
}

int ihip_reduce_rows_f32_ex(const float* x, float* out, int64_t M, int64_t N, int kind, float scale, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  const int bad = check_reduce_rows("reduce_rows_f32", x, out, M, N, kind);
  if (bad) return bad;
  const int64_t need = ihip_reduce_rows_f32_workspace_size(M, N);
  IHIP_REQUIRE(workspace == nullptr || workspace_bytes >= need,
               "reduce_rows_f32: workspace of %lld bytes, [%lld, %lld] needs %lld", (long long)workspace_bytes,
               (long long)M, (long long)N, (long long)need);
  IHIP_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 3) == 0, "reduce_rows_f32: workspace not 4-byte aligned");
  float* part = need > 0 ? static_cast<float*>(workspace) : nullptr;
  return finish(ihip::launch_reduce_rows_f32(x, out, M, N, kind, scale, part, static_cast<hipStream_t>(stream)),
                "reduce_rows_f32");
}

int ihip_reduce_rows_f32(const float* x, float* out, int64_t M, int64_t N, int kind, void* stream) {
  return ihip_reduce_rows_f32_ws(x, out, M, N, kind, nullptr, 0, stream);
}

int ihip_reduce_rows_f32_noalloc(const float* x, float* out, int64_t M, int64_t N, int kind, void* stream) {
  const int bad = check_reduce_rows("reduce_rows_f32_noalloc", x, out, M, N, kind);
  if (bad) return bad;
  const int64_t need = ihip_reduce_rows_f32_workspace_size(M, N);
  IHIP_REQUIRE(need <= kScratchFloats * static_cast<int64_t>(sizeof(float)),
               "reduce_rows_f32_noalloc: [%lld, %lld] needs %lld bytes of scratch, the maximum is %lld",
               (long long)M, (long long)N, (long long)need, (long long)(kScratchFloats * sizeof(float)));
  float* part = nullptr;
  if (need > 0) {  // every partial is written before it is read: nothing to clear
    const hipError_t e = scratch_address(&part);
    if (e != hipSuccess) return fail(static_cast<int>(e), "reduce_rows_f32_noalloc: scratch address: %s",
                                     hipGetErrorString(e));
  }
  return finish(ihip::launch_reduce_rows_f32(x, out, M, N, kind, 1.0f, part, static_cast<hipStream_t>(stream)),
                "reduce_rows_f32_noalloc");
}

int ihip_softmax_rows_f32_ex(const float* x, float* y, int64_t M, int64_t N, int rows_per_wg, void* stream) {
  const int64_t n = numel2(M, N);
  IHIP_REQUIRE(n >= 0, "softmax_rows_f32: invalid shape [%lld, %lld]", (long long)M, (long long)N);
  IHIP_REQUIRE(n == 0 || (x != nullptr && y != nullptr), "softmax_rows_f32: null pointer");
  IHIP_REQUIRE(rows_per_wg == 0 || rows_per_wg == 1 || rows_per_wg == 2 || rows_per_wg == 4,
               "softmax_rows_f32: rows_per_wg %d is not 0 (automatic), 1, 2 or 4", rows_per_wg);
  IHIP_REQUIRE(rows_per_wg <= 1 || n == 0 || ihip::softmax_rows_per_wg_form(x, y, N),
               "softmax_rows_f32: rows_per_wg %d needs the one-wave-per-row form (N %% 4 == 0, N <= 4096, "
               "16-byte aligned x and y); N = %lld runs one row per workgroup",
               rows_per_wg, (long long)N);
  return finish(ihip::launch_softmax_rows_f32(x, y, M, N, rows_per_wg, static_cast<hipStream_t>(stream), nullptr,
                                              nullptr, nullptr),
                "softmax_rows_f32");
}

int64_t ihip_softmax_rows_f32_workspace_size(int64_t M, int64_t N) {
  if (numel2(M, N) < 0) return 0;
  const ihip::SoftmaxSplit p = ihip::softmax_split_plan(M, N);
  return p.S > 0 ? 2 * M * p.S * static_cast<int64_t>(sizeof(float)) : 0;
}

int ihip_softmax_rows_f32_ws(const float* x, float* y, int64_t M, int64_t N, void* workspace, int64_t workspace_bytes,
                             void* stream) {
  return ihip_softmax_rows_f32_stats(x, y, nullptr, nullptr, M, N, workspace, workspace_bytes, stream);
}

int ihip_softmax_rows_f32_stats(const float* x, float* y, float* row_max, float* row_sum, int64_t M, int64_t N,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  const int64_t n = numel2(M, N);
  IHIP_REQUIRE(M <= 0 || N > 0 || (row_max == nullptr && row_sum == nullptr),
               "softmax_rows_f32_stats: rows of length 0 have no maximum");
  IHIP_REQUIRE(n >= 0, "softmax_rows_f32_stats: invalid shape [%lld, %lld]", (long long)M, (long long)N);
  IHIP_REQUIRE(n == 0 || (x != nullptr && y != nullptr), "softmax_rows_f32_stats: null pointer");
  IHIP_REQUIRE(workspace_bytes >= 0, "softmax_rows_f32_stats: negative workspace size %lld", (long long)workspace_bytes);
  IHIP_REQUIRE(workspace != nullptr || workspace_bytes == 0,
               "softmax_rows_f32_stats: workspace of %lld bytes at a null pointer", (long long)workspace_bytes);
  const int64_t need = ihip_softmax_rows_f32_workspace_size(M, N);
  IHIP_REQUIRE(workspace == nullptr || workspace_bytes >= need,
               "softmax_rows_f32_stats: workspace of %lld bytes, [%lld, %lld] needs %lld", (long long)workspace_bytes,
               (long long)M, (long long)N, (long long)need);
  IHIP_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 7) == 0, "softmax_rows_f32_stats: workspace not 8-byte aligned");
  float* part = need > 0 ? static_cast<float*>(workspace) : nullptr;
  return finish(ihip::launch_softmax_rows_f32(x, y, M, N, 0, static_cast<hipStream_t>(stream), part, row_max, row_sum),
                "softmax_rows_f32_stats");
}

int ihip_softmax_rows_f32(const float* x, float* y, int64_t M, int64_t N, void* stream) {
  return ihip_softmax_rows_f32_ex(x, y, M, N, 0, stream);
}

int ihip_layernorm_rows_f16(const uint16_t* x, const uint16_t* w, const uint16_t* b, uint16_t* y, float* mean,
                            float* rstd, int64_t M, int64_t N, float eps, void* stream) {
  const int64_t n = numel2(M, N);
  IHIP_REQUIRE(n >= 0, "layernorm_rows_f16: invalid shape [%lld, %lld]", (long long)M, (long long)N);
  IHIP_REQUIRE(n == 0 || (x != nullptr && y != nullptr && w != nullptr && b != nullptr),
               "layernorm_rows_f16: null pointer");
  return finish(ihip::launch_layernorm_rows_f16(x, w, b, y, mean, rstd, M, N, eps, static_cast<hipStream_t>(stream)),
                "layernorm_rows_f16");
}

int ihip_layernorm_rows_f32(const float* x, const float* w, const float* b, float* y, float* mean, float* rstd,
                            int64_t M, int64_t N, float eps, void* stream) {
  const int64_t n = numel2(M, N);
  IHIP_REQUIRE(n >= 0, "layernorm_rows_f32: invalid shape [%lld, %lld]", (long long)M, (long long)N);
  IHIP_REQUIRE(n == 0 || (x != nullptr && y != nullptr && w != nullptr && b != nullptr),
               "layernorm_rows_f32: null pointer");
  IHIP_REQUIRE(M <= 0x7fffffffLL, "layernorm_rows_f32: M = %lld exceeds 2^31 - 1 rows", (long long)M);
  return finish(ihip::launch_layernorm_rows_f32(x, w, b, y, mean, rstd, M, N, eps, static_cast<hipStream_t>(stream)),
                "layernorm_rows_f32");
}

int ihip_bias_gelu_tanh_axpy_bf16(const uint16_t* x, const uint16_t* bias, uint16_t* y, int64_t M, int64_t N,
                                  float alpha, void* stream) {
  const int64_t n = numel2(M, N);
  IHIP_REQUIRE(n >= 0, "bias_gelu_tanh_axpy_bf16: invalid shape [%lld, %lld]", (long long)M, (long long)N);
  IHIP_REQUIRE(n == 0 || (x != nullptr && bias != nullptr && y != nullptr), "bias_gelu_tanh_axpy_bf16: null pointer");
  return finish(ihip::launch_bias_gelu_axpy_bf16(x, bias, y, M, N, alpha, static_cast<hipStream_t>(stream)),
                "bias_gelu_tanh_axpy_bf16");
}

int ihip_gather2d_f32(const float* inp, const int32_t* row_idx, const int32_t* col_idx, float* out, int64_t M,
                      int64_t N, int64_t L, float other_value, void* stream) {
  const int64_t n = numel2(M, N);
  IHIP_REQUIRE(n >= 0 && L >= 0, "gather2d_f32: invalid shape inp [%lld, %lld], L = %lld", (long long)M, (long long)N,
               (long long)L);
  IHIP_REQUIRE(L == 0 || (row_idx != nullptr && col_idx != nullptr && out != nullptr), "gather2d_f32: null pointer");
  IHIP_REQUIRE(L == 0 || n == 0 || inp != nullptr, "gather2d_f32: inp is null");
  return finish(ihip::launch_gather2d_f32(inp, row_idx, col_idx, out, M, N, L, other_value,
                                          static_cast<hipStream_t>(stream)),
                "gather2d_f32");
}

int ihip_gemm_bf16_bias_relu_ex(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                                int64_t N, int64_t K, int transpose_a, int transpose_b, int relu, int tile,
                                void* stream) {
  IHIP_REQUIRE(numel2(M, K) >= 0 && numel2(K, N) >= 0 && numel2(M, N) >= 0,
               "gemm_bf16_bias_relu: invalid shape M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  IHIP_REQUIRE(M == 0 || N == 0 || C != nullptr, "gemm_bf16_bias_relu: C is null");
  IHIP_REQUIRE(M == 0 || N == 0 || K == 0 || (A != nullptr && B != nullptr), "gemm_bf16_bias_relu: A or B is null");
  IHIP_REQUIRE(tile == 0 || tile == 128 || tile == 256, "gemm_bf16_bias_relu: tile %d is not 0 (automatic), 128 or 256",
               tile);
  return finish(ihip::launch_gemm_bf16_bias_relu(A, B, bias, C, M, N, K, transpose_a != 0, transpose_b != 0, relu,
                                                 tile, static_cast<hipStream_t>(stream)),
                "gemm_bf16_bias_relu");
}

int ihip_gemm_f32_bias_relu(const float* A, const float* B, const float* bias, float* C, int64_t M, int64_t N,
                            int64_t K, int transpose_a, int transpose_b, int relu, int tile, void* stream) {
  IHIP_REQUIRE(numel2(M, K) >= 0 && numel2(K, N) >= 0 && numel2(M, N) >= 0,
               "gemm_f32_bias_relu: invalid shape M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  IHIP_REQUIRE(M == 0 || N == 0 || C != nullptr, "gemm_f32_bias_relu: C is null");
  IHIP_REQUIRE(M == 0 || N == 0 || K == 0 || (A != nullptr && B != nullptr), "gemm_f32_bias_relu: A or B is null");
  IHIP_REQUIRE(tile == 0 || tile == 64 || tile == 128, "gemm_f32_bias_relu: tile %d is not 0 (automatic), 64 or 128",
               tile);
  return finish(ihip::launch_gemm_f32_bias_relu(A, B, bias, C, M, N, K, transpose_a != 0, transpose_b != 0, relu, tile,
                                                static_cast<hipStream_t>(stream)),
                "gemm_f32_bias_relu");
}

int64_t ihip_gemm_workspace_size(int64_t M, int64_t N, int64_t K, int transpose_a, int transpose_b) {
  if (numel2(M, K) < 0 || numel2(K, N) < 0 || numel2(M, N) < 0) return 0;
  return ihip::gemm_workspace_bytes(M, N, K, transpose_a != 0, transpose_b != 0);
}

int ihip_gemm_bf16_bias_relu_ws(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                                int64_t N, int64_t K, int transpose_a, int transpose_b, int relu, int tile,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  IHIP_REQUIRE(numel2(M, K) >= 0 && numel2(K, N) >= 0 && numel2(M, N) >= 0,
               "gemm_bf16_bias_relu: invalid shape M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  IHIP_REQUIRE(M == 0 || N == 0 || C != nullptr, "gemm_bf16_bias_relu: C is null");
  IHIP_REQUIRE(M == 0 || N == 0 || K == 0 || (A != nullptr && B != nullptr), "gemm_bf16_bias_relu: A or B is null");
  IHIP_REQUIRE(tile == 0 || tile == 128 || tile == 256, "gemm_bf16_bias_relu: tile %d is not 0 (automatic), 128 or 256",
               tile);
  IHIP_REQUIRE(workspace_bytes >= 0 && (workspace_bytes == 0 || workspace != nullptr),
               "gemm_bf16_bias_relu: workspace of %lld bytes at a null pointer", (long long)workspace_bytes);
  return finish(ihip::launch_gemm_bf16_bias_relu_ws(A, B, bias, C, M, N, K, transpose_a != 0, transpose_b != 0, relu,
                                                    tile, workspace, workspace_bytes,
                                                    static_cast<hipStream_t>(stream)),
                "gemm_bf16_bias_relu");
}

int64_t ihip_gemm_splitk_workspace_size(int64_t M, int64_t N, int64_t K, int splits) {
  if (numel2(M, K) < 0 || numel2(K, N) < 0 || numel2(M, N) < 0 || splits < 0) return 0;
  return ihip::gemm_splitk_workspace_bytes(M, N, K, splits);
}

int ihip_gemm_bf16_bias_relu_splitk(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                                    int64_t N, int64_t K, int transpose_a, int transpose_b, int relu, int tile,
                                    int splits, void* workspace, int64_t workspace_bytes, void* stream) {
  IHIP_REQUIRE(numel2(M, K) >= 0 && numel2(K, N) >= 0 && numel2(M, N) >= 0,
               "gemm_bf16_bias_relu_splitk: invalid shape M=%lld N=%lld K=%lld", (long long)M, (long long)N,
               (long long)K);
  IHIP_REQUIRE(tile == 0 || tile == 128 || tile == 256,
               "gemm_bf16_bias_relu_splitk: tile %d is not 0 (automatic), 128 or 256", tile);
  IHIP_REQUIRE(splits >= 0, "gemm_bf16_bias_relu_splitk: splits %d is negative", splits);
  IHIP_REQUIRE(workspace_bytes >= 0 && (workspace_bytes == 0 || workspace != nullptr),
               "gemm_bf16_bias_relu_splitk: workspace of %lld bytes at a null pointer", (long long)workspace_bytes);
  if (M == 0 || N == 0) return 0;
  IHIP_REQUIRE(K > 0, "gemm_bf16_bias_relu_splitk: K = 0 (nothing to split)");
  const int64_t need = ihip::gemm_splitk_workspace_bytes(M, N, K, splits);
  IHIP_REQUIRE(workspace_bytes >= need, "gemm_bf16_bias_relu_splitk: workspace of %lld bytes, %lld needed",
               (long long)workspace_bytes, (long long)need);
  IHIP_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0,
               "gemm_bf16_bias_relu_splitk: workspace not 256-byte aligned");
  const hipError_t e = ihip::launch_gemm_split(A, B, bias, C, M, N, K, transpose_a != 0, transpose_b != 0, relu, tile,
                                               splits, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
  IHIP_REQUIRE(e != hipErrorNotSupported,
               "gemm_bf16_bias_relu_splitk: operands the tiled kernel cannot read in place (K %% 8, a [K, M] A "
               "with M %% 8, a [K, N] B with N %% 8, or a base not 16-byte aligned)");
  return finish(e, "gemm_bf16_bias_relu_splitk");
}

int ihip_gemm_bf16_bias_relu_t(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                               int64_t N, int64_t K, int transpose_a, int transpose_b, int relu, void* stream) {
  return ihip_gemm_bf16_bias_relu_ex(A, B, bias, C, M, N, K, transpose_a, transpose_b, relu, 0, stream);
}

int ihip_gemm_bf16_bias_relu(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                             int64_t N, int64_t K, int relu, void* stream) {
  return ihip_gemm_bf16_bias_relu_t(A, B, bias, C, M, N, K, 0, 0, relu, stream);
}

// Checks the arguments of an element-wise launch (also those of its operand-aware prepare)
// and right-aligns the shape into sh[4]; *total = element count.  Returns IHIP_OK or an error.
static int check_ew_launch(const char* who, const ihip_ew_instr* code, int32_t n_code, const ihip_ew_operand* inputs,
                           int32_t n_inputs, const ihip_ew_operand* outputs, int32_t n_outputs, const int64_t* shape,
                           int32_t rank, int64_t (&sh)[4], int64_t* total) {
  IHIP_REQUIRE(code != nullptr && n_code >= 1 && n_code <= IHIP_EW_NATIVE_MAX_CODE,
               "%s: need 1..%d instructions, got %d", who, IHIP_EW_NATIVE_MAX_CODE, (int)n_code);
  IHIP_REQUIRE(n_inputs >= 0 && n_inputs <= IHIP_EW_NATIVE_MAX_INPUTS && (n_inputs == 0 || inputs != nullptr),
               "%s: need 0..%d inputs, got %d", who, IHIP_EW_NATIVE_MAX_INPUTS, (int)n_inputs);
  IHIP_REQUIRE(n_outputs >= 1 && n_outputs <= IHIP_EW_NATIVE_MAX_OUTPUTS && outputs != nullptr,
               "%s: need 1..%d outputs, got %d", who, IHIP_EW_NATIVE_MAX_OUTPUTS, (int)n_outputs);
  IHIP_REQUIRE(rank >= 0 && rank <= IHIP_EW_MAX_RANK && (rank == 0 || shape != nullptr),
               "%s: rank %d outside 0..%d", who, (int)rank, IHIP_EW_MAX_RANK);
  for (int d = 0; d < 4; ++d) sh[d] = 1;
  *total = 1;
  for (int i = 0; i < rank; ++i) {
    sh[4 - rank + i] = shape[i];
    *total = numel2(*total, shape[i]);
    IHIP_REQUIRE(*total >= 0, "%s: invalid shape (axis %d = %lld)", who, i, (long long)shape[i]);
  }
  for (int k = 0; k < n_inputs; ++k) {
    IHIP_REQUIRE(ew_dtype_ok(inputs[k].dtype), "%s: input %d has unknown dtype %d", who, k, (int)inputs[k].dtype);
    IHIP_REQUIRE(*total == 0 || inputs[k].ptr != nullptr, "%s: input %d is null", who, k);
  }
  for (int k = 0; k < n_outputs; ++k) {
    IHIP_REQUIRE(ew_dtype_ok(outputs[k].dtype), "%s: output %d has unknown dtype %d", who, k, (int)outputs[k].dtype);
    IHIP_REQUIRE(*total == 0 || outputs[k].ptr != nullptr, "%s: output %d is null", who, k);
  }
  return check_program(code, n_code, n_inputs, n_outputs);
}

int ihip_elementwise_program(const ihip_ew_instr* code, int32_t n_code, const ihip_ew_operand* inputs,
                             int32_t n_inputs, const ihip_ew_operand* outputs, int32_t n_outputs,
                             const int64_t* shape, int32_t rank, void* stream) {
  int64_t sh[4], total = 0;
  const int bad = check_ew_launch("elementwise_program", code, n_code, inputs, n_inputs, outputs, n_outputs, shape,
                                  rank, sh, &total);
  if (bad) return bad;
  if (total == 0) return finish(hipSuccess, "elementwise_program");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int mode = g_ew_mode.load();
  const bool interp_ok = fits_interpreter(code, n_code, n_inputs, n_outputs);
  IHIP_REQUIRE(interp_ok || mode != IHIP_EW_MODE_INTERP,
               "elementwise_program: %d instructions, %d inputs, %d outputs exceed the interpreter kernel's limits "
               "(%d, %d, %d, registers < %d): such a program runs only as native code (mode AUTO or NATIVE)",
               (int)n_code, (int)n_inputs, (int)n_outputs, IHIP_EW_MAX_CODE, IHIP_EW_MAX_INPUTS, IHIP_EW_MAX_OUTPUTS,
               IHIP_EW_MAX_REGS);
  if (mode != IHIP_EW_MODE_INTERP) {
    std::string why;
    const hipError_t e = ihip::launch_elementwise_jit(code, n_code, inputs, n_inputs, outputs, n_outputs, sh, s, &why);
    if (e != hipErrorNotSupported || why.empty()) return finish(e, "elementwise_program (native)");
    if (mode == IHIP_EW_MODE_NATIVE || !interp_ok)
      return fail(static_cast<int>(e), "elementwise_program: native code unavailable: %s", why.c_str());
  }
  return finish(ihip::launch_elementwise_program(code, n_code, inputs, n_inputs, outputs, n_outputs, sh, s),
                "elementwise_program");
}

int ihip_elementwise_prepare(const ihip_ew_instr* code, int32_t n_code, const int32_t* input_dtypes, int32_t n_inputs,
                             const int32_t* output_dtypes, int32_t n_outputs) {
  IHIP_REQUIRE(code != nullptr && n_code >= 1 && n_code <= IHIP_EW_NATIVE_MAX_CODE,
               "elementwise_prepare: need 1..%d instructions, got %d", IHIP_EW_NATIVE_MAX_CODE, (int)n_code);
  IHIP_REQUIRE(n_inputs >= 0 && n_inputs <= IHIP_EW_NATIVE_MAX_INPUTS && (n_inputs == 0 || input_dtypes != nullptr),
               "elementwise_prepare: need 0..%d inputs, got %d", IHIP_EW_NATIVE_MAX_INPUTS, (int)n_inputs);
  IHIP_REQUIRE(n_outputs >= 1 && n_outputs <= IHIP_EW_NATIVE_MAX_OUTPUTS && output_dtypes != nullptr,
               "elementwise_prepare: need 1..%d outputs, got %d", IHIP_EW_NATIVE_MAX_OUTPUTS, (int)n_outputs);
  int in_dt[IHIP_EW_NATIVE_MAX_INPUTS] = {}, out_dt[IHIP_EW_NATIVE_MAX_OUTPUTS] = {};
  for (int k = 0; k < n_inputs; ++k) {
    IHIP_REQUIRE(ew_dtype_ok(input_dtypes[k]), "elementwise_prepare: input %d has unknown dtype %d", k,
                 (int)input_dtypes[k]);
    in_dt[k] = input_dtypes[k];
  }
  for (int k = 0; k < n_outputs; ++k) {
    IHIP_REQUIRE(ew_dtype_ok(output_dtypes[k]), "elementwise_prepare: output %d has unknown dtype %d", k,
                 (int)output_dtypes[k]);
    out_dt[k] = output_dtypes[k];
  }
  const int bad = check_program(code, n_code, n_inputs, n_outputs);
  if (bad) return bad;
  std::string why;
  if (!ihip::prepare_elementwise_jit(code, n_code, n_inputs, in_dt, n_outputs, out_dt, &why))
    return fail(static_cast<int>(hipErrorNotSupported), "elementwise_prepare: %s", why.c_str());
  g_last_error[0] = '\0';
  return IHIP_OK;
}

int ihip_elementwise_prepare_operands(const ihip_ew_instr* code, int32_t n_code, const ihip_ew_operand* inputs,
                                      int32_t n_inputs, const ihip_ew_operand* outputs, int32_t n_outputs,
                                      const int64_t* shape, int32_t rank) {
  int64_t sh[4], total = 0;
  const int bad = check_ew_launch("elementwise_prepare_operands", code, n_code, inputs, n_inputs, outputs, n_outputs,
                                  shape, rank, sh, &total);
  if (bad) return bad;
  std::string why;
  if (total != 0 &&
      !ihip::prepare_elementwise_jit_operands(code, n_code, inputs, n_inputs, outputs, n_outputs, sh, &why))
    return fail(static_cast<int>(hipErrorNotSupported), "elementwise_prepare_operands: %s", why.c_str());
  g_last_error[0] = '\0';
  return IHIP_OK;
}

int ihip_elementwise_source(const ihip_ew_instr* code, int32_t n_code, const ihip_ew_operand* inputs,
                            int32_t n_inputs, const ihip_ew_operand* outputs, int32_t n_outputs, const int64_t* shape,
                            int32_t rank, char* buf, int64_t buf_len, int64_t* src_len) {
  int64_t sh[4], total = 0;
  const int bad = check_ew_launch("elementwise_source", code, n_code, inputs, n_inputs, outputs, n_outputs, shape,
                                  rank, sh, &total);
  if (bad) return bad;
  IHIP_REQUIRE(buf_len >= 0 && (buf_len == 0 || buf != nullptr), "elementwise_source: buffer of %lld bytes is null",
               (long long)buf_len);
  const std::string src =
      total == 0 ? std::string() : ihip::source_elementwise_jit_operands(code, n_code, inputs, n_inputs, outputs,
                                                                         n_outputs, sh);
  if (src_len != nullptr) *src_len = static_cast<int64_t>(src.size());
  if (buf_len > 0) {
    const size_t n = src.size() < static_cast<size_t>(buf_len - 1) ? src.size() : static_cast<size_t>(buf_len - 1);
    memcpy(buf, src.data(), n);
    buf[n] = '\0';
  }
  g_last_error[0] = '\0';
  return IHIP_OK;
}

int ihip_elementwise_mode(int mode) {
  if (mode > IHIP_EW_MODE_NATIVE) return -1;
  if (mode < 0) return g_ew_mode.load();
  return g_ew_mode.exchange(mode);
}

}  // extern "C"
