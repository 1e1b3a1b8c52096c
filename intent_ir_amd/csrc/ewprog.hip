// Generic element-wise programs: one precompiled gfx950 kernel that runs a short
// register program (include/intentir_hip.h, IHIP_EW_*) over a rank-4 iteration space.
//
// The reference lowers every fused element-wise chain by generating CUDA source and
// compiling it per chain (backends/cuda/codegen/intentir_to_cuda.py:229-534).  Here the
// chain is data: the host packs the program into the kernel arguments, so it sits in the
// scalar register file / constant cache and every branch on it is wave-uniform.
//
// Layout and schedule
//  * the iteration space is [D0, D1, D2, D3]; a lane owns 4 consecutive elements of the
//    innermost axis, so loads and stores of contiguous operands are 16-byte (f32) or
//    8-byte (16-bit) vector accesses;
//  * grid.y strides over the flattened outer rows (D0*D1*D2), grid.x over the vectors
//    of a row; row coordinates are decoded once per row (uniform);
//  * inputs carry per-axis element strides (0 = broadcast), so bias vectors, [M,1]
//    columns, scalars and transposed views need no materialisation;
//  * registers are an [8][4] f32 array indexed by the (uniform) instruction fields; the
//    compiler addresses it with VGPR indexing mode, no scratch memory (a larger file
//    is demoted to scratch by the compiler).
#include "../../include/intentir_hip.h"
#include "common.hpp"

namespace ihip {

constexpr int kEwV = 4;  // elements per lane

struct EwLaunchArgs {
  ihip_ew_instr code[IHIP_EW_MAX_CODE];
  const void* in_ptr[IHIP_EW_MAX_INPUTS];
  int64_t in_stride[IHIP_EW_MAX_INPUTS][4];
  void* out_ptr[IHIP_EW_MAX_OUTPUTS];
  int32_t in_dtype[IHIP_EW_MAX_INPUTS];
  int32_t out_dtype[IHIP_EW_MAX_OUTPUTS];
  int64_t shape[4];
  int64_t rows;       // D0 * D1 * D2
  int64_t nvec;       // ceil(D3 / 4)
  int32_t n_code;
  uint32_t in_vec;    // bit k: input k can use vector loads (unit inner stride, aligned rows)
  uint32_t out_vec;   // bit k: output k can use vector stores
  uint32_t pad;
};

__device__ __forceinline__ float ld1(const void* p, int dt, int64_t i) {
  switch (dt) {
    case IHIP_DT_F32: return static_cast<const float*>(p)[i];
    case IHIP_DT_F16: return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
    case IHIP_DT_BF16: return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    case IHIP_DT_BOOL: return static_cast<float>(static_cast<const uint8_t*>(p)[i]);
    default: return static_cast<float>(static_cast<const int32_t*>(p)[i]);
  }
}

// 4 consecutive elements at element offset i (i % 4 == 0, base aligned).
__device__ __forceinline__ void ld4(const void* p, int dt, int64_t i, float (&v)[kEwV]) {
  switch (dt) {
    case IHIP_DT_F32: {
      const f32x4 q = *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i);
      v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
      break;
    }
    case IHIP_DT_F16:
    case IHIP_DT_BF16: {
      const u32x2 q = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(p) + i);
      const uint16_t h[4] = {static_cast<uint16_t>(q.x & 0xffffu), static_cast<uint16_t>(q.x >> 16),
                             static_cast<uint16_t>(q.y & 0xffffu), static_cast<uint16_t>(q.y >> 16)};
#pragma unroll
      for (int j = 0; j < kEwV; ++j) v[j] = dt == IHIP_DT_F16 ? f16_to_f32(h[j]) : bf16_to_f32(h[j]);
      break;
    }
    case IHIP_DT_BOOL: {
      const uint32_t q = *reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(p) + i);
#pragma unroll
      for (int j = 0; j < kEwV; ++j) v[j] = static_cast<float>((q >> (8 * j)) & 0xffu);
      break;
    }
    default: {
      const u32x4 q = *reinterpret_cast<const u32x4*>(static_cast<const int32_t*>(p) + i);
      v[0] = static_cast<float>(static_cast<int32_t>(q.x));
      v[1] = static_cast<float>(static_cast<int32_t>(q.y));
      v[2] = static_cast<float>(static_cast<int32_t>(q.z));
      v[3] = static_cast<float>(static_cast<int32_t>(q.w));
    }
  }
}

__device__ __forceinline__ uint16_t to_f16_bits(float x) { return f32_to_f16_rne(x); }
__device__ __forceinline__ uint16_t to_bf16_bits(float x) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x)); }

__device__ __forceinline__ void st1(void* p, int dt, int64_t i, float x) {
  switch (dt) {
    case IHIP_DT_F32: static_cast<float*>(p)[i] = x; break;
    case IHIP_DT_F16: static_cast<uint16_t*>(p)[i] = to_f16_bits(x); break;
    case IHIP_DT_BF16: static_cast<uint16_t*>(p)[i] = to_bf16_bits(x); break;
    case IHIP_DT_BOOL: static_cast<uint8_t*>(p)[i] = x != 0.0f ? 1 : 0; break;
    default: static_cast<int32_t*>(p)[i] = static_cast<int32_t>(x);
  }
}

__device__ __forceinline__ void st4(void* p, int dt, int64_t i, const float (&v)[kEwV]) {
  switch (dt) {
    case IHIP_DT_F32: *reinterpret_cast<f32x4*>(static_cast<float*>(p) + i) = f32x4{v[0], v[1], v[2], v[3]}; break;
    case IHIP_DT_F16:
    case IHIP_DT_BF16: {
      uint16_t h[4];
#pragma unroll
      for (int j = 0; j < kEwV; ++j) h[j] = dt == IHIP_DT_F16 ? to_f16_bits(v[j]) : to_bf16_bits(v[j]);
      const u32x2 q = {h[0] | (static_cast<uint32_t>(h[1]) << 16), h[2] | (static_cast<uint32_t>(h[3]) << 16)};
      *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p) + i) = q;
      break;
    }
    case IHIP_DT_BOOL: {
      uint32_t q = 0;
#pragma unroll
      for (int j = 0; j < kEwV; ++j) q |= (v[j] != 0.0f ? 1u : 0u) << (8 * j);
      *reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(p) + i) = q;
      break;
    }
    default:
      *reinterpret_cast<u32x4*>(static_cast<int32_t*>(p) + i) =
          u32x4{static_cast<uint32_t>(static_cast<int32_t>(v[0])), static_cast<uint32_t>(static_cast<int32_t>(v[1])),
                static_cast<uint32_t>(static_cast<int32_t>(v[2])), static_cast<uint32_t>(static_cast<int32_t>(v[3]))};
  }
}

__global__ __launch_bounds__(256) void ew_program_kernel(const EwLaunchArgs args) {
  const int64_t D1 = args.shape[1], D2 = args.shape[2], D3 = args.shape[3];
  for (int64_t row = blockIdx.y; row < args.rows; row += gridDim.y) {
    // uniform row decode
    int64_t c0 = 0, c1 = 0, c2 = row;
    if (row >= D2) {
      c2 = row % D2;
      const int64_t t = row / D2;
      c1 = t % D1;
      c0 = t / D1;
    }
    for (int64_t vec = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; vec < args.nvec;
         vec += static_cast<int64_t>(gridDim.x) * blockDim.x) {
      const int64_t c3 = vec * kEwV;
      const int valid = D3 - c3 < kEwV ? static_cast<int>(D3 - c3) : kEwV;
      float r[IHIP_EW_MAX_REGS * kEwV];  // register x holds elements r[4x .. 4x+3]
      for (int pc = 0; pc < args.n_code; ++pc) {
        const ihip_ew_instr in = args.code[pc];
        // readfirstlane: the indices are uniform; in SGPRs the register file is addressed with
        // VGPR indexing mode instead of a select chain over all 32 values
        const int a0 = __builtin_amdgcn_readfirstlane(in.a * kEwV);
        const int b0 = __builtin_amdgcn_readfirstlane(in.b * kEwV);
        // Every case leaves its result in t and the register file is written at one place
        // below: a write per case would make the compiler copy the whole file at the merge.
        // STORE writes its source register back unchanged.
        const int w0 = __builtin_amdgcn_readfirstlane((in.op == IHIP_EW_STORE ? in.a : in.dst) * kEwV);
        float t[kEwV];
        switch (in.op) {
          case IHIP_EW_LOAD: {
            const int k = in.a;
            const void* p = args.in_ptr[k];
            const int dt = args.in_dtype[k];
            const int64_t s3 = args.in_stride[k][3];
            const int64_t base = c0 * args.in_stride[k][0] + c1 * args.in_stride[k][1] + c2 * args.in_stride[k][2];
            if ((args.in_vec >> k) & 1u) {
              ld4(p, dt, base + c3, t);
            } else if (s3 == 0) {
              const float x = ld1(p, dt, base);
#pragma unroll
              for (int j = 0; j < kEwV; ++j) t[j] = x;
            } else {
#pragma unroll
              for (int j = 0; j < kEwV; ++j) t[j] = j < valid ? ld1(p, dt, base + (c3 + j) * s3) : 0.0f;
            }
            break;
          }
          case IHIP_EW_IMM:
#pragma unroll
            for (int j = 0; j < kEwV; ++j) t[j] = in.imm;
            break;
          case IHIP_EW_IOTA: {
            const int64_t c = in.a == 0 ? c0 : in.a == 1 ? c1 : in.a == 2 ? c2 : c3;
#pragma unroll
            for (int j = 0; j < kEwV; ++j) t[j] = static_cast<float>(in.a == 3 ? c + j : c);
            break;
          }
          case IHIP_EW_STORE: {
            const int k = in.b;
            void* p = args.out_ptr[k];
            const int dt = args.out_dtype[k];
            const int64_t off = row * D3 + c3;
#pragma unroll
            for (int j = 0; j < kEwV; ++j) t[j] = r[a0 + j];
            if ((args.out_vec >> k) & 1u) {
              st4(p, dt, off, t);
            } else {
#pragma unroll
              for (int j = 0; j < kEwV; ++j)
                if (j < valid) st1(p, dt, off + j, t[j]);
            }
            break;
          }
#define IHIP_EW_BIN(OPC, EXPR)                          \
  case OPC:                                             \
    _Pragma("unroll") for (int j = 0; j < kEwV; ++j) {  \
      const float x = r[a0 + j], y = r[b0 + j];         \
      t[j] = (EXPR);                                    \
    }                                                   \
    break;
#define IHIP_EW_UN(OPC, EXPR)                           \
  case OPC:                                             \
    _Pragma("unroll") for (int j = 0; j < kEwV; ++j) {  \
      const float x = r[a0 + j];                        \
      t[j] = (EXPR);                                    \
    }                                                   \
    break;
          IHIP_EW_UN(IHIP_EW_MOV, x)
          IHIP_EW_BIN(IHIP_EW_ADD, x + y)
          IHIP_EW_BIN(IHIP_EW_SUB, x - y)
          IHIP_EW_BIN(IHIP_EW_MUL, x * y)
          IHIP_EW_BIN(IHIP_EW_DIV, x / y)
          IHIP_EW_BIN(IHIP_EW_MAX, __builtin_elementwise_maximum(x, y))
          IHIP_EW_BIN(IHIP_EW_MIN, __builtin_elementwise_minimum(x, y))
          IHIP_EW_BIN(IHIP_EW_NE, x != y ? 1.0f : 0.0f)
          IHIP_EW_BIN(IHIP_EW_LT, x < y ? 1.0f : 0.0f)
          IHIP_EW_BIN(IHIP_EW_LE, x <= y ? 1.0f : 0.0f)
          IHIP_EW_BIN(IHIP_EW_GT, x > y ? 1.0f : 0.0f)
          IHIP_EW_BIN(IHIP_EW_GE, x >= y ? 1.0f : 0.0f)
          IHIP_EW_BIN(IHIP_EW_EQ, x == y ? 1.0f : 0.0f)
          IHIP_EW_BIN(IHIP_EW_AND, (x != 0.0f && y != 0.0f) ? 1.0f : 0.0f)
          IHIP_EW_BIN(IHIP_EW_OR, (x != 0.0f || y != 0.0f) ? 1.0f : 0.0f)
          IHIP_EW_UN(IHIP_EW_NOT, x == 0.0f ? 1.0f : 0.0f)
          IHIP_EW_UN(IHIP_EW_RELU, __builtin_elementwise_maximum(x, 0.0f))
          IHIP_EW_UN(IHIP_EW_EXP, expf(x))
          IHIP_EW_UN(IHIP_EW_RSQRT, 1.0f / sqrtf(x))
          IHIP_EW_UN(IHIP_EW_ABS, fabsf(x))
          IHIP_EW_UN(IHIP_EW_FLOOR, floorf(x))
          IHIP_EW_UN(IHIP_EW_NEG, -x)
          IHIP_EW_UN(IHIP_EW_CAST_F16, f16_to_f32(to_f16_bits(x)))
          IHIP_EW_UN(IHIP_EW_CAST_BF16, bf16_to_f32(to_bf16_bits(x)))
          IHIP_EW_UN(IHIP_EW_CAST_BOOL, x != 0.0f ? 1.0f : 0.0f)
          IHIP_EW_UN(IHIP_EW_CAST_I32, truncf(x))
#undef IHIP_EW_BIN
#undef IHIP_EW_UN
          case IHIP_EW_WHERE: {
            const int e0 = __builtin_amdgcn_readfirstlane(in.c * kEwV);
#pragma unroll
            for (int j = 0; j < kEwV; ++j) {
              float xb = r[b0 + j], xe = r[e0 + j];
              // keep the select on values: folded into a per-lane register index it would
              // become a select chain over the whole register file
              asm volatile("" : "+v"(xb), "+v"(xe));
              t[j] = r[a0 + j] != 0.0f ? xb : xe;
            }
            break;
          }
          default:  // the host rejects unknown opcodes before launch
#pragma unroll
            for (int j = 0; j < kEwV; ++j) t[j] = r[w0 + j];
            break;
        }
#pragma unroll
        for (int j = 0; j < kEwV; ++j) r[w0 + j] = t[j];
      }
    }
  }
}

static bool aligned(const void* p, int64_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

static int64_t elt_size(int dt) {
  return dt == IHIP_DT_F32 || dt == IHIP_DT_I32 ? 4 : dt == IHIP_DT_BOOL ? 1 : 2;
}

// Shapes and program are validated by the caller (capi.hip); shape is padded to rank 4.
hipError_t launch_elementwise_program(const ihip_ew_instr* code, int n_code, const ihip_ew_operand* inputs,
                                      int n_inputs, const ihip_ew_operand* outputs, int n_outputs,
                                      const int64_t (&shape)[4], hipStream_t s) {
  EwLaunchArgs a{};
  for (int i = 0; i < n_code; ++i) a.code[i] = code[i];
  a.n_code = n_code;
  for (int d = 0; d < 4; ++d) a.shape[d] = shape[d];
  a.rows = shape[0] * shape[1] * shape[2];
  a.nvec = (shape[3] + kEwV - 1) / kEwV;
  if (a.rows == 0 || a.nvec == 0) return hipSuccess;
  const bool inner4 = shape[3] % kEwV == 0;
  for (int k = 0; k < n_inputs; ++k) {
    a.in_ptr[k] = inputs[k].ptr;
    a.in_dtype[k] = inputs[k].dtype;
    for (int d = 0; d < 4; ++d) a.in_stride[k][d] = inputs[k].stride[d];
    const int64_t* st = inputs[k].stride;
    const bool rows4 = (st[0] % kEwV == 0 || shape[0] == 1) && (st[1] % kEwV == 0 || shape[1] == 1) &&
                       (st[2] % kEwV == 0 || shape[2] == 1);
    if (inner4 && st[3] == 1 && rows4 && aligned(inputs[k].ptr, kEwV * elt_size(inputs[k].dtype))) a.in_vec |= 1u << k;
  }
  for (int k = 0; k < n_outputs; ++k) {
    a.out_ptr[k] = const_cast<void*>(outputs[k].ptr);
    a.out_dtype[k] = outputs[k].dtype;
    if (inner4 && aligned(outputs[k].ptr, kEwV * elt_size(outputs[k].dtype))) a.out_vec |= 1u << k;
  }
  const int64_t bx = (a.nvec + 255) / 256;
  const unsigned gx = static_cast<unsigned>(bx < 1024 ? bx : 1024);
  int64_t gy = (4096 + gx - 1) / gx;  // a few thousand workgroups in total
  if (gy > a.rows) gy = a.rows;
  if (gy > 65535) gy = 65535;
  ew_program_kernel<<<dim3(gx, static_cast<unsigned>(gy)), dim3(256), 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace ihip
