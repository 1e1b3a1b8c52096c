// Native code for element-wise programs: the instruction list of ihip_elementwise_program
// (include/intentir_hip.h) is turned into straight-line gfx950 code with hiprtc, once per
// distinct program, operand types and operand access forms, and cached for the life of the
// process.
//
// The interpreter kernel (ewprog.hip) pays a uniform dispatch, operand moves through the
// indexed register file and an instruction fetch for every program instruction, which
// costs several times the HBM time of a chain longer than three or four instructions.
// Specialised code has none of that: registers are plain variables and every operand type
// is known, so a chain runs at the rate of its loads and stores.  This mirrors what the
// reference does per chain (CUDA source generated and compiled at first use,
// frontends/cuda/runtime.py:621-808), with the difference that the source is derived here
// from the already validated instruction list, inside the library, behind the same C call.
//
// Layout and schedule follow the interpreter kernel: a lane owns V consecutive elements of
// the innermost axis (V = 8 when all operands are 16-bit or narrower, so each access is one
// 16-byte vector; else 4), grid.y strides over outer rows, inputs carry per-axis strides.
// The access form of every operand (V-wide or 4-wide vectors, a broadcast element, strided
// elements, an LDS tile) is fixed in the generated source, so the code holds only the paths
// a launch takes; each distinct combination compiles once.
#include <hip/hiprtc.h>
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/intentir_hip.h"
#include "common.hpp"

namespace ihip {

struct EwJitArgs {
  const void* in_ptr[IHIP_EW_NATIVE_MAX_INPUTS];
  int64_t in_stride[IHIP_EW_NATIVE_MAX_INPUTS][4];
  void* out_ptr[IHIP_EW_NATIVE_MAX_OUTPUTS];
  int64_t shape[4];
  int64_t rows;
  int64_t nvec;  // ceil(D3 / V): lanes own V = 4 or 8 elements
};

namespace {

// Device prelude of every generated kernel; the struct must match EwJitArgs above.
const char* kPrelude = R"JIT(
typedef unsigned int u32;
typedef unsigned short u16;
typedef unsigned char u8;
typedef long long i64;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef u32 u32x4 __attribute__((ext_vector_type(4)));
typedef u32 u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
struct EwJitArgs {
  const void* in_ptr[32];
  i64 in_stride[32][4];
  void* out_ptr[8];
  i64 shape[4];
  i64 rows;
  i64 nvec;
};
// exp, division and 1/sqrt on the hardware approximations, each refined to within ~2 ulp of
// the correctly rounded result (the numpy float32 forms the interpreter uses round once or
// twice); non-finite inputs and results take the IEEE value.
__device__ __forceinline__ float ew_exp(float x) {
  // 2^(x*log2 e): the product carried as head t + tail, v_exp_f32 on the head, first-order
  // correction e*(1 + tail*ln 2) for the tail.  No correction where the head overflowed
  // (e = +inf: a negative tail would make inf - inf = NaN) or the input is not finite.
  const float t = x * 1.44269502f;
  const float tail = __builtin_fmaf(x, 1.92596303e-08f, __builtin_fmaf(x, 1.44269502f, -t));
  const float e = __builtin_amdgcn_exp2f(t);
  return __builtin_isfinite(tail) && __builtin_isfinite(e) ? __builtin_fmaf(e, tail * 0.693147182f, e) : e;
}
// x / y as v_rcp_f32 and one Newton step on the quotient.  `bad` is set where that form
// does not hold (zero, infinite or NaN reciprocal or quotient); those elements take ew_div,
// which falls back to IEEE division for exactly them, so a lane branches once per vector.
__device__ __forceinline__ float ew_div_fast(float x, float y, bool& bad) {
  const float r = __builtin_amdgcn_rcpf(y);
  const float q = x * r;
  bad |= !__builtin_isfinite(q) || r == 0.0f || !__builtin_isfinite(r);
  return __builtin_fmaf(__builtin_fmaf(-y, q, x), r, q);
}
__device__ __forceinline__ float ew_div(float x, float y) {
  bool bad = false;
  const float q = ew_div_fast(x, y, bad);
  return bad ? x / y : q;
}
// x / (exp(u) + 1), the logistic shape of GELU-tanh and sigmoid, in one pass, given t = u log2 e:
// e = 2^t on the hardware exp2 without the tail correction of ew_exp, then the reciprocal and
// Newton step of ew_div_fast.  Rounding t costs e a relative error of at most |u| 2^-24 per
// ulp of t, which reaches the quotient scaled by e / (e + 1): below 0.3 x 2^-24 for u <= 0,
// and for 0 < u <= 80 at most 80 x 2^-24 relative on a quotient below |x| e^-u, i.e. an
// absolute error below 0.37 x 2^-24 |x|.  For t <= 115.4 (u <= 80) the exp cannot overflow and
// the reciprocal of e + 1 (in [1.8e-35, 1]) is finite and non-zero, so only the quotient needs
// checking.  `bad` (t > 115.4, t NaN, a non-finite quotient) sends the vector to the unfused
// chain.
__device__ __forceinline__ float ew_logistic_div_fast(float x, float t, bool& bad) {
  const float d = __builtin_amdgcn_exp2f(t) + 1.0f;
  const float r = __builtin_amdgcn_rcpf(d);
  const float q = x * r;
  bad |= !(t <= 115.415603f) || !__builtin_isfinite(q);
  return __builtin_fmaf(__builtin_fmaf(-d, q, x), r, q);
}
// 1/sqrt(x) as v_rsq_f32 and one Newton step r + r/2 (1 - x r^2); `bad` as for division.
__device__ __forceinline__ float ew_rsqrt_fast(float x, bool& bad) {
  const float r = __builtin_amdgcn_rsqf(x);
  bad |= !(x > 0.0f) || !__builtin_isfinite(x) || !__builtin_isfinite(r);
  return __builtin_fmaf(r * 0.5f, __builtin_fmaf(-x * r, r, 1.0f), r);
}
__device__ __forceinline__ float ew_rsqrt(float x) {
  bool bad = false;
  const float r = ew_rsqrt_fast(x, bad);
  return bad ? 1.0f / sqrtf(x) : r;
}
__device__ __forceinline__ float h2f(u16 h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ float b2f(u16 b) { return __builtin_bit_cast(float, ((u32)b) << 16); }
__device__ __forceinline__ u16 f2h(float x) { return __builtin_bit_cast(u16, (_Float16)x); }
__device__ __forceinline__ u16 f2b(float x) { return __builtin_bit_cast(u16, (__bf16)x); }
// Two values rounded (RNE) to f16 (DT 1) or bf16 (DT 2) and packed low-first into one word,
// as one v_cvt_pk_* instruction.
template <int DT> __device__ __forceinline__ u32 pk2(float lo, float hi) {
  if (DT == 1) return __builtin_bit_cast(u32, f16x2{(_Float16)lo, (_Float16)hi});
  return __builtin_bit_cast(u32, bf16x2{(__bf16)lo, (__bf16)hi});
}
template <int DT> __device__ __forceinline__ float ld1(const void* p, i64 i) {
  if (DT == 0) return ((const float*)p)[i];
  if (DT == 1) return h2f(((const u16*)p)[i]);
  if (DT == 2) return b2f(((const u16*)p)[i]);
  if (DT == 3) return (float)((const u8*)p)[i];
  return (float)((const int*)p)[i];
}
// The 16-byte accesses of 32-bit operands are non-temporal (an element-wise program streams
// its operands once); measured on 512 MiB chains they stream 4-10% faster that way, while the
// same hint on the 16-byte accesses of 16-bit operands cost 10-15%.
template <int DT> __device__ __forceinline__ void ld4(const void* p, i64 i, float* v) {
  if (DT == 0) {
    const f32x4 q = __builtin_nontemporal_load((const f32x4*)((const float*)p + i));
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  } else if (DT == 1 || DT == 2) {
    const u32x2 q = *(const u32x2*)((const u16*)p + i);
    const u16 h[4] = {(u16)(q.x & 0xffffu), (u16)(q.x >> 16), (u16)(q.y & 0xffffu), (u16)(q.y >> 16)};
    for (int j = 0; j < 4; ++j) v[j] = DT == 1 ? h2f(h[j]) : b2f(h[j]);
  } else if (DT == 3) {
    const u32 q = *(const u32*)((const u8*)p + i);
    for (int j = 0; j < 4; ++j) v[j] = (float)((q >> (8 * j)) & 0xffu);
  } else {
    const u32x4 q = __builtin_nontemporal_load((const u32x4*)((const int*)p + i));
    v[0] = (float)(int)q.x; v[1] = (float)(int)q.y; v[2] = (float)(int)q.z; v[3] = (float)(int)q.w;
  }
}
template <int DT> __device__ __forceinline__ void st1(void* p, i64 i, float x) {
  if (DT == 0) ((float*)p)[i] = x;
  else if (DT == 1) ((u16*)p)[i] = f2h(x);
  else if (DT == 2) ((u16*)p)[i] = f2b(x);
  else if (DT == 3) ((u8*)p)[i] = x != 0.0f ? 1 : 0;
  else ((int*)p)[i] = (int)x;
}
template <int DT> __device__ __forceinline__ void st4(void* p, i64 i, const float* v) {
  if (DT == 0) {
    __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, (f32x4*)((float*)p + i));
  } else if (DT == 1 || DT == 2) {
    *(u32x2*)((u16*)p + i) = u32x2{pk2<DT>(v[0], v[1]), pk2<DT>(v[2], v[3])};
  } else if (DT == 3) {
    u32 q = 0;
    for (int j = 0; j < 4; ++j) q |= (v[j] != 0.0f ? 1u : 0u) << (8 * j);
    *(u32*)((u8*)p + i) = q;
  } else {
    __builtin_nontemporal_store(u32x4{(u32)(int)v[0], (u32)(int)v[1], (u32)(int)v[2], (u32)(int)v[3]},
                                (u32x4*)((int*)p + i));
  }
}
// 8 consecutive elements at offset i (i % 8 == 0, base aligned to 8 elements): one 16-byte
// access for 16-bit types, two for 32-bit ones.
template <int DT> __device__ __forceinline__ void ld8(const void* p, i64 i, float* v) {
  if (DT == 1 || DT == 2) {
    const u32x4 q = *(const u32x4*)((const u16*)p + i);
    const u32 w[4] = {q.x, q.y, q.z, q.w};
    for (int j = 0; j < 4; ++j) {
      const u16 lo = (u16)(w[j] & 0xffffu), hi = (u16)(w[j] >> 16);
      v[2 * j] = DT == 1 ? h2f(lo) : b2f(lo);
      v[2 * j + 1] = DT == 1 ? h2f(hi) : b2f(hi);
    }
  } else if (DT == 3) {
    const u32x2 q = *(const u32x2*)((const u8*)p + i);
    for (int j = 0; j < 4; ++j) v[j] = (float)((q.x >> (8 * j)) & 0xffu);
    for (int j = 0; j < 4; ++j) v[4 + j] = (float)((q.y >> (8 * j)) & 0xffu);
  } else {
    ld4<DT>(p, i, v);
    ld4<DT>(p, i + 4, v + 4);
  }
}
template <int DT> __device__ __forceinline__ void st8(void* p, i64 i, const float* v) {
  if (DT == 1 || DT == 2) {
    *(u32x4*)((u16*)p + i) = u32x4{pk2<DT>(v[0], v[1]), pk2<DT>(v[2], v[3]), pk2<DT>(v[4], v[5]), pk2<DT>(v[6], v[7])};
  } else if (DT == 3) {
    u32 q0 = 0, q1 = 0;
    for (int j = 0; j < 4; ++j) q0 |= (v[j] != 0.0f ? 1u : 0u) << (8 * j);
    for (int j = 0; j < 4; ++j) q1 |= (v[4 + j] != 0.0f ? 1u : 0u) << (8 * j);
    *(u32x2*)((u8*)p + i) = u32x2{q0, q1};
  } else {
    st4<DT>(p, i, v);
    st4<DT>(p, i + 4, v + 4);
  }
}
// EW_V (4 or 8) elements per lane, defined by the generated source.  The access form K of
// each operand is fixed when the source is generated: '8' / '4' = 8- / 4-element vectors at
// base + c3 (row starts and base aligned, inner size a multiple of the width), 'b' = one
// element broadcast along axis 3, 's' = element-wise at base + (c3 + j) * s3.
template <int DT, char K> __device__ __forceinline__ void ldk(const void* p, i64 base, i64 c3, i64 s3, int valid,
                                                            float* v) {
  if (K == '8') {
    ld8<DT>(p, base + c3, v);
  } else if (K == '4') {
    ld4<DT>(p, base + c3, v);
    if (EW_V == 8) {
      if (valid > 4) ld4<DT>(p, base + c3 + 4, v + 4);
      else for (int j = 4; j < EW_V; ++j) v[j] = 0.0f;
    }
  } else if (K == 'b') {
    const float x = ld1<DT>(p, base);
    for (int j = 0; j < EW_V; ++j) v[j] = x;
  } else {
    for (int j = 0; j < EW_V; ++j) v[j] = j < valid ? ld1<DT>(p, base + (c3 + j) * s3) : 0.0f;
  }
}
template <int DT, char K> __device__ __forceinline__ void stk(void* p, i64 off, int valid, const float* v) {
  if (K == '8') {
    st8<DT>(p, off, v);
  } else if (K == '4') {
    st4<DT>(p, off, v);
    if (EW_V == 8 && valid > 4) st4<DT>(p, off + 4, v + 4);
  } else {
    for (int j = 0; j < EW_V; ++j)
      if (j < valid) st1<DT>(p, off + j, v[j]);
  }
}
)JIT";

// Element expression of one instruction in terms of x = r[a][j], y = r[b][j], z = r[c][j].
const char* expr_of(int op) {
  switch (op) {
    case IHIP_EW_MOV: return "x";
    case IHIP_EW_ADD: return "x + y";
    case IHIP_EW_SUB: return "x - y";
    case IHIP_EW_MUL: return "x * y";
    case IHIP_EW_DIV: return "ew_div(x, y)";
    case IHIP_EW_MAX: return "__builtin_elementwise_maximum(x, y)";
    case IHIP_EW_MIN: return "__builtin_elementwise_minimum(x, y)";
    case IHIP_EW_NE: return "x != y ? 1.0f : 0.0f";
    case IHIP_EW_LT: return "x < y ? 1.0f : 0.0f";
    case IHIP_EW_LE: return "x <= y ? 1.0f : 0.0f";
    case IHIP_EW_GT: return "x > y ? 1.0f : 0.0f";
    case IHIP_EW_GE: return "x >= y ? 1.0f : 0.0f";
    case IHIP_EW_EQ: return "x == y ? 1.0f : 0.0f";
    case IHIP_EW_AND: return "(x != 0.0f && y != 0.0f) ? 1.0f : 0.0f";
    case IHIP_EW_OR: return "(x != 0.0f || y != 0.0f) ? 1.0f : 0.0f";
    case IHIP_EW_NOT: return "x == 0.0f ? 1.0f : 0.0f";
    case IHIP_EW_RELU: return "__builtin_elementwise_maximum(x, 0.0f)";
    case IHIP_EW_EXP: return "ew_exp(x)";
    case IHIP_EW_RSQRT: return "ew_rsqrt(x)";
    case IHIP_EW_ABS: return "fabsf(x)";
    case IHIP_EW_FLOOR: return "floorf(x)";
    case IHIP_EW_NEG: return "-x";
    case IHIP_EW_WHERE: return "x != 0.0f ? y : z";
    case IHIP_EW_CAST_F16: return "h2f(f2h(x))";
    case IHIP_EW_CAST_BF16: return "b2f(f2b(x))";
    case IHIP_EW_CAST_BOOL: return "x != 0.0f ? 1.0f : 0.0f";
    case IHIP_EW_CAST_I32: return "truncf(x)";
    default: return nullptr;
  }
}

std::string fmt(const char* f, ...) {
  va_list ap, ap2;
  va_start(ap, f);
  va_copy(ap2, ap);
  const int n = vsnprintf(nullptr, 0, f, ap);
  va_end(ap);
  std::string out(n > 0 ? static_cast<size_t>(n) : 0, '\0');
  if (n > 0) vsnprintf(&out[0], static_cast<size_t>(n) + 1, f, ap2);
  va_end(ap2);
  return out;
}

}  // namespace

// Kernel source of a validated program (registers < IHIP_EW_NATIVE_MAX_REGS, operands in range).
// Elements per lane: 8 when every operand is 16-bit or narrower (one 16-byte access each),
// else 4 (16-byte f32/i32 accesses).
int ew_jit_width(int n_inputs, const int* in_dt, int n_outputs, const int* out_dt) {
  for (int k = 0; k < n_inputs; ++k)
    if (in_dt[k] == IHIP_DT_F32 || in_dt[k] == IHIP_DT_I32) return 4;
  for (int k = 0; k < n_outputs; ++k)
    if (out_dt[k] == IHIP_DT_F32 || out_dt[k] == IHIP_DT_I32) return 4;
  return 8;
}

static bool is_tiled(char kind) { return kind == 'v' || kind == 't'; }

// Registers an instruction reads (up to 3) and the one it writes (-1 for a store).
static int ew_reads(const ihip_ew_instr& in, int (&r)[3]) {
  switch (in.op) {
    case IHIP_EW_LOAD: case IHIP_EW_IMM: case IHIP_EW_IOTA: return 0;
    case IHIP_EW_STORE: r[0] = in.a; return 1;
    case IHIP_EW_WHERE: r[0] = in.a; r[1] = in.b; r[2] = in.c; return 3;
    default:
      r[0] = in.a;
      if (in.op >= IHIP_EW_ADD && in.op <= IHIP_EW_OR) {
        r[1] = in.b;
        return 2;
      }
      return 1;
  }
}
static int ew_writes(const ihip_ew_instr& in) { return in.op == IHIP_EW_STORE ? -1 : in.dst; }

// Index of the instruction that last wrote register reg before pc, or -1.
static int ew_last_writer(const ihip_ew_instr* code, int pc, int reg) {
  for (int k = pc - 1; k >= 0; --k)
    if (ew_writes(code[k]) == reg) return k;
  return -1;
}

// True when the value instruction w writes is read by instruction `only` and no other, before
// the register is written again.
static bool ew_single_use(const ihip_ew_instr* code, int n_code, int w, int only) {
  const int reg = ew_writes(code[w]);
  for (int k = w + 1; k < n_code; ++k) {
    int r[3];
    const int nr = ew_reads(code[k], r);
    for (int i = 0; i < nr; ++i)
      if (r[i] == reg && k != only) return false;
    if (ew_writes(code[k]) == reg) return true;
  }
  return true;
}

// Logistic fusion plan: DIV(x, ADD(EXP(u), IMM 1.0)) with the exp and the add feeding only
// the division and u unchanged until it becomes x / (exp(u) + 1) in one step.  fuse_u[pc] = u's
// register at the division (-1 elsewhere) and fuse_e[pc] the exp's index; skip[pc] marks the
// exp and add it absorbs.
static void ew_plan_logistic(const ihip_ew_instr* code, int n_code, int* fuse_u, int* fuse_e, bool* skip) {
  for (int pc = 0; pc < n_code; ++pc) fuse_u[pc] = fuse_e[pc] = -1, skip[pc] = false;
  for (int pd = 0; pd < n_code; ++pd) {
    const ihip_ew_instr& dv = code[pd];
    if (dv.op != IHIP_EW_DIV || dv.a == dv.b) continue;
    const int pa = ew_last_writer(code, pd, dv.b);
    if (pa < 0 || code[pa].op != IHIP_EW_ADD || skip[pa] || !ew_single_use(code, n_code, pa, pd)) continue;
    for (int order = 0; order < 2; ++order) {
      const int re = order ? code[pa].b : code[pa].a, ro = order ? code[pa].a : code[pa].b;
      if (re == ro) continue;
      const int pe = ew_last_writer(code, pa, re), po = ew_last_writer(code, pa, ro);
      if (pe < 0 || po < 0 || code[pe].op != IHIP_EW_EXP || skip[pe]) continue;
      if (code[po].op != IHIP_EW_IMM || __builtin_bit_cast(uint32_t, code[po].imm) != 0x3f800000u) continue;
      if (!ew_single_use(code, n_code, pe, pa)) continue;
      // u still holds its value at the division: the skipped exp and add write nothing (their
      // values have no other reader), so only the instructions in between may not write u
      const int u = code[pe].a;
      bool kept = true;
      for (int k = pe + 1; k < pd && kept; ++k)
        if (k != pa) kept = ew_writes(code[k]) != u;
      if (!kept || dv.a == re) continue;
      fuse_u[pd] = u;
      fuse_e[pd] = pe;
      skip[pe] = skip[pa] = true;
      break;
    }
  }
}

// True when register reg is not written by instructions from..to-1.
static bool ew_unchanged(const ihip_ew_instr* code, int from, int to, int reg) {
  for (int k = from; k < to; ++k)
    if (ew_writes(code[k]) == reg) return false;
  return true;
}

// The IMM value register reg holds at pc, if its last writer is an IMM.
static bool ew_imm_at(const ihip_ew_instr* code, int pc, int reg, float* v) {
  const int w = ew_last_writer(code, pc, reg);
  if (w < 0 || code[w].op != IHIP_EW_IMM) return false;
  *v = code[w].imm;
  return true;
}

// For MUL at pc with operands {a, b}: the register multiplied by an IMM operand and the IMM.
static bool ew_mul_by_imm(const ihip_ew_instr* code, int pc, int* reg, float* k) {
  const ihip_ew_instr& m = code[pc];
  if (m.op != IHIP_EW_MUL) return false;
  if (ew_imm_at(code, pc, m.b, k)) return *reg = m.a, true;
  if (ew_imm_at(code, pc, m.a, k)) return *reg = m.b, true;
  return false;
}

// Expression of t = u * log2(e) for the fused logistic step at the division pd (u's register
// u_reg, read by the exp at pe), with the multiplies by constants folded:
//   u = w * k                          -> t = w * (k log2 e)
//   u = (z + k1 * ((z * z) * z)) * k   -> t = z * fma(z * z, k1 k log2 e, k log2 e)
// (any operand order; the cubic of GELU-tanh).  The values of w or z the folded form reads are
// those the matched instructions read: `saves` gets (pc, register) pairs, and the body keeps a
// copy s<pc>_<register> of that register as it is before instruction pc.  The folded forms
// round differently from the chain they replace, by a few ulp of t (the bound
// ew_logistic_div_fast states applies with a small factor).  The original instructions still
// run; where only the fallback reads their values the compiler moves them into it.
static std::string ew_logistic_t(const ihip_ew_instr* code, int pe, int u_reg,
                                 std::vector<std::pair<int, int>>& saves) {
  const double kLog2e = 1.4426950408889634;
  const int pu = ew_last_writer(code, pe, u_reg);
  int w = -1;
  float k = 0.0f;
  if (pu < 0 || !ew_mul_by_imm(code, pu, &w, &k)) return fmt("r[%d][j] * 1.44269502f", u_reg);
  const float K = static_cast<float>(k * kLog2e);
  if (!std::isfinite(K)) return fmt("r[%d][j] * 1.44269502f", u_reg);
  // w = z + c, c = b * k1, b = a * z, a = z * z, with z unchanged from a to w
  const int pw = ew_last_writer(code, pu, w);
  if (pw >= 0 && code[pw].op == IHIP_EW_ADD) {
    for (int order = 0; order < 2; ++order) {
      const int z = order ? code[pw].b : code[pw].a, c = order ? code[pw].a : code[pw].b;
      int b = -1;
      float k1 = 0.0f;
      const int pc = ew_last_writer(code, pw, c);
      if (pc < 0 || !ew_mul_by_imm(code, pc, &b, &k1)) continue;
      const int pb = ew_last_writer(code, pc, b);
      if (pb < 0 || code[pb].op != IHIP_EW_MUL || (code[pb].a != z && code[pb].b != z)) continue;
      const int a = code[pb].a == z ? code[pb].b : code[pb].a;
      const int pa = ew_last_writer(code, pb, a);
      if (pa < 0 || code[pa].op != IHIP_EW_MUL || code[pa].a != z || code[pa].b != z) continue;
      if (!ew_unchanged(code, pa, pw, z)) continue;
      const float K1 = static_cast<float>(static_cast<double>(k1) * k * kLog2e);
      if (!std::isfinite(K1)) continue;
      saves.emplace_back(pw, z);
      return fmt("s%d_%d[j] * __builtin_fmaf(s%d_%d[j] * s%d_%d[j], __builtin_bit_cast(float, %uu), "
                 "__builtin_bit_cast(float, %uu))",
                 pw, z, pw, z, pw, z, __builtin_bit_cast(uint32_t, K1), __builtin_bit_cast(uint32_t, K));
    }
  }
  saves.emplace_back(pu, w);
  return fmt("s%d_%d[j] * __builtin_bit_cast(float, %uu)", pu, w, __builtin_bit_cast(uint32_t, K));
}

// Program body: the instruction list as straight-line code over r[EW_NREG][EW_V].  Inputs and
// outputs are accessed in their form (in_kind / out_kind, see ldk); in the tiled form
// (`tiled`) staged inputs ('v', 't') are read from their LDS tile (slot = their rank among
// the staged inputs) and the other inputs from the registers they were prefetched into.
// preload (untiled form only): every LOAD was issued ahead into L<pc>[u] (u: the lane's row of
// the trip; L<pc>[0] for the row-invariant inputs of `rowinv`) and becomes a register copy;
// stores are predicated on live[u] and address row rb + u.
static std::string ew_jit_body(const ihip_ew_instr* code, int n_code, const int* in_dt, const int* out_dt,
                               const char* in_kind, const char* out_kind, bool tiled, const char* ind,
                               bool preload = false, uint32_t rowinv = 0) {
  std::string s;
  std::vector<int> fuse_u(n_code), fuse_e(n_code);
  std::vector<char> skip_v(n_code);
  bool* skip = reinterpret_cast<bool*>(skip_v.data());
  ew_plan_logistic(code, n_code, fuse_u.data(), fuse_e.data(), skip);
  // exponent expressions of the fused divisions, and the register copies they read
  std::vector<std::string> fused_t(n_code);
  std::vector<std::pair<int, int>> saves;
  for (int pc = 0; pc < n_code; ++pc) {
    if (fuse_u[pc] >= 0) fused_t[pc] = ew_logistic_t(code, fuse_e[pc], fuse_u[pc], saves);
  }
  for (int pc = 0; pc < n_code; ++pc) {
    const ihip_ew_instr& in = code[pc];
    for (const auto& sv : saves)
      if (sv.first == pc)
        s += fmt("%sfloat s%d_%d[EW_V]; for (int j = 0; j < EW_V; ++j) s%d_%d[j] = r[%d][j];\n", ind, pc, sv.second,
                 pc, sv.second, sv.second);
    if (skip[pc]) continue;
    if (fuse_u[pc] >= 0) {  // x / (exp(u) + 1): one fast pass, the unfused chain where it does not hold
      const std::string xs = fmt(" const float x = r[%d][j]; const float u = r[%d][j];", in.a, fuse_u[pc]);
      s += fmt("%s{ float t[EW_V]; bool bad = false; for (int j = 0; j < EW_V; ++j) { t[j] = "
               "ew_logistic_div_fast(r[%d][j], %s, bad); } if (bad) for (int j = 0; j < EW_V; ++j) {%s t[j] = "
               "ew_div(x, ew_exp(u) + 1.0f); } for (int j = 0; j < EW_V; ++j) r[%d][j] = t[j]; }\n",
               ind, in.a, fused_t[pc].c_str(), xs.c_str(), in.dst);
      continue;
    }
    switch (in.op) {
      case IHIP_EW_LOAD:
        if (preload) {
          s += fmt("%sfor (int j = 0; j < EW_V; ++j) r[%d][j] = L%d[%s][j];\n", ind, in.dst, pc,
                   (rowinv >> in.a) & 1u ? "0" : "u");
        } else if (tiled && is_tiled(in_kind[in.a])) {
          int slot = 0;
          for (int k = 0; k < in.a; ++k) slot += is_tiled(in_kind[k]);
          s += fmt("%sfor (int j = 0; j < EW_V; ++j) r[%d][j] = tile[%d][l3 + j][l2];\n", ind, in.dst, slot);
        } else if (tiled) {
          s += fmt("%sfor (int j = 0; j < EW_V; ++j) r[%d][j] = pre%d[pass][j];\n", ind, in.dst, in.a);
        } else {
          const int k = in.a;
          s += fmt("%sldk<%d, '%c'>(a.in_ptr[%d], c0 * a.in_stride[%d][0] + c1 * a.in_stride[%d][1] + c2 * "
                   "a.in_stride[%d][2], c3, a.in_stride[%d][3], valid, r[%d]);\n",
                   ind, in_dt[k], in_kind[k], k, k, k, k, k, in.dst);
        }
        break;
      case IHIP_EW_IMM:
        s += fmt("%sfor (int j = 0; j < EW_V; ++j) r[%d][j] = __builtin_bit_cast(float, %uu);\n", ind, in.dst,
                 __builtin_bit_cast(uint32_t, in.imm));
        break;
      case IHIP_EW_IOTA:
        if (preload)
          s += fmt("%sfor (int j = 0; j < EW_V; ++j) r[%d][j] = (float)(%s);\n", ind, in.dst,
                   in.a == 0 ? "c0[u]" : in.a == 1 ? "c1[u]" : in.a == 2 ? "c2[u]" : "c3 + j");
        else
          s += fmt("%sfor (int j = 0; j < EW_V; ++j) r[%d][j] = (float)(%s);\n", ind, in.dst,
                   in.a == 0 ? "c0" : in.a == 1 ? "c1" : in.a == 2 ? "c2" : "c3 + j");
        break;
      case IHIP_EW_STORE:
        if (preload)
          s += fmt("%sif (live[u]) stk<%d, '%c'>(a.out_ptr[%d], (rb + u) * D3 + c3, valid, r[%d]);\n", ind,
                   out_dt[in.b], out_kind[in.b], in.b, in.a);
        else
          s += fmt("%sstk<%d, '%c'>(a.out_ptr[%d], row * D3 + c3, valid, r[%d]);\n", ind, out_dt[in.b],
                   out_kind[in.b], in.b, in.a);
        break;
      default: {
        // read only the operands the opcode uses (the others may be unwritten registers)
        const bool two = in.op >= IHIP_EW_ADD && in.op <= IHIP_EW_OR;
        const bool three = in.op == IHIP_EW_WHERE;
        std::string xs = fmt(" const float x = r[%d][j];", in.a);
        if (two || three) xs += fmt(" const float y = r[%d][j];", in.b);
        if (three) xs += fmt(" const float z = r[%d][j];", in.c);
        if (in.op == IHIP_EW_DIV || in.op == IHIP_EW_RSQRT) {
          // fast form over the whole vector, one (rarely taken) branch to the checked form
          const bool div = in.op == IHIP_EW_DIV;
          s += fmt("%s{ float t[EW_V]; bool bad = false; for (int j = 0; j < EW_V; ++j) {%s t[j] = %s; }"
                   " if (bad) for (int j = 0; j < EW_V; ++j) {%s t[j] = %s; }"
                   " for (int j = 0; j < EW_V; ++j) r[%d][j] = t[j]; }\n",
                   ind, xs.c_str(), div ? "ew_div_fast(x, y, bad)" : "ew_rsqrt_fast(x, bad)", xs.c_str(),
                   expr_of(in.op), in.dst);
          break;
        }
        s += fmt("%s{ float t[EW_V]; for (int j = 0; j < EW_V; ++j) {%s", ind, xs.c_str());
        s += fmt(" t[j] = %s; } for (int j = 0; j < EW_V; ++j) r[%d][j] = t[j]; }\n", expr_of(in.op), in.dst);
      }
    }
  }
  return s;
}

// Rows per trip of the untiled form: as many as keep the preloaded row-varying inputs near 64
// floats per lane (one to four); the inputs of `rowinv` are loaded once per column vector.
int ew_jit_rows_per_trip(const ihip_ew_instr* code, int n_code, int V, uint32_t rowinv) {
  int loads = 0;
  for (int pc = 0; pc < n_code; ++pc) loads += code[pc].op == IHIP_EW_LOAD && !((rowinv >> code[pc].a) & 1u);
  const int u = loads == 0 ? 4 : 64 / (loads * V);
  return u < 1 ? 1 : u > 4 ? 4 : u;
}

std::string ew_jit_source(const ihip_ew_instr* code, int n_code, int n_inputs, const int* in_dt, int n_outputs,
                          const int* out_dt, const char* in_kind, const char* out_kind, uint32_t rowinv) {
  const int V = ew_jit_width(n_inputs, in_dt, n_outputs, out_dt);
  int nreg = IHIP_EW_MAX_REGS;  // registers the program writes: r[0 .. nreg - 1]
  for (int pc = 0; pc < n_code; ++pc)
    if (code[pc].op != IHIP_EW_STORE && code[pc].dst + 1 > nreg) nreg = code[pc].dst + 1;
  std::string s = fmt("#define EW_V %d\n#define EW_NREG %d\n", V, nreg);
  s += kPrelude;
  int nt = 0;
  for (int k = 0; k < n_inputs; ++k) nt += is_tiled(in_kind[k]);
  if (nt == 0) {
    // A lane takes one column vector (grid-strided) and, for it, EW_U rows per trip (rb ..
    // rb + EW_U - 1, grid-strided over row groups).  Inputs that do not vary along rows
    // (`rowinv`: zero stride on axes 0-2, e.g. a bias) are loaded once per column vector; the
    // loads of the other inputs for all EW_U rows are issued before any arithmetic, so EW_U x
    // (their loads) accesses are in flight per lane rather than one row's.  Rows past the last
    // load the last row and store nothing.
    s += fmt("#define EW_U %d\n", ew_jit_rows_per_trip(code, n_code, V, rowinv));
    s += "extern \"C\" __global__ __launch_bounds__(256) void ihip_ew_jit(const EwJitArgs a) {\n"
         "  const i64 D1 = a.shape[1], D2 = a.shape[2], D3 = a.shape[3];\n"
         "  for (i64 vec = (i64)blockIdx.x * blockDim.x + threadIdx.x; vec < a.nvec; vec += (i64)gridDim.x * blockDim.x) {\n"
         "    const i64 c3 = vec * EW_V;\n"
         "    const int valid = D3 - c3 < EW_V ? (int)(D3 - c3) : EW_V;\n";
    for (int pc = 0; pc < n_code; ++pc) {
      if (code[pc].op != IHIP_EW_LOAD || !((rowinv >> code[pc].a) & 1u)) continue;
      const int k = code[pc].a;
      s += fmt("    float L%d[1][EW_V];\n"
               "    ldk<%d, '%c'>(a.in_ptr[%d], 0, c3, a.in_stride[%d][3], valid, L%d[0]);\n",
               pc, in_dt[k], in_kind[k], k, k, pc);
    }
    s += "    for (i64 rb = (i64)blockIdx.y * EW_U; rb < a.rows; rb += (i64)gridDim.y * EW_U) {\n"
         "      i64 c0[EW_U], c1[EW_U], c2[EW_U];\n"
         "      bool live[EW_U];\n"
         "#pragma unroll\n"
         "      for (int u = 0; u < EW_U; ++u) {\n"
         "        live[u] = rb + u < a.rows;\n"
         "        const i64 row = live[u] ? rb + u : a.rows - 1;\n"
         "        c0[u] = 0; c1[u] = 0; c2[u] = row;\n"
         "        if (row >= D2) { c2[u] = row % D2; const i64 t = row / D2; c1[u] = t % D1; c0[u] = t / D1; }\n"
         "      }\n";
    for (int pc = 0; pc < n_code; ++pc) {
      if (code[pc].op != IHIP_EW_LOAD || ((rowinv >> code[pc].a) & 1u)) continue;
      const int k = code[pc].a;
      s += fmt("      float L%d[EW_U][EW_V];\n"
               "#pragma unroll\n"
               "      for (int u = 0; u < EW_U; ++u) ldk<%d, '%c'>(a.in_ptr[%d], c0[u] * a.in_stride[%d][0] + c1[u] * "
               "a.in_stride[%d][1] + c2[u] * a.in_stride[%d][2], c3, a.in_stride[%d][3], valid, L%d[u]);\n",
               pc, in_dt[k], in_kind[k], k, k, k, k, k, pc);
    }
    s += "#pragma unroll\n"
         "      for (int u = 0; u < EW_U; ++u) {\n"
         "        float r[EW_NREG][EW_V];\n";
    s += ew_jit_body(code, n_code, in_dt, out_dt, in_kind, out_kind, false, "        ", true, rowinv);
    s += "      }\n    }\n  }\n}\n";
    return s;
  }
  // Tiled form for inputs read across their unit-stride axis (axis 2 contiguous, axis 3
  // strided, e.g. a transpose): a workgroup takes 64 rows (axis 2) x 64 columns (axis 3).
  // Each staged input is read with consecutive threads on consecutive addresses of its axis 2
  // (16-byte vectors for kind 'v', elements for 't') and written to an LDS tile.  Then 64/EW_V
  // consecutive threads cover one row's 64 columns (EW_V each), so stores and the other
  // operands' accesses stay contiguous, in 16/EW_V passes of 4*EW_V rows.  The 65-float tile
  // pitch keeps both the staging writes and the reads conflict-free.
  // Every global load of a tile (staging, and the other inputs for all passes) is issued
  // before the first wait: lanes outside the tensor load from a clamped, valid address, so no
  // load sits behind a branch.  Such values only reach elements that are never stored.
  // Tile order: workgroups are dispatched in order of their linear id, and EW_GROUP
  // consecutive ids take consecutive axis-2 tiles at the same axis-3 tile.  With EW_GROUP =
  // 64 / element size, their staging reads cover 4 KiB of each source row; measured on
  // 8192^2 transposes: 4.9 TB/s (f32) and 4.6 TB/s (f16), against 4.3 and 3.7 with the
  // axis-3 tiles consecutive.
  int esz = 1;
  for (int k = 0; k < n_inputs; ++k)
    if (is_tiled(in_kind[k])) esz = std::max(esz, (in_dt[k] == IHIP_DT_F32 || in_dt[k] == IHIP_DT_I32) ? 4 : 2);
  s += fmt("#define EW_NT %d\n#define EW_GROUP %d\n", nt, 64 / esz);
  s += "extern \"C\" __global__ __launch_bounds__(256) void ihip_ew_jit(const EwJitArgs a) {\n"
       "  __shared__ float tile[EW_NT][64][65];\n"
       "  const i64 D0 = a.shape[0], D1 = a.shape[1], D2 = a.shape[2], D3 = a.shape[3];\n"
       "  const i64 T2 = (D2 + 63) / 64, ytiles = D0 * D1 * T2;\n"
       "  const int tid = threadIdx.x, l3 = (tid % (64 / EW_V)) * EW_V;\n"
       "  const i64 TX = (D3 + 63) / 64, ntiles = ytiles * TX;\n"
       "  for (i64 t = blockIdx.x + (i64)gridDim.x * blockIdx.y; t < ntiles; t += (i64)gridDim.x * gridDim.y) {\n"
       "    const i64 g = t / (EW_GROUP * TX), w = t % (EW_GROUP * TX);\n"
       "    const i64 gs = ytiles - g * EW_GROUP < EW_GROUP ? ytiles - g * EW_GROUP : EW_GROUP;\n"
       "    const i64 y = g * EW_GROUP + w % gs, u = y / T2, c2_0 = (y % T2) * 64, c1 = u % D1, c0 = u / D1;\n"
       "    {\n"
       "      const i64 c3_0 = (w / gs) * 64;\n";
  for (int k = 0; k < n_inputs; ++k) {
    if (in_kind[k] == 'v') {
      // VS elements of axis 2 per thread, 64/VS threads per tile row, 16/VS rows per thread
      const int vs = (in_dt[k] == IHIP_DT_F32 || in_dt[k] == IHIP_DT_I32) ? 4 : 8;
      s += fmt("      float sv%d[16 / %d][%d];\n"
               "      {\n"
               "        const void* p = a.in_ptr[%d];\n"
               "        const i64 base = c0 * a.in_stride[%d][0] + c1 * a.in_stride[%d][1], s3 = a.in_stride[%d][3];\n"
               "        const i64 g2 = c2_0 + (tid %% (64 / %d)) * %d;\n"
               "#pragma unroll\n"
               "        for (int i = 0; i < 16 / %d; ++i) {\n"
               "          const i64 g3 = c3_0 + i * 4 * %d + tid / (64 / %d);\n"
               "          ld%d<%d>(p, g2 < D2 && g3 < D3 ? base + g2 + g3 * s3 : base, sv%d[i]);\n"
               "        }\n"
               "      }\n",
               k, vs, vs, k, k, k, k, vs, vs, vs, vs, vs, vs, in_dt[k], k);
    } else if (in_kind[k] == 't') {
      s += fmt("      float sv%d[16];\n"
               "      {\n"
               "        const void* p = a.in_ptr[%d];\n"
               "        const i64 base = c0 * a.in_stride[%d][0] + c1 * a.in_stride[%d][1], s3 = a.in_stride[%d][3];\n"
               "        const i64 g2 = c2_0 + (tid & 63);\n"
               "#pragma unroll\n"
               "        for (int i = 0; i < 16; ++i) {\n"
               "          const i64 g3 = c3_0 + (tid >> 6) + 4 * i;\n"
               "          sv%d[i] = ld1<%d>(p, g2 < D2 && g3 < D3 ? base + g2 + g3 * s3 : base);\n"
               "        }\n"
               "      }\n",
               k, k, k, k, k, k, in_dt[k]);
    }
  }
  // the other inputs the program loads, for every pass, at clamped coordinates
  s += "      const i64 c3 = c3_0 + l3, c3c = c3 < D3 ? c3 : 0;\n"
       "      const int valid = D3 - c3 < EW_V ? (int)(D3 - c3) : EW_V;\n";
  uint32_t loaded = 0;
  for (int pc = 0; pc < n_code; ++pc)
    if (code[pc].op == IHIP_EW_LOAD && !is_tiled(in_kind[code[pc].a])) loaded |= 1u << code[pc].a;
  for (int k = 0; k < n_inputs; ++k)
    if ((loaded >> k) & 1u) s += fmt("      float pre%d[16 / EW_V][EW_V];\n", k);
  if (loaded) {
    s += "#pragma unroll\n"
         "      for (int pass = 0; pass < 16 / EW_V; ++pass) {\n"
         "        const i64 c2 = c2_0 + pass * 4 * EW_V + tid / (64 / EW_V), c2c = c2 < D2 ? c2 : D2 - 1;\n";
    for (int k = 0; k < n_inputs; ++k)
      if ((loaded >> k) & 1u)
        s += fmt("        ldk<%d, '%c'>(a.in_ptr[%d], c0 * a.in_stride[%d][0] + c1 * a.in_stride[%d][1] + c2c * "
                 "a.in_stride[%d][2], c3c, a.in_stride[%d][3], valid, pre%d[pass]);\n",
                 in_dt[k], in_kind[k], k, k, k, k, k, k);
    s += "      }\n";
  }
  s += "      __syncthreads();  // the previous tile is consumed\n";
  int slot = 0;
  for (int k = 0; k < n_inputs; ++k) {
    if (in_kind[k] == 'v') {
      const int vs = (in_dt[k] == IHIP_DT_F32 || in_dt[k] == IHIP_DT_I32) ? 4 : 8;
      s += fmt("#pragma unroll\n"
               "      for (int i = 0; i < 16 / %d; ++i)\n"
               "        for (int e = 0; e < %d; ++e)\n"
               "          tile[%d][i * 4 * %d + tid / (64 / %d)][(tid %% (64 / %d)) * %d + e] = sv%d[i][e];\n",
               vs, vs, slot, vs, vs, vs, vs, k);
      ++slot;
    } else if (in_kind[k] == 't') {
      s += fmt("#pragma unroll\n"
               "      for (int i = 0; i < 16; ++i) tile[%d][(tid >> 6) + 4 * i][tid & 63] = sv%d[i];\n", slot, k);
      ++slot;
    }
  }
  s += "      __syncthreads();\n"
       "#pragma unroll\n"
       "      for (int pass = 0; pass < 16 / EW_V; ++pass) {\n"
       "        const int l2 = pass * 4 * EW_V + tid / (64 / EW_V);\n"
       "        const i64 c2 = c2_0 + l2, row = (c0 * D1 + c1) * D2 + c2;\n"
       "        if (c2 < D2 && c3 < D3) {\n"
       "          float r[EW_NREG][EW_V];\n";
  s += ew_jit_body(code, n_code, in_dt, out_dt, in_kind, out_kind, true, "          ");
  s += "        }\n      }\n    }\n  }\n}\n";
  return s;
}

namespace {

// One specialised program: its code object, and the module loaded from it on each device.
struct JitEntry {
  std::string object;  // code object from hiprtc; empty when compilation failed
  std::string error;
  std::unordered_map<int, hipFunction_t> fn;  // device -> kernel
};

std::mutex g_jit_mu;
std::unordered_map<std::string, JitEntry> g_jit;  // key: generated source

void compile(const std::string& src, JitEntry& e) {
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, src.c_str(), "ihip_ew_jit.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS) {
    e.error = "hiprtcCreateProgram failed";
    return;
  }
  // gfx950 only; packed-FP32 instructions stay off as in the library's own kernels.
  const char* opts[] = {"--offload-arch=gfx950", "-O3", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
  const hiprtcResult r = hiprtcCompileProgram(prog, 6, opts);
  if (r != HIPRTC_SUCCESS) {
    size_t n = 0;
    hiprtcGetProgramLogSize(prog, &n);
    std::string log(n, '\0');
    if (n) hiprtcGetProgramLog(prog, &log[0]);
    e.error = std::string("hiprtc: ") + hiprtcGetErrorString(r) + ": " + log.substr(0, 300);
    hiprtcDestroyProgram(&prog);
    return;
  }
  size_t n = 0;
  hiprtcGetCodeSize(prog, &n);
  e.object.assign(n, '\0');
  hiprtcGetCode(prog, &e.object[0]);
  hiprtcDestroyProgram(&prog);
}

// Cache entry of a source, compiled on first request (caller holds g_jit_mu).
JitEntry& entry(const std::string& src) {
  auto it = g_jit.find(src);
  if (it == g_jit.end()) {
    it = g_jit.emplace(src, JitEntry{}).first;
    compile(src, it->second);
  }
  return it->second;
}

}  // namespace

namespace {

// Kernel arguments, generated source and grid of one launch of a validated program.
struct JitPlan {
  EwJitArgs a{};
  std::string src;
  unsigned gx = 0, gy = 0;
};

// Plans a launch: the access form of every operand (see ldk), the LDS-staged inputs, the
// arguments and the grid.  Returns false for an empty iteration space (nothing to launch).
// Pointers are only inspected for alignment, so this needs no device.
bool plan_jit(const ihip_ew_instr* code, int n_code, const ihip_ew_operand* inputs, int n_inputs,
              const ihip_ew_operand* outputs, int n_outputs, const int64_t (&shape)[4], JitPlan& pl) {
  EwJitArgs& a = pl.a;
  for (int d = 0; d < 4; ++d) a.shape[d] = shape[d];
  int in_dt[IHIP_EW_NATIVE_MAX_INPUTS] = {}, out_dt[IHIP_EW_NATIVE_MAX_OUTPUTS] = {};
  for (int k = 0; k < n_inputs; ++k) in_dt[k] = inputs[k].dtype;
  for (int k = 0; k < n_outputs; ++k) out_dt[k] = outputs[k].dtype;
  const int V = ew_jit_width(n_inputs, in_dt, n_outputs, out_dt);
  a.rows = shape[0] * shape[1] * shape[2];
  a.nvec = (shape[3] + V - 1) / V;
  if (a.rows == 0 || a.nvec == 0) return false;
  const auto esize = [](int dt) -> int64_t { return dt == IHIP_DT_F32 || dt == IHIP_DT_I32 ? 4 : dt == IHIP_DT_BOOL ? 1 : 2; };
  // W-element vectors need every row to start at a multiple of W elements and an aligned base.
  const auto vec_ok = [&](const void* ptr, const int64_t* st, int dt, int64_t w) {
    const bool rows = (st == nullptr) || ((st[0] % w == 0 || shape[0] == 1) && (st[1] % w == 0 || shape[1] == 1) &&
                                          (st[2] % w == 0 || shape[2] == 1) && st[3] == 1);
    return shape[3] % w == 0 && rows && reinterpret_cast<uintptr_t>(ptr) % (w * esize(dt)) == 0;
  };
  // Inputs read across their unit-stride axis (axis 2 contiguous, axis 3 strided) are staged
  // through LDS tiles, at most kMaxTiled of them (16.6 KiB each).
  constexpr int kMaxTiled = 4;
  uint32_t tile_mask = 0;
  if (shape[2] > 1 && shape[3] > 1)
    for (int k = 0; k < n_inputs && __builtin_popcount(tile_mask) < kMaxTiled; ++k)
      if (inputs[k].stride[2] == 1 && inputs[k].stride[3] != 0 && inputs[k].stride[3] != 1) tile_mask |= 1u << k;
  // A staged input is read in 16-byte vectors ('v', else element-wise 't') when every vector
  // starts at a multiple of its width and stays inside axis 2.
  const auto stage_vec = [&](int k) {
    const int64_t vs = (in_dt[k] == IHIP_DT_F32 || in_dt[k] == IHIP_DT_I32) ? 4 : 8;
    const int64_t* st = inputs[k].stride;
    return shape[2] % vs == 0 && st[3] % vs == 0 && (st[0] % vs == 0 || shape[0] == 1) &&
           (st[1] % vs == 0 || shape[1] == 1) && reinterpret_cast<uintptr_t>(inputs[k].ptr) % 16 == 0;
  };
  char in_kind[IHIP_EW_NATIVE_MAX_INPUTS + 1] = {}, out_kind[IHIP_EW_NATIVE_MAX_OUTPUTS + 1] = {};
  for (int k = 0; k < n_inputs; ++k) {
    a.in_ptr[k] = inputs[k].ptr;
    for (int d = 0; d < 4; ++d) a.in_stride[k][d] = inputs[k].stride[d];
    const int64_t* st = inputs[k].stride;
    in_kind[k] = ((tile_mask >> k) & 1u)                          ? (stage_vec(k) ? 'v' : 't')
                 : (V == 8 && vec_ok(inputs[k].ptr, st, in_dt[k], 8)) ? '8'
                 : vec_ok(inputs[k].ptr, st, in_dt[k], 4)               ? '4'
                 : st[3] == 0                                           ? 'b'
                                                                        : 's';
  }
  for (int k = 0; k < n_outputs; ++k) {
    a.out_ptr[k] = const_cast<void*>(outputs[k].ptr);
    out_kind[k] = (V == 8 && vec_ok(outputs[k].ptr, nullptr, out_dt[k], 8)) ? '8'
                  : vec_ok(outputs[k].ptr, nullptr, out_dt[k], 4)            ? '4'
                                                                             : 's';
  }
  // Inputs with zero stride (or extent 1) on axes 0-2 are the same for every row.
  uint32_t rowinv = 0;
  for (int k = 0; k < n_inputs; ++k) {
    const int64_t* st = inputs[k].stride;
    if ((st[0] == 0 || shape[0] == 1) && (st[1] == 0 || shape[1] == 1) && (st[2] == 0 || shape[2] == 1))
      rowinv |= 1u << k;
  }
  pl.src = ew_jit_source(code, n_code, n_inputs, in_dt, n_outputs, out_dt, in_kind, out_kind, rowinv);
  if (tile_mask != 0) {  // one workgroup per 64 x 64 tile (linear id; grid-strided beyond the grid limits)
    const int64_t tx = (shape[3] + 63) / 64, ty = shape[0] * shape[1] * ((shape[2] + 63) / 64);
    pl.gx = static_cast<unsigned>(tx < 65535 ? tx : 65535);
    pl.gy = static_cast<unsigned>(ty < 65535 ? ty : 65535);
  } else {
    // Up to 16384 256-lane workgroups, grid-strided over row groups and vectors beyond that.
    // A grid of 4096 left a partly filled last round of workgroups on the chip: on 512 MiB -
    // 1 GiB chains, 16384 ran 3-9% faster (bf16 GELU 5.26 -> 5.68 TB/s, f32 GELU 5.82 -> 6.17,
    // bias + ReLU 5.96 -> 6.15), as fast as one trip per lane (65535 row groups).
    const int64_t bx = (a.nvec + 255) / 256;
    pl.gx = static_cast<unsigned>(bx < 1024 ? bx : 1024);
    const int U = ew_jit_rows_per_trip(code, n_code, V, rowinv);
    int64_t gy = (16384 + pl.gx - 1) / pl.gx;
    if (gy > (a.rows + U - 1) / U) gy = (a.rows + U - 1) / U;
    if (gy > 65535) gy = 65535;
    pl.gy = static_cast<unsigned>(gy);
  }
  return true;
}

bool compile_checked(const std::string& src, std::string* why) {
  std::lock_guard<std::mutex> lock(g_jit_mu);
  JitEntry& e = entry(src);
  if (!e.error.empty() && why) *why = e.error;
  return e.error.empty();
}

}  // namespace

// Compile (once) the native code of a validated program for the given operand types, in the
// form that dense operands select (every input and output read and written in full-width
// vectors); no device is needed.  Returns false with *why set when compilation fails.
bool prepare_elementwise_jit(const ihip_ew_instr* code, int n_code, int n_inputs, const int* in_dt, int n_outputs,
                             const int* out_dt, std::string* why) {
  const char w = ew_jit_width(n_inputs, in_dt, n_outputs, out_dt) == 8 ? '8' : '4';
  char in_kind[IHIP_EW_NATIVE_MAX_INPUTS + 1] = {}, out_kind[IHIP_EW_NATIVE_MAX_OUTPUTS + 1] = {};
  for (int k = 0; k < n_inputs; ++k) in_kind[k] = w;
  for (int k = 0; k < n_outputs; ++k) out_kind[k] = w;
  return compile_checked(ew_jit_source(code, n_code, n_inputs, in_dt, n_outputs, out_dt, in_kind, out_kind, 0), why);
}

// Compile (once) exactly the code that launch_elementwise_jit would run for these operands and
// shape; no device is needed.
bool prepare_elementwise_jit_operands(const ihip_ew_instr* code, int n_code, const ihip_ew_operand* inputs,
                                      int n_inputs, const ihip_ew_operand* outputs, int n_outputs,
                                      const int64_t (&shape)[4], std::string* why) {
  JitPlan pl;
  if (!plan_jit(code, n_code, inputs, n_inputs, outputs, n_outputs, shape, pl)) return true;
  return compile_checked(pl.src, why);
}

// The source that launch_elementwise_jit would compile for these operands and shape ("" when
// the launch is empty); no device is needed.
std::string source_elementwise_jit_operands(const ihip_ew_instr* code, int n_code, const ihip_ew_operand* inputs,
                                            int n_inputs, const ihip_ew_operand* outputs, int n_outputs,
                                            const int64_t (&shape)[4]) {
  JitPlan pl;
  return plan_jit(code, n_code, inputs, n_inputs, outputs, n_outputs, shape, pl) ? pl.src : std::string();
}

// Launch the specialised kernel of a validated program; compiles on first use.  Returns
// hipErrorNotSupported with *why set when the program cannot be compiled.
hipError_t launch_elementwise_jit(const ihip_ew_instr* code, int n_code, const ihip_ew_operand* inputs, int n_inputs,
                                  const ihip_ew_operand* outputs, int n_outputs, const int64_t (&shape)[4],
                                  hipStream_t s, std::string* why) {
  JitPlan pl;
  if (!plan_jit(code, n_code, inputs, n_inputs, outputs, n_outputs, shape, pl)) return hipSuccess;
  int dev = 0;
  hipError_t he = hipGetDevice(&dev);
  if (he != hipSuccess) return he;
  hipFunction_t fn = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_jit_mu);
    JitEntry& e = entry(pl.src);
    if (!e.error.empty()) {
      if (why) *why = e.error;
      return hipErrorNotSupported;
    }
    auto f = e.fn.find(dev);
    if (f == e.fn.end()) {  // first launch on this device: load the module (kept until the process ends)
      hipModule_t mod = nullptr;
      he = hipModuleLoadData(&mod, e.object.data());
      if (he == hipSuccess) he = hipModuleGetFunction(&fn, mod, "ihip_ew_jit");
      if (he != hipSuccess) return he;
      e.fn.emplace(dev, fn);
    } else {
      fn = f->second;
    }
  }
  void* params[] = {&pl.a};
  return hipModuleLaunchKernel(fn, pl.gx, pl.gy, 1, 256, 1, 1, 0, s, params, nullptr);
}

}  // namespace ihip
