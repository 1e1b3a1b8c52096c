// Host-side checks of libintentir_hip's C-ABI, built with AddressSanitizer and
// UndefinedBehaviorSanitizer on the host code only (device code is compiled as usual and
// never launched: every call here either is rejected by the argument checks before any HIP
// call, or needs no device).  Exercises:
//  * every entry point's rejection paths (shapes, overflow, null pointers, kinds, knobs,
//    workspaces);
//  * the element-wise program checker on hand-written malformed programs and on 20000
//    pseudo-random ones (any byte values in every instruction field);
//  * the native-code planner and source generator (ihip_elementwise_source) on valid
//    programs with operands at many alignments, strides and shapes, and one hiprtc compile.
// Prints "ALL OK" and exits 0; a sanitizer report or a failed expectation exits non-zero.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "../../include/intentir_hip.h"

static int g_fail = 0;
#define EXPECT(cond, ...)                                  \
  do {                                                     \
    if (!(cond)) {                                         \
      fprintf(stderr, "FAILED %s:%d: ", __FILE__, __LINE__); \
      fprintf(stderr, __VA_ARGS__);                        \
      fprintf(stderr, " [%s]\n", ihip_last_error());       \
      ++g_fail;                                            \
    }                                                      \
  } while (0)

static void* fake(uintptr_t a) { return reinterpret_cast<void*>(a); }  // never dereferenced

static uint32_t g_rng = 12345;
static uint32_t rnd() {
  g_rng = g_rng * 1664525u + 1013904223u;
  return g_rng >> 8;
}

static ihip_ew_instr ins(int op, int dst, int a, int b = 0, int c = 0, float imm = 0.f) {
  ihip_ew_instr i;
  memset(&i, 0, sizeof(i));
  i.op = (uint8_t)op, i.dst = (uint8_t)dst, i.a = (uint8_t)a, i.b = (uint8_t)b, i.c = (uint8_t)c, i.imm = imm;
  return i;
}

static ihip_ew_operand opnd(uintptr_t p, int dt, int64_t s0, int64_t s1, int64_t s2, int64_t s3) {
  ihip_ew_operand o;
  memset(&o, 0, sizeof(o));
  o.ptr = fake(p), o.dtype = dt, o.stride[0] = s0, o.stride[1] = s1, o.stride[2] = s2, o.stride[3] = s3;
  return o;
}

static void row_kernels() {
  EXPECT(ihip_abi_version() == IHIP_ABI_VERSION, "abi");
  EXPECT(ihip_reduce_any_rows_f32(nullptr, nullptr, -1, 4, 0.f, nullptr) == IHIP_ERR_INVALID_ARG, "any shape");
  EXPECT(ihip_reduce_any_rows_f32(nullptr, nullptr, 1LL << 62, 1LL << 62, 0.f, nullptr) == IHIP_ERR_INVALID_ARG,
         "any overflow");
  EXPECT(ihip_reduce_any_rows_f32(nullptr, (uint8_t*)fake(64), 4, 4, 0.f, nullptr) == IHIP_ERR_INVALID_ARG, "any x");
  EXPECT(ihip_reduce_any_rows_u8(nullptr, nullptr, 4, -4, nullptr) == IHIP_ERR_INVALID_ARG, "any u8 shape");
  EXPECT(ihip_reduce_rows_f32(nullptr, nullptr, 4, 4, 7, nullptr) == IHIP_ERR_INVALID_ARG, "reduce kind");
  EXPECT(ihip_reduce_rows_f32((float*)fake(64), (float*)fake(64), 4, 0, IHIP_REDUCE_MAX, nullptr) ==
             IHIP_ERR_INVALID_ARG, "max over empty axis");
  EXPECT(ihip_reduce_rows_f32_ws((float*)fake(64), (float*)fake(64), 64, 1 << 20, 0, fake(256), 8, nullptr) ==
             IHIP_ERR_INVALID_ARG, "workspace too small");
  EXPECT(ihip_reduce_rows_f32_ws((float*)fake(64), (float*)fake(64), 64, 1 << 20, 0, fake(258), 1 << 20, nullptr) ==
             IHIP_ERR_INVALID_ARG, "workspace alignment");
  EXPECT(ihip_reduce_rows_f32_noalloc(nullptr, nullptr, -3, 5, 0, nullptr) == IHIP_ERR_INVALID_ARG, "noalloc shape");
  EXPECT(ihip_reduce_rows_f32_noalloc((float*)fake(64), (float*)fake(64), 64, 1 << 20, 9, nullptr) ==
             IHIP_ERR_INVALID_ARG, "noalloc kind");
  for (int64_t m : {0LL, 1LL, 7LL, 255LL, 256LL, 1LL << 40})
    for (int64_t n : {0LL, 1LL, 4095LL, 1LL << 20, 1LL << 40}) {
      const int64_t w = ihip_reduce_rows_f32_workspace_size(m, n);
      EXPECT(w >= 0 && w <= 256 * 64 * 4, "workspace size %lld for [%lld, %lld]", (long long)w, (long long)m,
             (long long)n);
    }
  EXPECT(ihip_softmax_rows_f32(nullptr, nullptr, 2, -1, nullptr) == IHIP_ERR_INVALID_ARG, "softmax shape");
  EXPECT(ihip_softmax_rows_f32_ex(nullptr, nullptr, 0, 8, 3, nullptr) == IHIP_ERR_INVALID_ARG, "rows_per_wg 3");
  EXPECT(ihip_softmax_rows_f32_ex((float*)fake(64), (float*)fake(128), 4, 8192, 2, nullptr) == IHIP_ERR_INVALID_ARG,
         "rows_per_wg on a multi-wave row");
  // long rows: 32 segments of 1024 vectors per 128256-float row at 64 rows, 2 floats each
  EXPECT(ihip_softmax_rows_f32_workspace_size(64, 128256) == 64 * 32 * 8, "softmax split workspace");
  EXPECT(ihip_softmax_rows_f32_workspace_size(64, 65536) == 0, "softmax rows not split");
  EXPECT(ihip_softmax_rows_f32_workspace_size(1, 1048580) == 257 * 8, "softmax split: 257 segments of 1024 vectors");
  EXPECT(ihip_softmax_rows_f32_workspace_size(1LL << 20, 1LL << 30) == 0, "softmax split grid past 2^31");
  EXPECT(ihip_softmax_rows_f32_workspace_size(-1, 128256) == 0, "softmax split negative");
  EXPECT(ihip_softmax_rows_f32_workspace_size(1LL << 40, 1LL << 40) == 0, "softmax split overflow");
  EXPECT(ihip_softmax_rows_f32_ws((float*)fake(64), (float*)fake(64), 64, 128256, fake(256), 8, nullptr) ==
             IHIP_ERR_INVALID_ARG, "softmax workspace too small");
  EXPECT(ihip_softmax_rows_f32_ws((float*)fake(64), (float*)fake(64), 64, 128256, fake(260), 16384, nullptr) ==
             IHIP_ERR_INVALID_ARG, "softmax workspace alignment");
  EXPECT(ihip_softmax_rows_f32_ws((float*)fake(64), (float*)fake(64), 64, 128256, nullptr, 4096, nullptr) ==
             IHIP_ERR_INVALID_ARG, "softmax workspace null with bytes");
  EXPECT(ihip_softmax_rows_f32_ws((float*)fake(64), (float*)fake(64), 64, 128256, fake(256), -8, nullptr) ==
             IHIP_ERR_INVALID_ARG, "softmax workspace negative");
  EXPECT(ihip_softmax_rows_f32_ws(nullptr, nullptr, 3, -2, nullptr, 0, nullptr) == IHIP_ERR_INVALID_ARG,
         "softmax ws shape");
  EXPECT(ihip_softmax_rows_f32_ws(nullptr, nullptr, 0, 128256, nullptr, 0, nullptr) == IHIP_OK, "softmax ws M = 0");
  for (int64_t m : {0LL, 1LL, 31LL, 4096LL, 1LL << 30, 1LL << 40})
    for (int64_t n : {0LL, 65536LL, 65537LL, 1LL << 20, 1LL << 22, 1LL << 40}) {
      const int64_t w = ihip_softmax_rows_f32_workspace_size(m, n);
      EXPECT(w >= 0 && (w == 0 || w % (8 * m) == 0) && w / 8 <= 0x7fffffffLL, "softmax workspace %lld for [%lld, %lld]",
             (long long)w, (long long)m, (long long)n);
    }
  EXPECT(ihip_layernorm_rows_f16(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 4, 8, 1e-5f, nullptr) ==
             IHIP_ERR_INVALID_ARG, "layernorm null");
  EXPECT(ihip_gather2d_f32((float*)fake(64), (int32_t*)fake(64), (int32_t*)fake(64), (float*)fake(64), 7, 9, -1, 0.f,
                           nullptr) == IHIP_ERR_INVALID_ARG, "gather negative L");
  EXPECT(ihip_gather2d_f32((float*)fake(64), nullptr, (int32_t*)fake(64), (float*)fake(64), 7, 9, 32, 0.f,
                           nullptr) == IHIP_ERR_INVALID_ARG, "gather null index");
  EXPECT(ihip_gather2d_f32(nullptr, (int32_t*)fake(64), (int32_t*)fake(64), (float*)fake(64), 7, 9, 32, 0.f,
                           nullptr) == IHIP_ERR_INVALID_ARG, "gather null inp");
  EXPECT(ihip_gather2d_f32((float*)fake(64), (int32_t*)fake(64), (int32_t*)fake(64), (float*)fake(64), 1LL << 40,
                           1LL << 40, 32, 0.f, nullptr) == IHIP_ERR_INVALID_ARG, "gather overflow");
  EXPECT(ihip_gather2d_f32(nullptr, nullptr, nullptr, nullptr, 7, 9, 0, 0.f, nullptr) == IHIP_OK, "gather L = 0");
  EXPECT(ihip_bias_gelu_tanh_axpy_bf16(nullptr, nullptr, nullptr, -2, 8, 0.5f, nullptr) == IHIP_ERR_INVALID_ARG,
         "gelu shape");
  EXPECT(ihip_gemm_bf16_bias_relu(nullptr, nullptr, nullptr, nullptr, 2, 2, 2, 1, nullptr) == IHIP_ERR_INVALID_ARG,
         "gemm null");
  EXPECT(ihip_gemm_bf16_bias_relu_ex(nullptr, nullptr, nullptr, nullptr, 0, 0, 0, 0, 0, 1, 64, nullptr) ==
             IHIP_ERR_INVALID_ARG, "gemm tile 64");
  EXPECT(ihip_gemm_bf16_bias_relu_t(nullptr, nullptr, nullptr, nullptr, 1LL << 40, 1LL << 40, 1LL << 40, 0, 0, 0,
                                    nullptr) == IHIP_ERR_INVALID_ARG, "gemm overflow");
  EXPECT(ihip_gemm_bf16_bias_relu_ws(nullptr, nullptr, nullptr, nullptr, 0, 0, 0, 0, 0, 1, 0, nullptr, 64, nullptr) ==
             IHIP_ERR_INVALID_ARG, "gemm workspace bytes at null");
  EXPECT(ihip_gemm_bf16_bias_relu_ws(nullptr, nullptr, nullptr, nullptr, 0, 0, 0, 0, 0, 1, 0, nullptr, -1, nullptr) ==
             IHIP_ERR_INVALID_ARG, "gemm negative workspace");
  EXPECT(ihip_gemm_workspace_size(1LL << 40, 1LL << 40, 1LL << 40, 0, 0) == 0, "gemm workspace size overflow");
  EXPECT(ihip_gemm_workspace_size(7, 9, 3, 0, 0) == 256 + 256, "gemm workspace size 7x9x3");
  EXPECT(ihip_gemm_workspace_size(64, 263, 64, 0, 1) == 0, "gemm workspace size with B as [N, K]");
  // split-K: sizes, and argument errors caught before any launch (no device needed)
  EXPECT(ihip_gemm_workspace_size(1024, 1024, 8192, 0, 0) == 4LL * 1024 * 1024 * 4, "gemm split-K workspace (4 segments)");
  EXPECT(ihip_gemm_splitk_workspace_size(1024, 1024, 8192, 1) == 0, "no partials unsplit");
  // 2 segments x 8 rows x 4 floats (N = 3 padded to 4) x 4 bytes = 256; 2 x 3 x 12 x 4 = 288 -> 512
  EXPECT(ihip_gemm_splitk_workspace_size(8, 3, 4096, 2) == 256, "partials padded to 4 columns");
  EXPECT(ihip_gemm_splitk_workspace_size(3, 12, 4096, 2) == 512, "partials 256-byte aligned");
  EXPECT(ihip_gemm_splitk_workspace_size(8, 8, 4096, -1) == 0, "negative split count");
  EXPECT(ihip_gemm_splitk_workspace_size(1LL << 40, 1LL << 40, 1LL << 40, 0) == 0, "split-K size overflow");
  EXPECT(ihip_gemm_bf16_bias_relu_splitk(nullptr, nullptr, nullptr, nullptr, 8, 8, 64, 0, 0, 1, 64, 2, nullptr, 0,
                                         nullptr) == IHIP_ERR_INVALID_ARG,
         "split-K tile 64");
  EXPECT(ihip_gemm_bf16_bias_relu_splitk(nullptr, nullptr, nullptr, nullptr, 8, 8, 64, 0, 0, 1, 0, -2, nullptr, 0,
                                         nullptr) == IHIP_ERR_INVALID_ARG,
         "split-K negative count");
  EXPECT(ihip_gemm_bf16_bias_relu_splitk(nullptr, nullptr, nullptr, nullptr, 8, 8, 0, 0, 0, 1, 0, 2, nullptr, 0,
                                         nullptr) == IHIP_ERR_INVALID_ARG,
         "split-K with K = 0");
  EXPECT(ihip_gemm_bf16_bias_relu_splitk(nullptr, nullptr, nullptr, nullptr, 8, 8, 4096, 0, 0, 1, 0, 2, nullptr, 100,
                                         nullptr) == IHIP_ERR_INVALID_ARG,
         "split-K workspace bytes at a null pointer");
  EXPECT(ihip_gemm_bf16_bias_relu_splitk(nullptr, nullptr, nullptr, nullptr, 8, 8, 4096, 0, 0, 1, 0, 2, nullptr, 0,
                                         nullptr) == IHIP_ERR_INVALID_ARG,
         "split-K workspace too small");
  EXPECT(ihip_gemm_bf16_bias_relu_splitk(nullptr, nullptr, nullptr, nullptr, 0, 8, 4096, 0, 0, 1, 0, 2, nullptr, 0,
                                         nullptr) == 0,
         "split-K with M = 0 is a no-op");
}

static void program_checker() {
  const int64_t shape[2] = {4, 8};
  ihip_ew_operand in[2] = {opnd(256, IHIP_DT_F32, 0, 0, 8, 1), opnd(512, IHIP_DT_F32, 0, 0, 0, 1)};
  ihip_ew_operand out[1] = {opnd(1024, IHIP_DT_F32, 0, 0, 0, 0)};
  struct Bad {
    std::vector<ihip_ew_instr> code;
    const char* what;
  } bad[] = {
      {{ins(99, 0, 0)}, "unknown opcode"},
      {{ins(IHIP_EW_LOAD, 0, 5), ins(IHIP_EW_STORE, 0, 0)}, "load of a missing input"},
      {{ins(IHIP_EW_LOAD, 255, 0), ins(IHIP_EW_STORE, 0, 255)}, "register out of range"},
      {{ins(IHIP_EW_ADD, 0, 1, 2), ins(IHIP_EW_STORE, 0, 0)}, "reads unwritten registers"},
      {{ins(IHIP_EW_LOAD, 0, 0)}, "output never stored"},
      {{ins(IHIP_EW_LOAD, 0, 0), ins(IHIP_EW_STORE, 0, 0), ins(IHIP_EW_STORE, 0, 0)}, "output stored twice"},
      {{ins(IHIP_EW_LOAD, 0, 0), ins(IHIP_EW_STORE, 0, 3)}, "store to a missing output"},
      {{ins(IHIP_EW_IOTA, 0, 4), ins(IHIP_EW_STORE, 0, 0)}, "iota axis"},
      {{ins(IHIP_EW_LOAD, 0, 0), ins(IHIP_EW_WHERE, 1, 0, 0, 7), ins(IHIP_EW_STORE, 0, 1)}, "where operand"},
  };
  for (auto& b : bad)
    EXPECT(ihip_elementwise_program(b.code.data(), (int)b.code.size(), in, 2, out, 1, shape, 2, nullptr) ==
               IHIP_ERR_INVALID_ARG, "%s accepted", b.what);
  std::vector<ihip_ew_instr> big(IHIP_EW_NATIVE_MAX_CODE + 1, ins(IHIP_EW_IMM, 0, 0));
  EXPECT(ihip_elementwise_program(big.data(), (int)big.size(), in, 2, out, 1, shape, 2, nullptr) ==
             IHIP_ERR_INVALID_ARG, "too many instructions");
  {  // past the interpreter kernel's register file: refused in INTERP mode before any launch
    const int prev = ihip_elementwise_mode(IHIP_EW_MODE_INTERP);
    ihip_ew_instr wide[] = {ins(IHIP_EW_LOAD, 9, 0), ins(IHIP_EW_STORE, 0, 9)};
    EXPECT(ihip_elementwise_program(wide, 2, in, 2, out, 1, shape, 2, nullptr) == IHIP_ERR_INVALID_ARG,
           "register 9 accepted by the interpreter");
    ihip_elementwise_mode(prev);
  }
  ihip_ew_instr ok[] = {ins(IHIP_EW_LOAD, 0, 0), ins(IHIP_EW_STORE, 0, 0)};
  const int64_t shape5[5] = {1, 1, 1, 1, 1};
  EXPECT(ihip_elementwise_program(ok, 2, in, 2, out, 1, shape5, 5, nullptr) == IHIP_ERR_INVALID_ARG, "rank 5");
  ihip_ew_operand badt = opnd(256, 17, 0, 0, 8, 1);
  EXPECT(ihip_elementwise_program(ok, 2, &badt, 1, out, 1, shape, 2, nullptr) == IHIP_ERR_INVALID_ARG, "dtype");
  const int64_t negshape[2] = {4, -8};
  EXPECT(ihip_elementwise_program(ok, 2, in, 2, out, 1, negshape, 2, nullptr) == IHIP_ERR_INVALID_ARG, "negative axis");
  // random programs, mostly well formed (registers read after they are written, one store per
  // output) with a few corrupt fields: every one is accepted or rejected cleanly, and each
  // accepted one goes through the native-code planner, fusion planner and source generator
  const int64_t empty[2] = {0, 8};
  const int ops[] = {IHIP_EW_IMM, IHIP_EW_IOTA, IHIP_EW_MOV, IHIP_EW_ADD, IHIP_EW_SUB, IHIP_EW_MUL, IHIP_EW_DIV,
                     IHIP_EW_MAX, IHIP_EW_MIN, IHIP_EW_NE, IHIP_EW_LT, IHIP_EW_AND, IHIP_EW_OR, IHIP_EW_NOT,
                     IHIP_EW_RELU, IHIP_EW_EXP, IHIP_EW_RSQRT, IHIP_EW_ABS, IHIP_EW_FLOOR, IHIP_EW_NEG, IHIP_EW_WHERE,
                     IHIP_EW_CAST_F16, IHIP_EW_CAST_BF16, IHIP_EW_CAST_BOOL, IHIP_EW_CAST_I32, IHIP_EW_LOAD};
  int accepted = 0, sourced = 0;
  for (int t = 0; t < 20000; ++t) {
    // every fourth program runs past the interpreter limits (native form: more registers and
    // instructions, so the generator's register array and fusion planner see larger programs)
    const bool wide = t % 4 == 0;
    const int n = 2 + (int)(rnd() % ((wide ? 3 * IHIP_EW_MAX_CODE : IHIP_EW_MAX_CODE) - 2));
    std::vector<ihip_ew_instr> code;
    std::vector<int> live = {0};  // registers that hold values
    const auto pick = [&]() { return live[rnd() % live.size()]; };
    code.push_back(ins(IHIP_EW_LOAD, 0, 0));
    for (int k = 1; k + 1 < n; ++k) {
      const int op = ops[rnd() % (sizeof(ops) / sizeof(ops[0]))];
      const int dst = (int)(rnd() % (wide ? 5 * IHIP_EW_MAX_REGS : IHIP_EW_MAX_REGS));
      ihip_ew_instr c = ins(op, dst, pick(), pick(), pick(), (rnd() % 4 == 0) ? 1.0f : (float)(int)(rnd() % 9) - 4.f);
      if (op == IHIP_EW_LOAD) c.a = (uint8_t)(rnd() % 2);
      if (op == IHIP_EW_IOTA) c.a = (uint8_t)(rnd() % 4);
      code.push_back(c);
      bool known = false;
      for (int r : live) known |= r == dst;
      if (!known) live.push_back(dst);
    }
    code.push_back(ins(IHIP_EW_STORE, 0, pick(), 0));
    if (rnd() % 8 == 0) {  // corrupt one field
      ihip_ew_instr& c = code[rnd() % code.size()];
      switch (rnd() % 4) {
        case 0: c.op = (uint8_t)(rnd() % 256); break;
        case 1: c.dst = (uint8_t)(rnd() % 256); break;
        case 2: c.a = (uint8_t)(rnd() % 256); break;
        default: c.b = (uint8_t)(rnd() % 256); break;
      }
    }
    const int st = ihip_elementwise_program(code.data(), (int)code.size(), in, 2, out, 1, empty, 2, nullptr);
    EXPECT(st == IHIP_OK || st == IHIP_ERR_INVALID_ARG, "random program status %d", st);
    if (st != IHIP_OK) continue;
    ++accepted;
    int64_t len = -1;
    const int64_t sh[2] = {3 + (int64_t)(rnd() % 40), 1 + (int64_t)(rnd() % 70)};
    EXPECT(ihip_elementwise_source(code.data(), (int)code.size(), in, 2, out, 1, sh, 2, nullptr, 0, &len) == IHIP_OK &&
               len > 0, "source of an accepted program");
    sourced += len > 0;
  }
  printf("random programs accepted: %d of 20000, sources generated: %d\n", accepted, sourced);
  EXPECT(accepted > 5000, "too few random programs accepted (%d) to exercise the generator", accepted);
}

static void source_generator() {
  // GELU-like chain with a logistic division, over f32 and 16-bit operands at many layouts
  std::vector<ihip_ew_instr> code = {
      ins(IHIP_EW_LOAD, 0, 0),          ins(IHIP_EW_LOAD, 1, 1),      ins(IHIP_EW_ADD, 1, 0, 1),
      ins(IHIP_EW_MUL, 2, 1, 1),        ins(IHIP_EW_IMM, 3, 0, 0, 0, 0.044715f), ins(IHIP_EW_MUL, 3, 2, 3),
      ins(IHIP_EW_MUL, 3, 3, 1),        ins(IHIP_EW_ADD, 3, 1, 3),    ins(IHIP_EW_IMM, 2, 0, 0, 0, -1.5957691f),
      ins(IHIP_EW_MUL, 2, 3, 2),        ins(IHIP_EW_EXP, 2, 2),       ins(IHIP_EW_IMM, 3, 0, 0, 0, 1.0f),
      ins(IHIP_EW_ADD, 3, 2, 3),        ins(IHIP_EW_DIV, 3, 1, 3),    ins(IHIP_EW_ADD, 0, 3, 0),
      ins(IHIP_EW_STORE, 0, 0),
  };
  int generated = 0, fused = 0;
  const int dts[3] = {IHIP_DT_F32, IHIP_DT_F16, IHIP_DT_BF16};
  for (int d = 0; d < 3; ++d)
    for (uintptr_t mis : {(uintptr_t)0, (uintptr_t)2, (uintptr_t)4, (uintptr_t)8})
      for (int layout = 0; layout < 3; ++layout) {
        const int64_t M = 37 + layout, N = 64 + 3 * layout;
        const int64_t shape[2] = {M, N};
        ihip_ew_operand in[2] = {layout == 2 ? opnd(4096 + mis, dts[d], 0, 0, 1, M) : opnd(4096 + mis, dts[d], 0, 0, N, 1),
                                 opnd(1 << 20, dts[d], 0, 0, 0, layout == 1 ? 0 : 1)};
        ihip_ew_operand out[1] = {opnd((1 << 21) + mis, dts[d], 0, 0, 0, 0)};
        int64_t len = -1;
        EXPECT(ihip_elementwise_source(code.data(), (int)code.size(), in, 2, out, 1, shape, 2, nullptr, 0, &len) ==
                   IHIP_OK, "source length");
        std::vector<char> buf((size_t)len + 1, 'x');
        EXPECT(ihip_elementwise_source(code.data(), (int)code.size(), in, 2, out, 1, shape, 2, buf.data(), len + 1,
                                       nullptr) == IHIP_OK, "source text");
        EXPECT(strlen(buf.data()) == (size_t)len, "source NUL-terminated at its length");
        char small[17];
        EXPECT(ihip_elementwise_source(code.data(), (int)code.size(), in, 2, out, 1, shape, 2, small, 17, nullptr) ==
                   IHIP_OK && strlen(small) == 16, "source truncated");
        generated += len > 0;
        fused += strstr(buf.data(), "ew_logistic_div_fast(r[") != nullptr;
      }
  EXPECT(generated == 36 && fused == 36, "generated %d, fused %d of 36", generated, fused);
  const int in_dt[2] = {IHIP_DT_BF16, IHIP_DT_BF16}, out_dt[1] = {IHIP_DT_BF16};
  EXPECT(ihip_elementwise_prepare(code.data(), (int)code.size(), in_dt, 2, out_dt, 1) == IHIP_OK, "hiprtc compile");
  const int prev = ihip_elementwise_mode(-1);
  EXPECT(ihip_elementwise_mode(7) == -1 && ihip_elementwise_mode(-1) == prev, "mode");
}

int main() {
  row_kernels();
  program_checker();
  source_generator();
  if (g_fail) {
    fprintf(stderr, "%d checks failed\n", g_fail);
    return 1;
  }
  printf("ALL OK\n");
  return 0;
}
