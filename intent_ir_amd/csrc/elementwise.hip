// Fused element-wise chain: y = alpha * gelu_tanh(x + bias[col]) + x  (bf16 in/out, f32 math)
//
// One kernel, no intermediate tensor: every element is read once and written once.
// Schedule: a thread owns one 16-byte column vector (8 bf16) and walks kRows rows,
// so the bias vector is loaded once per thread and all kRows loads are in flight
// together; a wave covers 1 KiB of contiguous row per load instruction.
//
// Arithmetic: gelu_tanh(z) = z / (1 + exp(-2*sqrt(2/pi)*(z + 0.044715*z^3))).  The
// kernel evaluates the same expression with the exponential as 2^t on the hardware exp2,
// t = z * (k + k*0.044715 * z^2) with k = -2*sqrt(2/pi)*log2(e), and folds alpha into the
// reciprocal: alpha * z / (1 + e) = z * rcp(e/alpha + 1/alpha), one FMA before the rcp and
// one after it (y = z * r + x).  Outputs are packed two at a time by the hardware
// round-to-nearest-even conversion (v_cvt_pk_bf16_f32).  That is ~7.5 VALU instructions
// per element plus the two transcendentals, against ~16 for the op-by-op form with a
// software bf16 rounding; at 8 TB/s the op-by-op form would be VALU-bound.  Error: a few
// float32 ulps of the op-by-op reference, three orders of magnitude below the bf16 output
// rounding.  alpha = 0 or 1/alpha not finite (no reciprocal to fold) takes the unfolded
// form z * rcp(1 + e) * alpha + x.
#include "common.hpp"

namespace ihip {

// -2*sqrt(2/pi) * log2(e): the exponent of the logistic form in base 2, and its cubic term.
constexpr float kGeluExp2Scale = -2.3022082f;
constexpr float kGeluExp2Cubic = -2.3022082f * 0.044715f;
constexpr float kGeluCubic = 0.044715f;

// t = z * (k + c z^2): the base-2 exponent of the logistic form.
__device__ __forceinline__ float gelu_exp2_arg(float z) {
  return z * __builtin_fmaf(kGeluExp2Cubic, z * z, kGeluExp2Scale);
}

// alpha * gelu_tanh(x + b) + x with ia = 1 / alpha folded into the reciprocal.
__device__ __forceinline__ float gelu_axpy_folded(float xv, float bv, float ia) {
  const float z = xv + bv;
  const float e = __builtin_amdgcn_exp2f(gelu_exp2_arg(z));
  return __builtin_fmaf(z, __builtin_amdgcn_rcpf(__builtin_fmaf(e, ia, ia)), xv);
}

// The unfolded form, for any alpha (0, or one whose reciprocal overflows).
__device__ __forceinline__ float gelu_axpy(float xv, float bv, float alpha) {
  const float z = xv + bv;
  const float p = __builtin_fmaf(kGeluCubic, z * z, 1.0f);
  const float e = __builtin_amdgcn_exp2f((z * p) * kGeluExp2Scale);
  const float g = z * __builtin_amdgcn_rcpf(1.0f + e);
  return __builtin_fmaf(g, alpha, xv);
}

template <bool kFolded>
__device__ __forceinline__ uint32_t bf16x2_apply(uint32_t xw, float b0, float b1, float a) {
  const float x0 = __uint_as_float(xw << 16), x1 = __uint_as_float(xw & 0xffff0000u);
  const float y0 = kFolded ? gelu_axpy_folded(x0, b0, a) : gelu_axpy(x0, b0, a);
  const float y1 = kFolded ? gelu_axpy_folded(x1, b1, a) : gelu_axpy(x1, b1, a);
  return pack_bf16x2_rne(y0, y1);
}

// a: 1/alpha when kFolded, else alpha.  lanes: threads per row of the workgroup (256, or for rows
// of fewer than 256 vectors n8 rounded up to a power of two, so that 256 / lanes rows share the
// workgroup instead of leaving most threads idle: N = 64 ran at 17% of HBM peak); thread t takes
// column t % lanes of rows (t / lanes) + r * (256 / lanes), r < kRows, of its row block.
// kExact: the grid tiles the tensor exactly (one row block per grid row, every column and row in
// range), so the rows need no guards and their addresses are one per-lane offset from a uniform
// base and stride (0.6% faster at [32768, 8192] than 64-bit addresses per row).
template <int kRows, bool kFolded, bool kExact>
__global__ __launch_bounds__(256) void bias_gelu_axpy_bf16_vec(const u32x4* __restrict__ x, const u32x4* __restrict__ bias,
                                                               u32x4* __restrict__ y, int64_t M, int64_t n8, float a,
                                                               int lanes) {
  const int64_t col = static_cast<int64_t>(blockIdx.x) * lanes + (threadIdx.x & (lanes - 1));
  const int64_t sub = threadIdx.x / lanes, per = 256 / lanes;  // row within a group of per rows
  if (!kExact && col >= n8) return;
  const u32x4 bw = bias[col];
  float bf[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    bf[2 * j] = __uint_as_float(bw[j] << 16);
    bf[2 * j + 1] = __uint_as_float(bw[j] & 0xffff0000u);
  }
  if constexpr (kExact) {
    const int64_t row0 = static_cast<int64_t>(blockIdx.y) * kRows * per;
    const u32x4* const xb = x + row0 * n8;
    u32x4* const yb = y + row0 * n8;
    const uint32_t off = static_cast<uint32_t>(sub * n8 + col);  // vectors; the launcher checks the range
    const int64_t rs = per * n8;
    u32x4 v[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) v[r] = __builtin_nontemporal_load(xb + r * rs + off);
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = bf16x2_apply<kFolded>(v[r][j], bf[2 * j], bf[2 * j + 1], a);
      __builtin_nontemporal_store(o, yb + r * rs + off);
    }
    return;
  }
  for (int64_t row0 = static_cast<int64_t>(blockIdx.y) * kRows * per + sub; row0 < M;
       row0 += static_cast<int64_t>(gridDim.y) * kRows * per) {
    u32x4 v[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const int64_t row = row0 + r * per;
      if (row < M) v[r] = __builtin_nontemporal_load(x + row * n8 + col);
    }
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const int64_t row = row0 + r * per;
      if (row < M) {
        u32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = bf16x2_apply<kFolded>(v[r][j], bf[2 * j], bf[2 * j + 1], a);
        __builtin_nontemporal_store(o, y + row * n8 + col);
      }
    }
  }
}

__global__ __launch_bounds__(256) void bias_gelu_axpy_bf16_any(const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ bias,
                                                               uint16_t* __restrict__ y, int64_t total, int64_t N,
                                                               float alpha) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const float xv = bf16_to_f32(x[i]);
    y[i] = f32_to_bf16_rne(gelu_axpy(xv, bf16_to_f32(bias[i % N]), alpha));
  }
}

hipError_t launch_bias_gelu_axpy_bf16(const uint16_t* x, const uint16_t* bias, uint16_t* y, int64_t M, int64_t N,
                                      float alpha, hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(bias) | reinterpret_cast<uintptr_t>(y);
  if (N % 8 == 0 && (al & 15) == 0) {
    constexpr int kRows = 4;  // 4 rows per thread: 1.4% ahead of 8 at [32768, 8192] (2: 0.6% behind, 16: 9%)
    const int64_t n8 = N / 8;
    int lanes = 1;
    while (lanes < 256 && lanes < n8) lanes *= 2;
    const int64_t per = 256 / lanes;
    int64_t row_blocks = (M + kRows * per - 1) / (kRows * per);
    if (row_blocks > 65535) row_blocks = 65535;  // grid.y limit; the kernel strides over the rest
    const dim3 grid(static_cast<unsigned>((n8 + lanes - 1) / lanes), static_cast<unsigned>(row_blocks));
    const u32x4* x8 = reinterpret_cast<const u32x4*>(x);
    const u32x4* b8 = reinterpret_cast<const u32x4*>(bias);
    u32x4* y8 = reinterpret_cast<u32x4*>(y);
    const float ia = 1.0f / alpha;
    // exact tiling: every row block and column block full, one row block per grid row, and the
    // per-lane offset (rows of the group times n8, plus the column) below 2^32 vectors
    const bool exact = M % (kRows * per) == 0 && n8 % lanes == 0 && row_blocks * kRows * per == M &&
                       (per - 1) * n8 + n8 < (int64_t(1) << 32);
    if (alpha != 0.0f && __builtin_isfinite(ia) && __builtin_isfinite(alpha)) {
      if (exact)
        bias_gelu_axpy_bf16_vec<kRows, true, true><<<grid, dim3(256), 0, s>>>(x8, b8, y8, M, n8, ia, lanes);
      else
        bias_gelu_axpy_bf16_vec<kRows, true, false><<<grid, dim3(256), 0, s>>>(x8, b8, y8, M, n8, ia, lanes);
    } else {
      if (exact)
        bias_gelu_axpy_bf16_vec<kRows, false, true><<<grid, dim3(256), 0, s>>>(x8, b8, y8, M, n8, alpha, lanes);
      else
        bias_gelu_axpy_bf16_vec<kRows, false, false><<<grid, dim3(256), 0, s>>>(x8, b8, y8, M, n8, alpha, lanes);
    }
  } else {
    const int64_t total = M * N;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    bias_gelu_axpy_bf16_any<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s>>>(x, bias, y, total, N, alpha);
  }
  return hipGetLastError();
}

}  // namespace ihip
