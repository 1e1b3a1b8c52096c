// Shared device helpers for the IntentIR gfx950 kernels.
//
// Everything here is written for CDNA4 wave64: reductions are 6 xor-shuffle
// steps over 64 lanes, vectors are 16-byte (dwordx4) accesses, and 16-bit
// floats are carried as raw bit patterns so the kernels control rounding.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ihip {

constexpr int kWave = 64;

// Number of XCDs on MI355X.  Workgroups are dispatched round-robin over them,
// and each XCD has a private L2, so tile schedules group work by XCD.
constexpr int kNumXcd = 8;

// 16-byte vectors as clang extended vectors, so they can go through the
// nontemporal builtins (streaming accesses that should not linger in cache).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- 16-bit floats
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// float32 -> bf16 bits, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Two float32 -> one word of two bf16 (lo in bits 0-15), round to nearest even, with
// gfx950's v_cvt_pk_bf16_f32 (NaN stays NaN).
__device__ __forceinline__ uint32_t pack_bf16x2_rne(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// float32 -> f16 bits with the hardware conversion (round to nearest even).
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// ---------------------------------------------------------------- exp
// e^d for d <= 0 or NaN (softmax arguments x - max).  t = d*log2(e) is carried as
// a head RN(d*L) and a tail (its exact rounding error plus d*(log2 e - L)); the
// head goes through the hardware 2^x and the tail through a first-order
// correction, |tail| <= 2^-24 |t|.  Relative error about 2 ulp for d >= -87;
// below that the result is under 1e-38.  d is first clamped to -160 (e^-160 is 0 in
// f32): without the clamp d = -inf (a masked logit) gives t = -inf and a NaN tail
// (-inf + inf), and 0 * NaN would make the result NaN instead of 0.  The clamp is
// NaN-propagating, so NaN still maps to NaN.
__device__ __forceinline__ float exp_nonpos(float d) {
  constexpr float kL = 1.44269502f;        // RN(log2 e)
  constexpr float kLlo = 1.92596303e-08f;  // log2 e - kL
  constexpr float kLn2 = 0.693147182f;
  d = __builtin_elementwise_maximum(d, -160.0f);
  const float t = d * kL;
  const float tail = __builtin_fmaf(d, kLlo, __builtin_fmaf(d, kL, -t));
  const float e = __builtin_amdgcn_exp2f(t);
  return __builtin_fmaf(e, tail * kLn2, e);
}

// ---------------------------------------------------------------- reductions
// max with numpy semantics: a NaN operand wins (np.maximum propagates NaN).
// gfx950 has an IEEE 754-2019 maximum (v_maximum3_f32): NaN in, NaN out.
__device__ __forceinline__ float max_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max_nan(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = max_nan(v, __shfl_xor(v, off, kWave));
  return v;
}

__device__ __forceinline__ uint32_t wave_or(uint32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v |= __shfl_xor(v, off, kWave);
  return v;
}

// Block-wide reductions across the waves of a workgroup (LDS scratch of
// blockDim.x/64 floats supplied by the caller; result broadcast to all threads).
__device__ __forceinline__ float block_sum(float v, float* scratch) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) scratch[w] = v;
  __syncthreads();
  float r = 0.f;
  for (int i = 0; i < nw; ++i) r += scratch[i];
  return r;
}

__device__ __forceinline__ float block_max_nan(float v, float* scratch) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = wave_max_nan(v);
  __syncthreads();
  if (lane == 0) scratch[w] = v;
  __syncthreads();
  float r = scratch[0];
  for (int i = 1; i < nw; ++i) r = max_nan(r, scratch[i]);
  return r;
}

// Workgroup b of a G-workgroup launch runs on XCD b % 8 (workgroups are dispatched to the XCDs
// round robin).  Its position in an order where every XCD holds one contiguous run (G / 8
// workgroups, one more on the first G % 8 XCDs), so that the tiles an XCD runs together are
// neighbours in the tile order and share that XCD's L2.  A bijection on [0, G).
__device__ __forceinline__ int xcd_contiguous(int b, int G) {
  const int x = b % kNumXcd, q = G / kNumXcd, r = G % kNumXcd;
  return x * q + (x < r ? x : r) + b / kNumXcd;
}

// Optional per-row outputs of a softmax: the row maximum and the sum of exp(x - max) over
// the row (the statistics the kernels compute anyway); a null pointer is not written.
struct SoftmaxStats {
  float* max;
  float* sum;
};

__device__ __forceinline__ void put_softmax_stats(const SoftmaxStats& st, int64_t row, float mx, float sum) {
  if (st.max != nullptr) st.max[row] = mx;
  if (st.sum != nullptr) st.sum[row] = sum;
}

// Row split of a long-row softmax (rows.hip): S segments per row of 256 * vpl 16-byte
// vectors, two floats of workspace per segment; S = 0 when rows are not split.
struct SoftmaxSplit {
  int S;
  int vpl;
};
SoftmaxSplit softmax_split_plan(int64_t M, int64_t N);

}  // namespace ihip
