// LayerNorm forward in float32 over the last axis: x, y f32 [M, N]; w, b f32 [N]; mean, rstd
// f32 [M] (null: not written).  The op order of the reference LayerNorm IR
// (pipeline/tilelang/core.py:1322-1384, pipeline/cuda/core.py:496-546) and of its CUDA
// kernel (backends/cuda/runtime/kernels/layernorm.cuh:11-98):
//   mean = sum(x) / N;  d = x - mean;  var = sum(d * d) / N;  rstd = 1 / sqrt(var + eps);
//   y = ((d * rstd) * w) + b
// with every step a separately rounded f32 operation (no fused multiply-adds: the kernels
// below are compiled with contraction off), so y differs from numpy's only through the order
// in which the two row sums are accumulated.
//
// Three forms, all reading x from HBM once where the row fits in registers:
//  * N % 4 == 0, N <= 4096, 16-byte aligned tensors: a wave per row, the row held in
//    registers (kVpl 16-byte vectors per lane), 4 rows per 256-thread workgroup with w and b
//    staged in LDS once per workgroup (instead of once per row from L2);
//  * N % 4 == 0, 4096 < N <= 65536, aligned: kW waves per row (the row in registers across
//    them), the wave sums exchanged through LDS and folded in a fixed order, w and b from L2;
//  * any other shape (odd N, unaligned views, N > 65536): a 256-thread workgroup per row that
//    reads x three times (the second and third reads of a row come from L2).
#include "common.hpp"

namespace ihip {

#pragma clang fp contract(off)

// Rows (waves) per workgroup of the one-wave-per-row form: 4 ran [8192, 4096] 2% ahead of 16
// (45.7 against 46.8 us, graph replays, rotated buffers) and of 2 or 8.
constexpr int kLn32Rows = 4;

template <int kVpl>
__global__ __launch_bounds__(64 * kLn32Rows) void layernorm_rows_f32_wave(
    const f32x4* __restrict__ x, const f32x4* __restrict__ w, const f32x4* __restrict__ b, f32x4* __restrict__ y,
    float* __restrict__ mean_out, float* __restrict__ rstd_out, int64_t M, int n4, int N, float eps) {
  __shared__ f32x4 w_lds[kVpl * kWave], b_lds[kVpl * kWave];
  const int lane = threadIdx.x & 63;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kLn32Rows + (threadIdx.x >> 6);
  const bool live = row0 < M;  // waves past the last row read row M - 1 and store nothing
  const int64_t row = live ? row0 : M - 1;
  const f32x4* xr = x + row * n4 + lane;
  f32x4 xv[kVpl];
#pragma unroll
  for (int i = 0; i < kVpl; ++i)
    xv[i] = lane + i * kWave < n4 ? __builtin_nontemporal_load(xr + i * kWave) : f32x4{0.f, 0.f, 0.f, 0.f};
  for (int t = threadIdx.x; t < n4; t += 64 * kLn32Rows) {  // staged after the row loads are issued
    w_lds[t] = w[t];
    b_lds[t] = b[t];
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kVpl; ++i) s += (xv[i][0] + xv[i][1]) + (xv[i][2] + xv[i][3]);  // padding holds +0
  const float mean = wave_sum(s) / static_cast<float>(N);
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < kVpl; ++i) {
    const bool in = lane + i * kWave < n4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float d = xv[i][j] - mean;
      q += in ? d * d : 0.f;
    }
  }
  const float rstd = 1.0f / sqrtf(wave_sum(q) / static_cast<float>(N) + eps);
  __syncthreads();  // w and b staged
  f32x4* yr = y + row * n4;
#pragma unroll
  for (int i = 0; i < kVpl; ++i) {
    const int idx = lane + i * kWave;  // lanes past n4 read LDS entries never staged and store nothing
    const f32x4 wv = w_lds[idx], bv = b_lds[idx];
    f32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = ((xv[i][j] - mean) * rstd) * wv[j] + bv[j];
    if (live && idx < n4) __builtin_nontemporal_store(o, yr + idx);
  }
  if (live && lane == 0) {
    if (mean_out != nullptr) mean_out[row] = mean;
    if (rstd_out != nullptr) rstd_out[row] = rstd;
  }
}

// kW waves per row, one row per workgroup: wave v holds the vectors (v * 64 + lane) + i * 64 * kW.
template <int kVpl, int kW>
__global__ __launch_bounds__(64 * kW) void layernorm_rows_f32_multi(
    const f32x4* __restrict__ x, const f32x4* __restrict__ w, const f32x4* __restrict__ b, f32x4* __restrict__ y,
    float* __restrict__ mean_out, float* __restrict__ rstd_out, int n4, int N, float eps) {
  __shared__ float part_s[kW], part_q[kW];
  const int lane = threadIdx.x & 63, v = threadIdx.x >> 6;
  const int64_t row = blockIdx.x;
  const int base = v * kWave + lane;
  const f32x4* xr = x + row * n4 + base;
  f32x4 xv[kVpl];
#pragma unroll
  for (int i = 0; i < kVpl; ++i)
    xv[i] = base + i * kWave * kW < n4 ? __builtin_nontemporal_load(xr + i * kWave * kW) : f32x4{0.f, 0.f, 0.f, 0.f};
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kVpl; ++i) s += (xv[i][0] + xv[i][1]) + (xv[i][2] + xv[i][3]);
  s = wave_sum(s);
  if (lane == 0) part_s[v] = s;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < kW; ++k) tot += part_s[k];
  const float mean = tot / static_cast<float>(N);
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < kVpl; ++i) {
    const bool in = base + i * kWave * kW < n4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float d = xv[i][j] - mean;
      q += in ? d * d : 0.f;
    }
  }
  q = wave_sum(q);
  if (lane == 0) part_q[v] = q;
  __syncthreads();
  float qt = 0.f;
#pragma unroll
  for (int k = 0; k < kW; ++k) qt += part_q[k];
  const float rstd = 1.0f / sqrtf(qt / static_cast<float>(N) + eps);
  f32x4* yr = y + row * n4;
#pragma unroll
  for (int i = 0; i < kVpl; ++i) {
    const int idx = base + i * kWave * kW;
    if (idx < n4) {
      const f32x4 wv = w[idx], bv = b[idx];
      f32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = ((xv[i][j] - mean) * rstd) * wv[j] + bv[j];
      __builtin_nontemporal_store(o, yr + idx);
    }
  }
  if (v == 0 && lane == 0) {
    if (mean_out != nullptr) mean_out[row] = mean;
    if (rstd_out != nullptr) rstd_out[row] = rstd;
  }
}

// Any N and alignment: one row per 256-thread workgroup, element-wise, three passes over x.
constexpr int kLn32AnyThreads = 256;

__global__ __launch_bounds__(kLn32AnyThreads) void layernorm_rows_f32_any(
    const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ b, float* __restrict__ y,
    float* __restrict__ mean_out, float* __restrict__ rstd_out, int64_t N, float eps) {
  __shared__ float scratch[kLn32AnyThreads / kWave];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const float* xr = x + row * N;
  float* yr = y + row * N;
  float s = 0.f;
  for (int64_t i = tid; i < N; i += kLn32AnyThreads) s += xr[i];
  const float mean = block_sum(s, scratch) / static_cast<float>(N);
  float q = 0.f;
  for (int64_t i = tid; i < N; i += kLn32AnyThreads) {
    const float d = xr[i] - mean;
    q += d * d;
  }
  const float rstd = 1.0f / sqrtf(block_sum(q, scratch) / static_cast<float>(N) + eps);
  for (int64_t i = tid; i < N; i += kLn32AnyThreads) yr[i] = ((xr[i] - mean) * rstd) * w[i] + b[i];
  if (tid == 0) {
    if (mean_out != nullptr) mean_out[row] = mean;
    if (rstd_out != nullptr) rstd_out[row] = rstd;
  }
}

template <int kVpl>
static void launch_ln32_wave(const f32x4* x4, const f32x4* w4, const f32x4* b4, f32x4* y4, float* mean, float* rstd,
                             int64_t M, int n4, int N, float eps, hipStream_t s) {
  const int64_t blocks = (M + kLn32Rows - 1) / kLn32Rows;
  layernorm_rows_f32_wave<kVpl><<<dim3(static_cast<unsigned>(blocks)), dim3(64 * kLn32Rows), 0, s>>>(
      x4, w4, b4, y4, mean, rstd, M, n4, N, eps);
}

template <int kW>
static void launch_ln32_multi(const f32x4* x4, const f32x4* w4, const f32x4* b4, f32x4* y4, float* mean, float* rstd,
                              int64_t M, int n4, int N, float eps, hipStream_t s) {
  layernorm_rows_f32_multi<16, kW><<<dim3(static_cast<unsigned>(M)), dim3(64 * kW), 0, s>>>(x4, w4, b4, y4, mean,
                                                                                             rstd, n4, N, eps);
}

// True when every tensor is 16-byte aligned and rows are whole 16-byte vectors.
static bool ln32_vector_form(const void* x, const void* w, const void* b, const void* y, int64_t N) {
  const auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  return N % 4 == 0 && al(x) && al(w) && al(b) && al(y);
}

hipError_t launch_layernorm_rows_f32(const float* x, const float* w, const float* b, float* y, float* mean,
                                     float* rstd, int64_t M, int64_t N, float eps, hipStream_t s) {
  if (M == 0) return hipSuccess;
  if (M > 0x7fffffffLL) return hipErrorInvalidValue;
  if (N == 0) {  // mean of an empty row: 0 / 0 (NaN), as numpy's sum / N; y is empty
    layernorm_rows_f32_any<<<dim3(static_cast<unsigned>(M)), dim3(kLn32AnyThreads), 0, s>>>(x, w, b, y, mean, rstd,
                                                                                            N, eps);
    return hipGetLastError();
  }
  if (ln32_vector_form(x, w, b, y, N) && N <= 65536) {
    const auto* x4 = reinterpret_cast<const f32x4*>(x);
    const auto* w4 = reinterpret_cast<const f32x4*>(w);
    const auto* b4 = reinterpret_cast<const f32x4*>(b);
    auto* y4 = reinterpret_cast<f32x4*>(y);
    const int n4 = static_cast<int>(N / 4), Ni = static_cast<int>(N);
    if (n4 <= 64) launch_ln32_wave<1>(x4, w4, b4, y4, mean, rstd, M, n4, Ni, eps, s);
    else if (n4 <= 128) launch_ln32_wave<2>(x4, w4, b4, y4, mean, rstd, M, n4, Ni, eps, s);
    else if (n4 <= 256) launch_ln32_wave<4>(x4, w4, b4, y4, mean, rstd, M, n4, Ni, eps, s);
    else if (n4 <= 512) launch_ln32_wave<8>(x4, w4, b4, y4, mean, rstd, M, n4, Ni, eps, s);
    else if (n4 <= 1024) launch_ln32_wave<16>(x4, w4, b4, y4, mean, rstd, M, n4, Ni, eps, s);
    else if (n4 <= 2048) launch_ln32_multi<2>(x4, w4, b4, y4, mean, rstd, M, n4, Ni, eps, s);
    else if (n4 <= 4096) launch_ln32_multi<4>(x4, w4, b4, y4, mean, rstd, M, n4, Ni, eps, s);
    else if (n4 <= 8192) launch_ln32_multi<8>(x4, w4, b4, y4, mean, rstd, M, n4, Ni, eps, s);
    else launch_ln32_multi<16>(x4, w4, b4, y4, mean, rstd, M, n4, Ni, eps, s);
    return hipGetLastError();
  }
  layernorm_rows_f32_any<<<dim3(static_cast<unsigned>(M)), dim3(kLn32AnyThreads), 0, s>>>(x, w, b, y, mean, rstd, N,
                                                                                          eps);
  return hipGetLastError();
}

}  // namespace ihip
