// Row kernels over a row-major [M, N] matrix: reduce_any, reduce_sum/max,
// softmax (f32) and LayerNorm forward (f16 in/out, f32 statistics).
//
// Layout and schedule (gfx950, wave64):
//  * one wave owns one row (the row reductions spread few long rows over 16 waves);
//    workgroups hold 1 (streaming reductions), 4 (softmax) or 16 (LayerNorm) rows;
//  * lanes read the row with 16-byte loads, lane l taking vectors l, l+64, ...,
//    so every load instruction of a wave covers 1 KiB of contiguous HBM;
//  * rows that fit in registers are read from HBM exactly once; statistics are
//    reduced with 6 xor-shuffle steps, never through LDS;
//  * shapes the vector path cannot take (N not a multiple of the vector width,
//    misaligned base, rows too long for registers) go to a workgroup-per-row
//    kernel with scalar accesses.
#include "common.hpp"

namespace ihip {

// ============================================================== reduce_any
// out[m] = any(x[m, :] != c)   (numpy semantics: NaN != c is true, -0.0 != 0 is false)
// For c == 0 the test is on the bits: |x| has a non-zero bit pattern.
template <bool kZero, int kUnroll>
__global__ __launch_bounds__(256) void reduce_any_rows_f32_vec(const float* __restrict__ x, uint8_t* __restrict__ out,
                                                               int64_t M, int64_t N, float c) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= M) return;
  // head of up to 3 elements to the row's first 16-byte boundary, n4 aligned vectors, tail of
  // up to 3 elements (neither when rows start aligned)
  const float* rowp = x + row * N;
  const int64_t to_edge = (4 - ((reinterpret_cast<uintptr_t>(rowp) >> 2) & 3)) & 3;
  const int64_t head = to_edge < N ? to_edge : N;
  const int64_t n4 = (N - head) >> 2;
  const int64_t tail = N - head - 4 * n4;
  const f32x4* xr = reinterpret_cast<const f32x4*>(rowp + head);
  uint32_t acc = 0;
  if (lane < head) acc |= kZero ? (__float_as_uint(rowp[lane]) & 0x7fffffffu) : static_cast<uint32_t>(rowp[lane] != c);
  if (lane < tail) {
    const float t = rowp[head + 4 * n4 + lane];
    acc |= kZero ? (__float_as_uint(t) & 0x7fffffffu) : static_cast<uint32_t>(t != c);
  }
  for (int64_t base = lane; base < n4; base += kWave * kUnroll) {
    f32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + static_cast<int64_t>(u) * kWave;
      v[u] = (i < n4) ? __builtin_nontemporal_load(xr + i) : f32x4{c, c, c, c};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (kZero) {
        acc |= (__float_as_uint(v[u].x) | __float_as_uint(v[u].y) | __float_as_uint(v[u].z) |
                __float_as_uint(v[u].w)) & 0x7fffffffu;
      } else {
        acc |= static_cast<uint32_t>(v[u].x != c) | static_cast<uint32_t>(v[u].y != c) |
               static_cast<uint32_t>(v[u].z != c) | static_cast<uint32_t>(v[u].w != c);
      }
    }
  }
  acc = wave_or(acc);
  if (lane == 0) out[row] = acc != 0u;
}

__global__ __launch_bounds__(256) void reduce_any_rows_f32_scalar(const float* __restrict__ x, uint8_t* __restrict__ out,
                                                                  int64_t M, int64_t N, float c) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= M) return;
  const float* xr = x + row * N;
  uint32_t acc = 0;
  for (int64_t i = lane; i < N; i += kWave) acc |= static_cast<uint32_t>(xr[i] != c);
  acc = wave_or(acc);
  if (lane == 0) out[row] = acc != 0u;
}

// bool/u8 input: out[m] = any(x[m, :] != 0).  A wave per row ORs 16-byte words of the row's
// aligned body, 16 loads per lane in flight, as the f32 kernel; the head (bytes before the row's
// first 16-byte boundary) and the tail (after its last) are < 16 bytes each, one byte per lane
// on the first lanes, so any N and any base alignment take the vector form.
template <int kUnroll>
__global__ __launch_bounds__(64) void reduce_any_rows_u8_vec(const uint8_t* __restrict__ x, uint8_t* __restrict__ out,
                                                             int64_t M, int64_t N) {
  const int lane = threadIdx.x & 63;
  const int64_t row = blockIdx.x;
  if (row >= M) return;
  const uint8_t* rowp = x + row * N;
  const int64_t to_edge = (16 - (reinterpret_cast<uintptr_t>(rowp) & 15)) & 15;
  const int64_t head = to_edge < N ? to_edge : N;
  const int64_t n16 = (N - head) >> 4;
  const int64_t tail = N - head - 16 * n16;
  const u32x4* xr = reinterpret_cast<const u32x4*>(rowp + head);
  uint32_t acc = 0;
  if (lane < head) acc |= rowp[lane];
  if (lane < tail) acc |= rowp[head + 16 * n16 + lane];
  for (int64_t base = lane; base < n16; base += kWave * kUnroll) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + static_cast<int64_t>(u) * kWave;
      v[u] = i < n16 ? __builtin_nontemporal_load(xr + i) : u32x4(0u);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc |= v[u].x | v[u].y | v[u].z | v[u].w;
  }
  acc = wave_or(acc);
  if (lane == 0) out[row] = acc != 0u;
}

// Short rows (at most 64 16-byte vectors): G lanes per row (G = 2 .. 32 for f32, 4 .. 32 for u8), 64 / G
// rows per wave, at most two vectors per lane loaded together, the row's head and tail elements (before its first
// 16-byte boundary and after its last) on the group's first lanes, and an OR over the group.
// kEsz: element bytes (4: f32 compared with c, or by its bits when kZero; 1: u8, any non-zero).
template <int G, int kEsz, bool kZero>
__global__ __launch_bounds__(256) void reduce_any_rows_grouped(const void* __restrict__ x, uint8_t* __restrict__ out,
                                                               int64_t M, int64_t N, float c) {
  constexpr int kPerVec = 16 / kEsz;
  const int lig = threadIdx.x & (G - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (256 / G) + threadIdx.x / G;
  auto test = [&](const char* p) -> uint32_t {
    if constexpr (kEsz == 1) {
      return *reinterpret_cast<const uint8_t*>(p);
    } else {
      const float v = *reinterpret_cast<const float*>(p);
      return kZero ? (__float_as_uint(v) & 0x7fffffffu) : static_cast<uint32_t>(v != c);
    }
  };
  uint32_t acc = 0;
  if (row < M) {  // no early return: the group's shuffles below need every lane
    const char* rowp = reinterpret_cast<const char*>(x) + row * N * kEsz;
    const int64_t to_edge = ((16 - (reinterpret_cast<uintptr_t>(rowp) & 15)) & 15) / kEsz;
    const int64_t head = to_edge < N ? to_edge : N;
    const int64_t nb = (N - head) / kPerVec;
    const int64_t tail = N - head - nb * kPerVec;
    for (int64_t t = lig; t < head; t += G) acc |= test(rowp + t * kEsz);
    for (int64_t t = lig; t < tail; t += G) acc |= test(rowp + (head + nb * kPerVec + t) * kEsz);
    const u32x4* body = reinterpret_cast<const u32x4*>(rowp + head * kEsz);
    // at most 2 vectors per lane (G >= nb / 2), both loads issued before either is used
    u32x4 q[2] = {u32x4(0u), u32x4(0u)};
    if (nb > 0) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int64_t v = lig + i * G;
        q[i] = __builtin_nontemporal_load(body + (v < nb ? v : nb - 1));
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (lig + i * G >= nb) continue;
      const u32x4 w = q[i];
      if constexpr (kEsz == 1) {
        acc |= w.x | w.y | w.z | w.w;
      } else if constexpr (kZero) {
        acc |= (w.x | w.y | w.z | w.w) & 0x7fffffffu;
      } else {
        acc |= static_cast<uint32_t>(__uint_as_float(w.x) != c) | static_cast<uint32_t>(__uint_as_float(w.y) != c) |
               static_cast<uint32_t>(__uint_as_float(w.z) != c) | static_cast<uint32_t>(__uint_as_float(w.w) != c);
      }
    }
  }
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) acc |= __shfl_xor(acc, off, kWave);
  if (row < M && lig == 0) out[row] = acc != 0u;
}

// Lanes per row for a row of `bytes` bytes in the grouped form: about two 16-byte vectors per
// lane, min_g .. 32; 0 when the row is long enough for a wave of its own (more than 64 vectors).
static int any_group_lanes(int64_t bytes, int min_g) {
  const int64_t nvec = bytes / 16;
  if (nvec > 64) return 0;
  int g = min_g;
  while (g < 32 && 2 * g < nvec) g *= 2;
  return g;
}

template <int kEsz, bool kZero>
static void launch_any_grouped(const void* x, uint8_t* out, int64_t M, int64_t N, float c, int g, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((M * g + 255) / 256)), block(256);
  switch (g) {
    case 2: reduce_any_rows_grouped<2, kEsz, kZero><<<grid, block, 0, s>>>(x, out, M, N, c); break;
    case 4: reduce_any_rows_grouped<4, kEsz, kZero><<<grid, block, 0, s>>>(x, out, M, N, c); break;
    case 8: reduce_any_rows_grouped<8, kEsz, kZero><<<grid, block, 0, s>>>(x, out, M, N, c); break;
    case 16: reduce_any_rows_grouped<16, kEsz, kZero><<<grid, block, 0, s>>>(x, out, M, N, c); break;
    default: reduce_any_rows_grouped<32, kEsz, kZero><<<grid, block, 0, s>>>(x, out, M, N, c); break;
  }
}

// Row kernels take the number of rows per workgroup from blockDim.x / 64.  Streaming kernels
// launch one-wave workgroups (measured 2-3% faster than four-wave ones on MI355X at 128 MiB).
constexpr int kStreamBlock = 64;

hipError_t launch_reduce_any_rows_f32(const float* x, uint8_t* out, int64_t M, int64_t N, float c, hipStream_t s) {
  if (M == 0) return hipSuccess;
  if (M > 0x7fffffffLL) return hipErrorInvalidValue;  // one workgroup per row
  const dim3 grid(static_cast<unsigned>(M)), block(kStreamBlock);
  // 16-byte loads over each row's aligned body whenever x is 4-byte aligned (any N)
  const bool vec = (reinterpret_cast<uintptr_t>(x) & 3) == 0;
  const int g = vec ? any_group_lanes(4 * N, 2) : 0;  // f32: a head and tail of at most 3 elements
  if (g > 0) {  // short rows: several per wave
    if (c == 0.0f)
      launch_any_grouped<4, true>(x, out, M, N, c, g, s);
    else
      launch_any_grouped<4, false>(x, out, M, N, c, g, s);
  } else if (!vec) {
    reduce_any_rows_f32_scalar<<<grid, block, 0, s>>>(x, out, M, N, c);
  } else if (c == 0.0f) {
    if (N / 4 >= kWave * 16)
      reduce_any_rows_f32_vec<true, 16><<<grid, block, 0, s>>>(x, out, M, N, c);
    else
      reduce_any_rows_f32_vec<true, 4><<<grid, block, 0, s>>>(x, out, M, N, c);
  } else {
    if (N / 4 >= kWave * 16)
      reduce_any_rows_f32_vec<false, 16><<<grid, block, 0, s>>>(x, out, M, N, c);
    else
      reduce_any_rows_f32_vec<false, 4><<<grid, block, 0, s>>>(x, out, M, N, c);
  }
  return hipGetLastError();
}

hipError_t launch_reduce_any_rows_u8(const uint8_t* x, uint8_t* out, int64_t M, int64_t N, hipStream_t s) {
  if (M == 0) return hipSuccess;
  if (M > 0x7fffffffLL) return hipErrorInvalidValue;  // one workgroup per row in the vector form
  const dim3 grid(static_cast<unsigned>(M)), block(kStreamBlock);
  const int g = any_group_lanes(N, 4);  // u8: a head and tail of up to 15 bytes over the group's lanes
  if (g > 0)  // short rows: several per wave
    launch_any_grouped<1, false>(x, out, M, N, 0.0f, g, s);
  else if (N / 16 >= kWave * 16)
    reduce_any_rows_u8_vec<16><<<grid, block, 0, s>>>(x, out, M, N);
  else
    reduce_any_rows_u8_vec<4><<<grid, block, 0, s>>>(x, out, M, N);
  return hipGetLastError();
}

// ============================================================== reduce_sum / reduce_max
// kind 0: out[m] = sum(x[m, :]) (f32 accumulation); kind 1: out[m] = max(x[m, :]) (NaN-propagating,
// as np.max).  Replaces the reference's row reductions (_kernel_reduce_sum/max over the last
// axis, backends/cuda/codegen/intentir_to_cuda.py:1553-1690).
//
// Vector form: W waves per row (one-wave workgroups for many rows, 16 waves when there are few
// rows to spread over the CUs).  Lane l of wave w takes 16-byte vectors (w*64 + l) + i*64*W
// with kUnroll non-temporal loads in flight, folded into kAcc f32x4 partials; the 4*kAcc
// partials are combined pairwise, then across the wave (6 xor-shuffles) and the row's waves
// (LDS).  Sums start from +0.0 as numpy's add.reduce does, so a row of -0.0 (and an empty
// row) sums to +0.0 as there; out-of-range elements contribute the start value.
template <int kKind>
__device__ __forceinline__ float red_op(float a, float b) {
  return kKind == 0 ? a + b : max_nan(a, b);
}

// kSplit: the row is split over S workgroups (segments); workgroup blockIdx.x takes segment
// blockIdx.x % S of row blockIdx.x / S, i.e. aligned vectors [seg*per, (seg+1)*per) of the
// row's body (segment 0 also the head, segment S-1 the tail), and writes its partial to
// part[row * S + seg] instead of out[row]; reduce_rows_combine then folds the S partials.
// scale multiplies the row's result as it is written (reduce_sum{scale}); split partials are
// written unscaled and reduce_rows_combine scales their fold.
template <int kKind, int W, int kUnroll, int kAcc, bool kSplit = false>
__global__ __launch_bounds__(64 * W) void reduce_rows_f32_vec(const float* __restrict__ x, float* __restrict__ out,
                                                              int64_t M, int64_t N, float scale, int S = 1,
                                                              float* __restrict__ part = nullptr) {
  static_assert(kUnroll % kAcc == 0 && (kAcc & (kAcc - 1)) == 0, "loads fold evenly into a power-of-two of partials");
  const float id = kKind == 0 ? 0.0f : -__builtin_inff();
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row = kSplit ? blockIdx.x / S : blockIdx.x;
  const int seg = kSplit ? static_cast<int>(blockIdx.x % S) : 0;
  if (row >= M) return;
  // The row splits into a head of up to 3 elements (to its first 16-byte boundary), n4
  // aligned vectors and a tail of up to 3 elements; rows that start aligned with N % 4 == 0
  // have neither head nor tail.
  const float* rowp = x + row * N;
  const int64_t to_edge = (4 - ((reinterpret_cast<uintptr_t>(rowp) >> 2) & 3)) & 3;
  const int64_t head = to_edge < N ? to_edge : N;
  const int64_t n4 = (N - head) >> 2;
  const int64_t tail = N - head - 4 * n4;
  const f32x4* xr = reinterpret_cast<const f32x4*>(rowp + head);
  // vectors [v0, v1) of the body: all of it, or this segment's share
  const int64_t per = kSplit ? (n4 + S - 1) / S : n4;
  const int64_t v0 = kSplit ? (seg * per < n4 ? seg * per : n4) : 0;
  const int64_t v1 = kSplit ? (v0 + per < n4 ? v0 + per : n4) : n4;
  f32x4 acc[kAcc];
#pragma unroll
  for (int u = 0; u < kAcc; ++u) acc[u] = f32x4{id, id, id, id};
  for (int64_t base = v0 + wave * kWave + lane; base < v1; base += static_cast<int64_t>(kWave) * W * kUnroll) {
    f32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + static_cast<int64_t>(u) * kWave * W;
      v[u] = (i < v1) ? __builtin_nontemporal_load(xr + i) : f32x4{id, id, id, id};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      f32x4& a = acc[u % kAcc];
      a.x = red_op<kKind>(a.x, v[u].x);
      a.y = red_op<kKind>(a.y, v[u].y);
      a.z = red_op<kKind>(a.z, v[u].z);
      a.w = red_op<kKind>(a.w, v[u].w);
    }
  }
#pragma unroll
  for (int h = kAcc / 2; h > 0; h /= 2)
#pragma unroll
    for (int u = 0; u < h; ++u) {
      acc[u].x = red_op<kKind>(acc[u].x, acc[u + h].x);
      acc[u].y = red_op<kKind>(acc[u].y, acc[u + h].y);
      acc[u].z = red_op<kKind>(acc[u].z, acc[u + h].z);
      acc[u].w = red_op<kKind>(acc[u].w, acc[u + h].w);
    }
  float r = red_op<kKind>(red_op<kKind>(acc[0].x, acc[0].y), red_op<kKind>(acc[0].z, acc[0].w));
  if (wave == 0) {  // head and tail elements (at most 3 each) join lanes 0..2 of the first wave
    if (lane < head && seg == 0) r = red_op<kKind>(r, rowp[lane]);
    if (lane < tail && seg == S - 1) r = red_op<kKind>(r, rowp[head + 4 * n4 + lane]);
  }
  r = kKind == 0 ? wave_sum(r) : wave_max_nan(r);
  float* dst = kSplit ? part + row * S + seg : out + row;
  const float f = kSplit ? 1.0f : scale;
  if (W > 1) {
    __shared__ float wpart[W];
    if (lane == 0) wpart[wave] = r;
    __syncthreads();
    if (threadIdx.x == 0) {
      float t = wpart[0];
#pragma unroll
      for (int i = 1; i < W; ++i) t = red_op<kKind>(t, wpart[i]);
      *dst = t * f;
    }
  } else if (lane == 0) {
    *dst = r * f;
  }
}

// out[row] = fold of the row's S <= 64 segment partials part[row*S ..], one wave per row, lane
// l holding partial l; the xor-shuffle tree fixes the order, so results are reproducible.
template <int kKind>
__global__ __launch_bounds__(256) void reduce_rows_combine(const float* __restrict__ part, float* __restrict__ out,
                                                           int64_t M, int S, float scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= M) return;
  float r = lane < S ? part[row * S + lane] : (kKind == 0 ? 0.0f : -__builtin_inff());
  r = kKind == 0 ? wave_sum(r) : wave_max_nan(r);
  if (lane == 0) out[row] = r * scale;
}

// Scalar form for rows the vector form cannot take (N % 4 != 0 or a base not 16-byte aligned).
template <int kKind>
__global__ __launch_bounds__(256) void reduce_rows_f32(const float* __restrict__ x, float* __restrict__ out, int64_t M,
                                                       int64_t N, float scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= M) return;
  const float* xr = x + row * N;
  float acc = kKind == 0 ? 0.0f : -__builtin_inff();
  for (int64_t i = lane; i < N; i += kWave) acc = red_op<kKind>(acc, xr[i]);
  acc = kKind == 0 ? wave_sum(acc) : wave_max_nan(acc);
  if (lane == 0) out[row] = acc * scale;
}

// Loads in flight per lane in the one-wave form (8 measured level with 16 on [8192, 4096]).
constexpr int kRedUnroll = 16;

// Row split for rows too few to fill the GPU: S segments per row (1 = no split), so that
// M * S workgroups of 16 waves give every CU about two, each segment at least
// kRedSegMinVec 16-byte vectors (64 KiB).  Depends on the shape only.
constexpr int kRedMaxSegments = 64;
constexpr int64_t kRedSplitRows = 256;      // rows below this may split (fewer rows than CUs)
constexpr int64_t kRedSplitTarget = 512;    // workgroups to aim for
constexpr int64_t kRedSegMinVec = 4096;
int reduce_rows_segments(int64_t M, int64_t N) {
  if (M <= 0 || M >= kRedSplitRows || N <= 0) return 1;
  const int64_t n4 = N / 4;
  int64_t S = (kRedSplitTarget + M - 1) / M;
  if (S > kRedMaxSegments) S = kRedMaxSegments;
  while (S > 1 && n4 / S < kRedSegMinVec) --S;
  return static_cast<int>(S);
}

// Short rows (at most 128 16-byte vectors): G lanes per row (G = 1 .. 32, about two vectors per
// lane, four at 65-128 vectors, loaded together: a loop with one load per trip ran N = 16-32 at
// 45% of HBM peak, against 69-71% now), 64 / G rows per wave, the row's head and tail elements on the
// group's first lanes, and
// the group's values combined with xor shuffles (a wave per row left most lanes idle: N = 32
// ran at 5% of HBM peak, 128 at 19%).  kKind 0: sum, 1: NaN-propagating max.
template <int kKind, int G, int kV>
__global__ __launch_bounds__(256) void reduce_rows_f32_grouped(const float* __restrict__ x, float* __restrict__ out,
                                                               int64_t M, int64_t N, float scale) {
  const int lig = threadIdx.x & (G - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (256 / G) + threadIdx.x / G;
  auto op = [](float a, float b) { return kKind == 0 ? a + b : max_nan(a, b); };
  float acc = kKind == 0 ? 0.f : -__builtin_inff();
  if (row < M) {  // no early return: the group's shuffles need every lane
    const float* rowp = x + row * N;
    const int64_t to_edge = (4 - ((reinterpret_cast<uintptr_t>(rowp) >> 2) & 3)) & 3;
    const int64_t head = to_edge < N ? to_edge : N;
    const int64_t nb = (N - head) >> 2;
    const int64_t tail = N - head - 4 * nb;
    for (int64_t t = lig; t < head; t += G) acc = op(acc, rowp[t]);
    for (int64_t t = lig; t < tail; t += G) acc = op(acc, rowp[head + 4 * nb + t]);
    const f32x4* body = reinterpret_cast<const f32x4*>(rowp + head);
    if (nb > 0) {  // at most kV vectors per lane, all loads issued before the first is used
      f32x4 q[kV];
#pragma unroll
      for (int i = 0; i < kV; ++i) {
        const int64_t v = lig + i * G;
        q[i] = __builtin_nontemporal_load(body + (v < nb ? v : nb - 1));
      }
#pragma unroll
      for (int i = 0; i < kV; ++i)
        if (lig + i * G < nb) acc = op(acc, op(op(q[i].x, q[i].y), op(q[i].z, q[i].w)));
    }
  }
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) acc = op(acc, __shfl_xor(acc, off, kWave));
  if (row < M && lig == 0) out[row] = acc * scale;
}

template <int kKind, int G>
static void launch_reduce_grouped_g(const float* x, float* out, int64_t M, int64_t N, float scale, int kv, dim3 grid,
                                    hipStream_t s) {
  if (kv <= 1)
    reduce_rows_f32_grouped<kKind, G, 1><<<grid, dim3(256), 0, s>>>(x, out, M, N, scale);
  else if (kv <= 2)
    reduce_rows_f32_grouped<kKind, G, 2><<<grid, dim3(256), 0, s>>>(x, out, M, N, scale);
  else
    reduce_rows_f32_grouped<kKind, G, 4><<<grid, dim3(256), 0, s>>>(x, out, M, N, scale);
}

template <int kKind>
static void launch_reduce_grouped(const float* x, float* out, int64_t M, int64_t N, float scale, hipStream_t s) {
  const int64_t nvec = N / 4;
  // about two vectors per lane (four at 65-128 vectors); one per lane measured 12-18% slower at
  // 16-32 vectors and, with the loads issued together, 14-16% slower at 4-8
  int g = 1;
  while (g < 32 && 2 * g < nvec) g *= 2;
  const int kv = static_cast<int>((nvec + g - 1) / g);  // body vectors per lane at most (<= 4)
  const dim3 grid(static_cast<unsigned>((M * g + 255) / 256));
  switch (g) {
    case 1: launch_reduce_grouped_g<kKind, 1>(x, out, M, N, scale, kv, grid, s); break;
    case 2: launch_reduce_grouped_g<kKind, 2>(x, out, M, N, scale, kv, grid, s); break;
    case 4: launch_reduce_grouped_g<kKind, 4>(x, out, M, N, scale, kv, grid, s); break;
    case 8: launch_reduce_grouped_g<kKind, 8>(x, out, M, N, scale, kv, grid, s); break;
    case 16: launch_reduce_grouped_g<kKind, 16>(x, out, M, N, scale, kv, grid, s); break;
    default: launch_reduce_grouped_g<kKind, 32>(x, out, M, N, scale, kv, grid, s); break;
  }
}

template <int kKind>
static void launch_reduce_rows(const float* x, float* out, int64_t M, int64_t N, float scale, float* part, int S,
                               hipStream_t s) {
  // 16-byte loads over each row's aligned body whenever x is 4-byte aligned (any N)
  if ((reinterpret_cast<uintptr_t>(x) & 3) != 0 || N == 0) {
    reduce_rows_f32<kKind><<<dim3(static_cast<unsigned>((M + 3) / 4)), dim3(256), 0, s>>>(x, out, M, N, scale);
    return;
  }
  const int64_t n4 = N / 4;
  const dim3 grid(static_cast<unsigned>(M));
  if (S > 1 && part != nullptr) {  // few long rows split over S workgroups each, then combined
    reduce_rows_f32_vec<kKind, 16, 8, 4, true><<<dim3(static_cast<unsigned>(M * S)), dim3(1024), 0, s>>>(
        x, out, M, N, scale, S, part);
    reduce_rows_combine<kKind><<<dim3(static_cast<unsigned>((M + 3) / 4)), dim3(256), 0, s>>>(part, out, M, S, scale);
  } else if (n4 <= 2 * kWave) {  // short rows: several per wave
    launch_reduce_grouped<kKind>(x, out, M, N, scale, s);
  } else if (M >= 2048 || n4 <= 4 * kWave) {  // enough rows for the CUs, or short rows: a wave per row
    reduce_rows_f32_vec<kKind, 1, kRedUnroll, 4><<<grid, dim3(64), 0, s>>>(x, out, M, N, scale);
  } else {  // few long rows: 16 waves per row
    reduce_rows_f32_vec<kKind, 16, 8, 4><<<grid, dim3(1024), 0, s>>>(x, out, M, N, scale);
  }
}

// part: workspace of M * reduce_rows_segments(M, N) floats, or null (no row split).
hipError_t launch_reduce_rows_f32(const float* x, float* out, int64_t M, int64_t N, int kind, float scale,
                                  float* part, hipStream_t s) {
  if (M == 0) return hipSuccess;
  if (M > 0x7fffffffLL) return hipErrorInvalidValue;  // one workgroup per row
  const int S = part != nullptr ? reduce_rows_segments(M, N) : 1;
  if (kind == 0)
    launch_reduce_rows<0>(x, out, M, N, scale, part, S, s);
  else
    launch_reduce_rows<1>(x, out, M, N, scale, part, S, s);
  return hipGetLastError();
}

// ============================================================== softmax (last axis, f32)
// y = exp(x - max) * (1 / sum(exp(x - max))).  The reference interpreter divides
// every element by the sum; multiplying by the row's correctly rounded
// reciprocal adds at most one rounding (|rel. diff| < 2.4e-7).  max propagates
// NaN (v_maximum3_f32), so a row holding a NaN comes out all NaN, as in numpy.
// About 14 VALU instructions per element, so the kernel stays HBM-bound.
// kVpl: f32x4 vectors held per lane; kFull: n4 == 64 * kVpl; kR: consecutive rows per wave
// (with rows of at most 1024 floats, two rows per wave ran [16384, 1024] 2.8% faster than a
// wave per row, and four such waves per workgroup 2.6% faster again than two).  The compiler
// issues the second row's loads after the first row's maximum; pinned ahead of it (all loads
// first) the kernel ran 2% slower.  The loads are unconditional: a wave whose second row
// is past the last re-reads the last row and stores nothing for it (loads under a row guard
// cost 4%).
// kWaves: waves per workgroup (a constant, so that the kernel reads no hidden argument before
// its first loads).
template <int kVpl, bool kFull, int kR, int kWaves>
__global__ __launch_bounds__(256) void softmax_rows_f32_reg(const f32x4* __restrict__ x, f32x4* __restrict__ y,
                                                            int64_t M, int n4, SoftmaxStats st) {
  const int lane = threadIdx.x & 63;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6)) * kR;
  if (row0 >= M) return;
  const float ninf = -__builtin_inff();
  f32x4 v[kR][kVpl];
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    const int64_t rr = kR == 1 ? row0 : (row0 + r < M ? row0 + r : M - 1);
    const f32x4* xr = x + rr * n4;
#pragma unroll
    for (int i = 0; i < kVpl; ++i) {
      const int idx = lane + i * kWave;
      v[r][i] = (kFull || idx < n4) ? __builtin_nontemporal_load(xr + idx) : f32x4{ninf, ninf, ninf, ninf};
    }
  }
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    f32x4* yr = y + (row0 + r) * n4;
    float mx = ninf;
#pragma unroll
    for (int i = 0; i < kVpl; ++i)
      mx = max_nan(max_nan(mx, v[r][i].x), max_nan(max_nan(v[r][i].y, v[r][i].z), v[r][i].w));
    mx = wave_max_nan(mx);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < kVpl; ++i) {
      v[r][i].x = exp_nonpos(v[r][i].x - mx);
      v[r][i].y = exp_nonpos(v[r][i].y - mx);
      v[r][i].z = exp_nonpos(v[r][i].z - mx);
      v[r][i].w = exp_nonpos(v[r][i].w - mx);
      if (kFull || lane + i * kWave < n4) sum += (v[r][i].x + v[r][i].y) + (v[r][i].z + v[r][i].w);
    }
    sum = wave_sum(sum);
    if (lane == 0 && (kR == 1 || row0 + r < M)) put_softmax_stats(st, row0 + r, mx, sum);
    const float inv = 1.0f / sum;
#pragma unroll
    for (int i = 0; i < kVpl; ++i) {
      const int idx = lane + i * kWave;
      if ((kFull || idx < n4) && (kR == 1 || row0 + r < M)) {
        f32x4 o;
        o.x = v[r][i].x * inv;
        o.y = v[r][i].y * inv;
        o.z = v[r][i].z * inv;
        o.w = v[r][i].w * inv;
        __builtin_nontemporal_store(o, yr + idx);
      }
    }
  }
}

// Rows longer than one wave holds (N > 4096): kW waves share a row, one row per workgroup.
// Wave v holds the vectors (v*64 + lane) + i*64*kW, i < kVpl, in registers, so the row is
// read from HBM once; the row max and sum are exchanged through LDS and every wave combines
// the kW partials in the same order.  Same arithmetic per element as the one-wave kernel.
template <int kVpl, int kW>
__global__ __launch_bounds__(64 * kW) void softmax_rows_f32_multi(const f32x4* __restrict__ x, f32x4* __restrict__ y,
                                                                  int64_t M, int n4, SoftmaxStats st) {
  __shared__ float part_m[kW], part_s[kW];
  const int lane = threadIdx.x & 63, v = threadIdx.x >> 6;
  const int64_t row = blockIdx.x;
  if (row >= M) return;  // uniform per workgroup
  const f32x4* xr = x + row * n4 + v * kWave + lane;
  f32x4* yr = y + row * n4 + v * kWave + lane;
  const float ninf = -__builtin_inff();
  f32x4 xv[kVpl];
#pragma unroll
  for (int i = 0; i < kVpl; ++i)
    xv[i] = v * kWave + lane + i * kWave * kW < n4 ? __builtin_nontemporal_load(xr + i * kWave * kW)
                                                   : f32x4{ninf, ninf, ninf, ninf};
  float mx = ninf;
#pragma unroll
  for (int i = 0; i < kVpl; ++i) mx = max_nan(max_nan(mx, xv[i].x), max_nan(max_nan(xv[i].y, xv[i].z), xv[i].w));
  mx = wave_max_nan(mx);
  if (lane == 0) part_m[v] = mx;
  __syncthreads();
  mx = part_m[0];
#pragma unroll
  for (int k = 1; k < kW; ++k) mx = max_nan(mx, part_m[k]);
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < kVpl; ++i) {
    xv[i].x = exp_nonpos(xv[i].x - mx);
    xv[i].y = exp_nonpos(xv[i].y - mx);
    xv[i].z = exp_nonpos(xv[i].z - mx);
    xv[i].w = exp_nonpos(xv[i].w - mx);
    if (v * kWave + lane + i * kWave * kW < n4) sum += (xv[i].x + xv[i].y) + (xv[i].z + xv[i].w);
  }
  sum = wave_sum(sum);
  if (lane == 0) part_s[v] = sum;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < kW; ++k) tot += part_s[k];
  if (threadIdx.x == 0) put_softmax_stats(st, row, mx, tot);
  const float inv = 1.0f / tot;
#pragma unroll
  for (int i = 0; i < kVpl; ++i)
    if (v * kWave + lane + i * kWave * kW < n4) __builtin_nontemporal_store(xv[i] * inv, yr + i * kWave * kW);
}

// Rows whose length is not a multiple of 4 (or a base not 16-byte aligned), up to 65536: the
// row is still held in registers and read once, with 4-byte loads.  Element (i*kW + v)*64 + lane
// belongs to lane `lane` of wave v, so each load instruction of a wave covers 256 contiguous
// bytes; kW waves per row, partials through LDS as in the vector multi-wave form.
template <int kEpl, int kW>
__global__ __launch_bounds__(64 * kW) void softmax_rows_f32_regs(const float* __restrict__ x, float* __restrict__ y,
                                                                 int64_t M, int64_t N, SoftmaxStats st) {
  __shared__ float part_m[kW], part_s[kW];
  const int lane = threadIdx.x & 63, v = threadIdx.x >> 6;
  const int64_t row = blockIdx.x;
  if (row >= M) return;  // uniform per workgroup
  const float* xr = x + row * N + v * kWave + lane;
  float* yr = y + row * N + v * kWave + lane;
  const int64_t left = N - (v * kWave + lane);  // elements of this lane: index i*kW*64 < left
  const float ninf = -__builtin_inff();
  float e[kEpl];
#pragma unroll
  for (int i = 0; i < kEpl; ++i) e[i] = i * kW * kWave < left ? __builtin_nontemporal_load(xr + i * kW * kWave) : ninf;
  float mx = ninf;
#pragma unroll
  for (int i = 0; i < kEpl; ++i) mx = max_nan(mx, e[i]);
  mx = wave_max_nan(mx);
  if (kW > 1) {
    if (lane == 0) part_m[v] = mx;
    __syncthreads();
    mx = part_m[0];
#pragma unroll
    for (int k = 1; k < kW; ++k) mx = max_nan(mx, part_m[k]);
  }
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < kEpl; ++i) {
    e[i] = exp_nonpos(e[i] - mx);
    if (i * kW * kWave < left) sum += e[i];
  }
  sum = wave_sum(sum);
  if (kW > 1) {
    if (lane == 0) part_s[v] = sum;
    __syncthreads();
    sum = 0.f;
#pragma unroll
    for (int k = 0; k < kW; ++k) sum += part_s[k];
  }
  if (threadIdx.x == 0) put_softmax_stats(st, row, mx, sum);
  const float inv = 1.0f / sum;
#pragma unroll
  for (int i = 0; i < kEpl; ++i)
    if (i * kW * kWave < left) __builtin_nontemporal_store(e[i] * inv, yr + i * kW * kWave);
}

// Rows whose starts are not all 16-byte aligned (N % 4 != 0), 1024 < N <= 4096*kW, with x and
// y sharing their alignment modulo 16 bytes: each row is split into a head of h < 4 elements
// (up to the first 16-byte boundary), a 16-byte aligned body of nb vectors held in registers
// exactly as in the multi-wave vector form, and a tail of t < 4 elements.  Thread j < h holds
// head element j, thread j < t tail element j.  Every access is bounded by the row: body
// vector k < nb covers elements h + 4k .. h + 4k + 3 < h + 4nb <= N.
template <int kVpl, int kW>
__global__ __launch_bounds__(64 * kW) void softmax_rows_f32_skew(const float* __restrict__ x, float* __restrict__ y,
                                                                 int64_t M, int64_t N, SoftmaxStats st) {
  __shared__ float part_m[kW], part_s[kW];
  const int lane = threadIdx.x & 63, v = threadIdx.x >> 6, tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  if (row >= M) return;  // uniform per workgroup
  const float* xr = x + row * N;
  float* yr = y + row * N;
  const int64_t to_edge = (4 - ((reinterpret_cast<uintptr_t>(xr) >> 2) & 3)) & 3;
  const int64_t head = to_edge < N ? to_edge : N;
  const int64_t nb = (N - head) >> 2;
  const int64_t tail = N - head - 4 * nb;
  const int64_t first = v * kWave + lane;  // this lane's first body vector
  const f32x4* xb = reinterpret_cast<const f32x4*>(xr + head) + first;
  f32x4* yb = reinterpret_cast<f32x4*>(yr + head) + first;
  const float ninf = -__builtin_inff();
  f32x4 xv[kVpl];
#pragma unroll
  for (int i = 0; i < kVpl; ++i)
    xv[i] = first + i * kWave * kW < nb ? __builtin_nontemporal_load(xb + i * kWave * kW)
                                        : f32x4{ninf, ninf, ninf, ninf};
  float hv = tid < head ? xr[tid] : ninf;
  float tv = tid < tail ? xr[head + 4 * nb + tid] : ninf;
  float mx = max_nan(hv, tv);
#pragma unroll
  for (int i = 0; i < kVpl; ++i) mx = max_nan(max_nan(mx, xv[i].x), max_nan(max_nan(xv[i].y, xv[i].z), xv[i].w));
  mx = wave_max_nan(mx);
  if (lane == 0) part_m[v] = mx;
  __syncthreads();
  mx = part_m[0];
#pragma unroll
  for (int k = 1; k < kW; ++k) mx = max_nan(mx, part_m[k]);
  hv = exp_nonpos(hv - mx);
  tv = exp_nonpos(tv - mx);
  float sum = (tid < head ? hv : 0.f) + (tid < tail ? tv : 0.f);
#pragma unroll
  for (int i = 0; i < kVpl; ++i) {
    xv[i].x = exp_nonpos(xv[i].x - mx);
    xv[i].y = exp_nonpos(xv[i].y - mx);
    xv[i].z = exp_nonpos(xv[i].z - mx);
    xv[i].w = exp_nonpos(xv[i].w - mx);
    if (first + i * kWave * kW < nb) sum += (xv[i].x + xv[i].y) + (xv[i].z + xv[i].w);
  }
  sum = wave_sum(sum);
  if (lane == 0) part_s[v] = sum;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < kW; ++k) tot += part_s[k];
  if (tid == 0) put_softmax_stats(st, row, mx, tot);
  const float inv = 1.0f / tot;
#pragma unroll
  for (int i = 0; i < kVpl; ++i)
    if (first + i * kWave * kW < nb) __builtin_nontemporal_store(xv[i] * inv, yb + i * kWave * kW);
  if (tid < head) yr[tid] = hv * inv;
  if (tid < tail) yr[head + 4 * nb + tid] = tv * inv;
}

// (m, s) <- the statistics of the union of two sets of elements: maxima m and m2, sums of
// exponentials s = sum(exp(x - m)) and s2 = sum(exp(x - m2)).  A set whose maximum is -inf
// (empty, or all of it masked) adds 0; a NaN maximum propagates.  Commutative, so a
// butterfly over a wave leaves every lane with the same pair.
__device__ __forceinline__ void softmax_fold(float& m, float& s, float m2, float s2) {
  const float ninf = -__builtin_inff();
  const float nm = max_nan(m, m2);
  s = (m == ninf ? 0.f : s * exp_nonpos(m - nm)) + (m2 == ninf ? 0.f : s2 * exp_nonpos(m2 - nm));
  m = nm;
}

// Folds every thread's (m, s) into the workgroup's, in a fixed order (xor butterfly within each
// wave, then the waves in order through LDS); every thread returns the same pair.
template <int kW>
__device__ __forceinline__ void block_softmax_fold(float& m, float& s, float* fm, float* fs) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) softmax_fold(m, s, __shfl_xor(m, off, kWave), __shfl_xor(s, off, kWave));
  const int lane = threadIdx.x & 63, v = threadIdx.x >> 6;
  if (lane == 0) fm[v] = m, fs[v] = s;
  __syncthreads();
  m = fm[0];
  s = fs[0];
#pragma unroll
  for (int k = 1; k < kW; ++k) softmax_fold(m, s, fm[k], fs[k]);
}

// Rows no other form holds (longer than 65536 floats without a workspace, or x and y at
// different offsets modulo 16 bytes): one 1024-thread workgroup per row, two passes over x.
// The first keeps a running maximum and sum of exponentials per thread (the sum rescaled by
// exp(old - new) when the maximum grows) and folds them over the workgroup; the second writes
// exp(x - max) * (1 / sum) with the register kernels' arithmetic.  kVec: x and y 4-byte
// aligned at the same offset modulo 16 bytes: a head and tail of < 4 elements on the first
// threads around 16-byte loads of the body; otherwise 4-byte loads throughout.
template <bool kVec>
__global__ __launch_bounds__(1024) void softmax_rows_f32_online(const float* __restrict__ x, float* __restrict__ y,
                                                                int64_t N, SoftmaxStats st) {
  constexpr int kW = 16, kT = 1024, kU = 4;
  __shared__ float fm[kW], fs[kW];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const float* xr = x + row * N;
  float* yr = y + row * N;
  const float ninf = -__builtin_inff();
  float m = ninf, s = 0.f;
  // adds four elements (-inf for none) to the thread's running pair
  auto add4 = [&](float a, float b, float c, float d) {
    const float nm = max_nan(m, max_nan(max_nan(a, b), max_nan(c, d)));
    if (nm != ninf) {
      s = (m == ninf ? 0.f : s * exp_nonpos(m - nm)) +
          ((exp_nonpos(a - nm) + exp_nonpos(b - nm)) + (exp_nonpos(c - nm) + exp_nonpos(d - nm)));
      m = nm;
    }
  };
  if constexpr (kVec) {
    const int64_t to_edge = (4 - ((reinterpret_cast<uintptr_t>(xr) >> 2) & 3)) & 3;
    const int64_t head = to_edge < N ? to_edge : N;
    const int64_t nb = (N - head) >> 2, tail = N - head - 4 * nb;
    const f32x4* xb = reinterpret_cast<const f32x4*>(xr + head);
    f32x4* yb = reinterpret_cast<f32x4*>(yr + head);
    for (int64_t i = tid; i < nb; i += kU * kT) {
      f32x4 q[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) q[u] = i + u * kT < nb ? xb[i + u * kT] : f32x4{ninf, ninf, ninf, ninf};
#pragma unroll
      for (int u = 0; u < kU; ++u) add4(q[u].x, q[u].y, q[u].z, q[u].w);
    }
    add4(tid < head ? xr[tid] : ninf, tid < tail ? xr[head + 4 * nb + tid] : ninf, ninf, ninf);
    block_softmax_fold<kW>(m, s, fm, fs);
    if (tid == 0) put_softmax_stats(st, row, m, s);
    const float inv = 1.0f / s;
    for (int64_t i = tid; i < nb; i += kU * kT) {
      f32x4 q[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u)
        if (i + u * kT < nb) q[u] = __builtin_nontemporal_load(xb + i + u * kT);
#pragma unroll
      for (int u = 0; u < kU; ++u)
        if (i + u * kT < nb) {
          const f32x4 e = {exp_nonpos(q[u].x - m), exp_nonpos(q[u].y - m), exp_nonpos(q[u].z - m),
                           exp_nonpos(q[u].w - m)};
          __builtin_nontemporal_store(e * inv, yb + i + u * kT);
        }
    }
    if (tid < head) yr[tid] = exp_nonpos(xr[tid] - m) * inv;
    if (tid < tail) yr[head + 4 * nb + tid] = exp_nonpos(xr[head + 4 * nb + tid] - m) * inv;
  } else {
    for (int64_t i = tid; i < N; i += 4 * kT)
      add4(xr[i], i + kT < N ? xr[i + kT] : ninf, i + 2 * kT < N ? xr[i + 2 * kT] : ninf,
           i + 3 * kT < N ? xr[i + 3 * kT] : ninf);
    block_softmax_fold<kW>(m, s, fm, fs);
    if (tid == 0) put_softmax_stats(st, row, m, s);
    const float inv = 1.0f / s;
    for (int64_t i = tid; i < N; i += kT) yr[i] = exp_nonpos(xr[i] - m) * inv;
  }
}

// Rows of 65536 < N <= 4 * kResMaxVecs floats (N % 4 == 0, x and y 16-byte aligned; vocabulary-
// width rows): one 1024-thread workgroup per row, and the whole row held on the CU, so x is read
// from HBM once where the two-pass kernel above reads it twice.  The first kResVpl * 1024
// 16-byte vectors sit in registers (vector t + i * 1024 in thread t; 96 VGPRs); the rest, up to
// kResLdsVecs vectors, is copied straight into LDS by direct-to-LDS loads (global_load_lds_
// dwordx4: lane l of a wave writes its 16 bytes at m0 + 16 l, so wave v's copy b covers LDS
// vectors 64 (16 b + v) ..., with no VGPR on the way), issued before the register loads, and
// thread t works the LDS vectors t + u * 1024.
// One workgroup fills the CU, so nothing else hides its arithmetic, and about 12 VALU slots per
// element would otherwise sit between the loads and the stores.  So each group of kResGroup
// register vectors is reduced as it arrives, under the loads of the later ones: its maximum g,
// e = exp(x - g) in place of x, and the sum of e folded into the thread's running (maximum,
// sum) as the two-pass kernel folds; the thread's LDS vectors form one more group.  After the
// workgroup's fold (fixed order) every output is one multiply, e * (exp(g - max) / sum), under
// the stores.  Against exp(x - max) / sum that adds two roundings (a few ulp); special values
// follow numpy: a group of -inf only holds e = 0, a NaN or +inf makes the row NaN, and a row
// of -inf gives NaN.
// kFull: the row fills the registers (n4 >= kResVpl * 1024), so their loads and stores need no
// guard; only such rows have an LDS part.
constexpr int kResT = 1024, kResW = kResT / kWave, kResVpl = 24, kResGroup = 4;
// LDS: the part of the row past the registers plus the two 16-float partial arrays, 160 KiB
constexpr int kResLdsVecs = (160 * 1024 - 2 * kResW * 4) / 16;
constexpr int kResLdsIters = (kResLdsVecs + kResT - 1) / kResT;
constexpr int64_t kResMaxVecs = static_cast<int64_t>(kResVpl) * kResT + kResLdsVecs;
static_assert(kResVpl % kResGroup == 0, "whole groups");

__device__ __forceinline__ void lds_copy16(const float* sbase, uint32_t voff, uint32_t lds_addr) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_addr) : "memory");
}

__device__ __forceinline__ float max4(f32x4 q) { return max_nan(max_nan(q.x, q.y), max_nan(q.z, q.w)); }
__device__ __forceinline__ f32x4 exp4(f32x4 q, float g) {
  return f32x4{exp_nonpos(q.x - g), exp_nonpos(q.y - g), exp_nonpos(q.z - g), exp_nonpos(q.w - g)};
}

template <bool kFull>
__global__ __launch_bounds__(kResT) void softmax_rows_f32_resident(const f32x4* __restrict__ x, f32x4* __restrict__ y,
                                                                  int n4, SoftmaxStats st) {
  typedef __attribute__((address_space(3))) f32x4 lds_f32x4_t;
  __shared__ __attribute__((aligned(16))) f32x4 rest_raw[kResLdsVecs];
  __shared__ float part_m[kResW], part_s[kResW];
  lds_f32x4_t* rest = (lds_f32x4_t*)rest_raw;
  const int tid = threadIdx.x, v = tid >> 6;
  const int64_t row = blockIdx.x;
  const f32x4* xr = x + row * n4;
  f32x4* yr = y + row * n4;
  const float ninf = -__builtin_inff();
  const int nl = n4 - kResVpl * kResT;  // vectors past the registers (uniform; > 0 only when kFull)
  if constexpr (kFull) {
    if (nl > 0) {
      const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(rest));
      const float* sbase = reinterpret_cast<const float*>(xr + kResVpl * kResT);
      const int vs = __builtin_amdgcn_readfirstlane(v);  // the wave index in a scalar register, for m0
#pragma unroll
      for (int b = 0; b < kResLdsIters; ++b) {
        const int first = (b * kResW + vs) * kWave;
        const int lane = tid & 63;
        if (first < nl && first + lane < nl)
          lds_copy16(sbase, static_cast<uint32_t>(first + lane) * 16u, lds_base + static_cast<uint32_t>(first) * 16u);
      }
    }
  }
  f32x4 xv[kResVpl];
#pragma unroll
  for (int i = 0; i < kResVpl; ++i) {
    xv[i] = kFull || tid + i * kResT < n4 ? __builtin_nontemporal_load(xr + tid + i * kResT)
                                          : f32x4{ninf, ninf, ninf, ninf};
    __builtin_amdgcn_sched_barrier(0);  // issue order = use order, so each group waits only for its own loads
  }
  float m = ninf, s = 0.f, lg = ninf;
  if constexpr (kFull) {
    if (nl > 0) {
      // the copies were issued before the kResVpl register loads: once at most that many loads
      // are outstanding, this wave's copies have landed; the barrier waits for every wave's
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kResVpl) : "memory");
      __syncthreads();
      for (int u = 0; u < kResLdsIters; ++u)
        if (tid + u * kResT < nl) lg = max_nan(lg, max4(rest[tid + u * kResT]));
      float ls = 0.f;
      for (int u = 0; u < kResLdsIters; ++u) {
        const int j = tid + u * kResT;
        if (j < nl) {
          const f32x4 e = lg == ninf ? f32x4{0.f, 0.f, 0.f, 0.f} : exp4(rest[j], lg);
          ls += (e.x + e.y) + (e.z + e.w);
          rest[j] = e;
        }
      }
      softmax_fold(m, s, lg, ls);
    }
  }
  float gmax[kResVpl / kResGroup];
#pragma unroll
  for (int g = 0; g < kResVpl / kResGroup; ++g) {
    float gm = ninf;
#pragma unroll
    for (int i = g * kResGroup; i < (g + 1) * kResGroup; ++i) gm = max_nan(gm, max4(xv[i]));
    float gs = 0.f;
#pragma unroll
    for (int i = g * kResGroup; i < (g + 1) * kResGroup; ++i) {
      xv[i] = gm == ninf ? f32x4{0.f, 0.f, 0.f, 0.f} : exp4(xv[i], gm);
      gs += (xv[i].x + xv[i].y) + (xv[i].z + xv[i].w);
    }
    softmax_fold(m, s, gm, gs);
    gmax[g] = gm;
  }
  block_softmax_fold<kResW>(m, s, part_m, part_s);
  if (tid == 0) put_softmax_stats(st, row, m, s);
  const float inv = 1.0f / s;
#pragma unroll
  for (int g = 0; g < kResVpl / kResGroup; ++g) {
    const float c = exp_nonpos(gmax[g] - m) * inv;
#pragma unroll
    for (int i = g * kResGroup; i < (g + 1) * kResGroup; ++i)
      if (kFull || tid + i * kResT < n4) __builtin_nontemporal_store(xv[i] * c, yr + tid + i * kResT);
  }
  if constexpr (kFull) {
    const float c = exp_nonpos(lg - m) * inv;
    for (int u = 0; u < kResLdsIters; ++u) {
      const int j = tid + u * kResT;
      if (j < nl) __builtin_nontemporal_store(rest[j] * c, yr + kResVpl * kResT + j);
    }
  }
}

// ------------------------------------------------------------- long rows, split over workgroups
// Rows longer than 65536 floats are cut into S segments of kSplitThreads * kVpl 16-byte vectors
// of the row's body, one workgroup each, and run in two launches:
//   softmax_split_stats: segment j's maximum m_j and s_j = sum(exp(x - m_j)) over the segment,
//     written to part[2 * (row * S + j) + {0, 1}];
//   softmax_split_write: the row's maximum mx = max_j m_j and sum = sum_j s_j * exp(m_j - mx),
//     folded in a fixed order (softmax_fold: a segment whose maximum is -inf, all of it masked,
//     adds 0), then y = exp(x - mx) * (1 / sum) over the segment.
// x is read twice and y written once, as by the workgroup-per-row kernel, but every CU is
// busy for few rows, and each element's arithmetic is that of the register-resident
// kernels: only the sum's rounding order differs.  Special values come out as numpy's: a NaN
// anywhere gives a NaN maximum and NaN everywhere; +inf gives inf - inf = NaN in its segment's
// s_j and so everywhere; a row of -inf gives mx = -inf and NaN.
// kSkew: rows start 4-byte aligned, x and y at the same offset modulo 16 bytes, and every row
// splits into a head of up to 3 elements before its first 16-byte boundary, the body, and a
// tail of up to 3; head and tail belong to segment 0.  Without kSkew rows are 16-byte aligned
// (N % 4 == 0).  Launch: grid M * S, block kSplitThreads; blockIdx.x = row * S + j, so both
// launches place a segment on the same XCD (workgroups go to the XCDs round robin).  The first
// launch reads x with ordinary loads, so that the caches keep what they can of it for the
// second (non-temporal) read: 2-6 points of HBM peak at 33-130 MB of x against non-temporal
// loads in both, and no worse at 1 GiB.
constexpr int kSplitThreads = 256;
constexpr int64_t kSplitMaxSegments = 1 << 20;

struct SplitRow {
  int64_t head, nb, tail;  // elements before the body, body vectors, elements after it
};

template <bool kSkew>
__device__ __forceinline__ SplitRow split_row(const float* xr, int64_t N) {
  if (!kSkew) return {0, N >> 2, 0};
  const int64_t to_edge = (4 - ((reinterpret_cast<uintptr_t>(xr) >> 2) & 3)) & 3;
  const int64_t head = to_edge < N ? to_edge : N;
  const int64_t nb = (N - head) >> 2;
  return {head, nb, N - head - 4 * nb};
}

template <int kVpl, bool kSkew>
__global__ __launch_bounds__(kSplitThreads) void softmax_split_stats(const float* __restrict__ x,
                                                                     float* __restrict__ part, int64_t N, int S) {
  constexpr int kW = kSplitThreads / kWave;
  __shared__ float part_m[kW], part_s[kW];
  const int tid = threadIdx.x, lane = tid & 63, v = tid >> 6;
  const int64_t row = blockIdx.x / S;
  const int seg = static_cast<int>(blockIdx.x % S);
  const float* xr = x + row * N;
  const SplitRow r = split_row<kSkew>(xr, N);
  const int64_t first = static_cast<int64_t>(seg) * (kSplitThreads * kVpl) + tid;
  const f32x4* xb = reinterpret_cast<const f32x4*>(xr + r.head) + first;
  const float ninf = -__builtin_inff();
  f32x4 xv[kVpl];
#pragma unroll
  for (int i = 0; i < kVpl; ++i)
    xv[i] = first + i * kSplitThreads < r.nb ? xb[i * kSplitThreads] : f32x4{ninf, ninf, ninf, ninf};
  const bool ht = kSkew && seg == 0;  // uniform: this segment holds the head and the tail
  float hv = ht && tid < r.head ? xr[tid] : ninf;
  float tv = ht && tid < r.tail ? xr[r.head + 4 * r.nb + tid] : ninf;
  float mx = max_nan(hv, tv);
#pragma unroll
  for (int i = 0; i < kVpl; ++i) mx = max_nan(max_nan(mx, xv[i].x), max_nan(max_nan(xv[i].y, xv[i].z), xv[i].w));
  mx = wave_max_nan(mx);
  if (lane == 0) part_m[v] = mx;
  __syncthreads();
  mx = part_m[0];
#pragma unroll
  for (int k = 1; k < kW; ++k) mx = max_nan(mx, part_m[k]);
  float sum = (ht && tid < r.head ? exp_nonpos(hv - mx) : 0.f) + (ht && tid < r.tail ? exp_nonpos(tv - mx) : 0.f);
#pragma unroll
  for (int i = 0; i < kVpl; ++i) {
    const float e = (exp_nonpos(xv[i].x - mx) + exp_nonpos(xv[i].y - mx)) +
                    (exp_nonpos(xv[i].z - mx) + exp_nonpos(xv[i].w - mx));
    if (first + i * kSplitThreads < r.nb) sum += e;
  }
  sum = wave_sum(sum);
  if (lane == 0) part_s[v] = sum;
  __syncthreads();
  if (tid == 0) {
    float tot = 0.f;
#pragma unroll
    for (int k = 0; k < kW; ++k) tot += part_s[k];
    part[2 * static_cast<int64_t>(blockIdx.x)] = mx;
    part[2 * static_cast<int64_t>(blockIdx.x) + 1] = tot;
  }
}

template <int kVpl, bool kSkew>
__global__ __launch_bounds__(kSplitThreads) void softmax_split_write(const float* __restrict__ x,
                                                                     float* __restrict__ y,
                                                                     const float* __restrict__ part, int64_t N,
                                                                     int S, SoftmaxStats st) {
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x / S;
  const int seg = static_cast<int>(blockIdx.x % S);
  const float* xr = x + row * N;
  float* yr = y + row * N;
  const SplitRow r = split_row<kSkew>(xr, N);
  const int64_t first = static_cast<int64_t>(seg) * (kSplitThreads * kVpl) + tid;
  const f32x4* xb = reinterpret_cast<const f32x4*>(xr + r.head) + first;
  f32x4* yb = reinterpret_cast<f32x4*>(yr + r.head) + first;
  const float ninf = -__builtin_inff();
  f32x4 xv[kVpl];
#pragma unroll
  for (int i = 0; i < kVpl; ++i)
    xv[i] = first + i * kSplitThreads < r.nb ? __builtin_nontemporal_load(xb + i * kSplitThreads)
                                             : f32x4{ninf, ninf, ninf, ninf};
  const bool ht = kSkew && seg == 0;
  const float hv = ht && tid < r.head ? xr[tid] : ninf;
  const float tv = ht && tid < r.tail ? xr[r.head + 4 * r.nb + tid] : ninf;
  // the row's statistics from its S partials, folded in a fixed order (partials j = t, t + 256,
  // ... by thread t, then the workgroup), so every workgroup of the row gets the same pair
  __shared__ float fm[kSplitThreads / kWave], fs[kSplitThreads / kWave];
  const float* pr = part + 2 * row * S;
  float mx = ninf, tot = 0.f;
  for (int j = tid; j < S; j += kSplitThreads) softmax_fold(mx, tot, pr[2 * j], pr[2 * j + 1]);
  block_softmax_fold<kSplitThreads / kWave>(mx, tot, fm, fs);
  if (seg == 0 && tid == 0) put_softmax_stats(st, row, mx, tot);
  const float inv = 1.0f / tot;
#pragma unroll
  for (int i = 0; i < kVpl; ++i) {
    if (first + i * kSplitThreads < r.nb) {
      const f32x4 e = {exp_nonpos(xv[i].x - mx), exp_nonpos(xv[i].y - mx), exp_nonpos(xv[i].z - mx),
                       exp_nonpos(xv[i].w - mx)};
      __builtin_nontemporal_store(e * inv, yb + i * kSplitThreads);
    }
  }
  if (ht && tid < r.head) yr[tid] = exp_nonpos(hv - mx) * inv;
  if (ht && tid < r.tail) yr[r.head + 4 * r.nb + tid] = exp_nonpos(tv - mx) * inv;
}

// Split of an [M, N] softmax: S segments per row of 256 * vpl vectors, or S = 0 (not split).
// Rows of at most 65536 floats stay in registers.  Longer rows are split when the workgroup-per-
// row kernel would leave CUs idle: fewer than 192 rows, or a last round of at most 160 rows
// after one or two full rounds of 256 (measured on MI355X at N = 65540, 128256 and 262144: the
// split is 5-20% faster there and 2-12% slower elsewhere, where both read x twice but the
// row kernel finds more of its second read in the caches).  The longest segments (16 vectors
// per thread) unless that leaves fewer than 4096 workgroups (then 8, then 4): more workgroups
// keep more of x in flight, 1-13% faster than a target of 512.  Depends on the shape only.
SoftmaxSplit softmax_split_plan(int64_t M, int64_t N) {
  if (M <= 0 || N <= 65536) return {0, 0};
  const bool idle = M < 192 || (M > 256 && M < 640 && M % 256 != 0 && M % 256 <= 160);
  if (!idle) return {0, 0};
  const int64_t n4 = N / 4;  // body vectors of a row, at most
  int vpl = 16;
  int64_t S = (n4 + kSplitThreads * vpl - 1) / (kSplitThreads * vpl);
  while (vpl > 4 && M * S < 4096) {
    vpl /= 2;
    S = (n4 + kSplitThreads * vpl - 1) / (kSplitThreads * vpl);
  }
  if (S > kSplitMaxSegments || M * S > 0x7fffffffLL) return {0, 0};
  return {static_cast<int>(S), vpl};
}

template <bool kSkew>
static void launch_softmax_split(const float* x, float* y, int64_t M, int64_t N, const SoftmaxSplit& p, float* part,
                                 const SoftmaxStats& st, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(M * p.S)), block(kSplitThreads);
  if (p.vpl == 16) {
    softmax_split_stats<16, kSkew><<<grid, block, 0, s>>>(x, part, N, p.S);
    softmax_split_write<16, kSkew><<<grid, block, 0, s>>>(x, y, part, N, p.S, st);
  } else if (p.vpl == 8) {
    softmax_split_stats<8, kSkew><<<grid, block, 0, s>>>(x, part, N, p.S);
    softmax_split_write<8, kSkew><<<grid, block, 0, s>>>(x, y, part, N, p.S, st);
  } else {
    softmax_split_stats<4, kSkew><<<grid, block, 0, s>>>(x, part, N, p.S);
    softmax_split_write<4, kSkew><<<grid, block, 0, s>>>(x, y, part, N, p.S, st);
  }
}

// Short rows (N % 4 == 0, at most 32 16-byte vectors, x and y 16-byte aligned): G lanes per row,
// one vector per lane, 64 / G rows per wave (a wave per row left most lanes idle: N = 32 ran
// at 20% of HBM peak, 64 at 38%).  The same arithmetic per element as the register kernels; the
// max and the sum are reduced over the group with xor shuffles.
template <int G>
__global__ __launch_bounds__(256) void softmax_rows_f32_grouped(const f32x4* __restrict__ x, f32x4* __restrict__ y,
                                                                int64_t M, int n4, SoftmaxStats st) {
  const int lig = threadIdx.x & (G - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (256 / G) + threadIdx.x / G;
  const bool valid = row < M && lig < n4;  // no early return: the group's shuffles need every lane
  const float ninf = -__builtin_inff();
  f32x4 v = valid ? __builtin_nontemporal_load(x + row * n4 + lig) : f32x4{ninf, ninf, ninf, ninf};
  float mx = max_nan(max_nan(v.x, v.y), max_nan(v.z, v.w));
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) mx = max_nan(mx, __shfl_xor(mx, off, kWave));
  v.x = exp_nonpos(v.x - mx);
  v.y = exp_nonpos(v.y - mx);
  v.z = exp_nonpos(v.z - mx);
  v.w = exp_nonpos(v.w - mx);
  float sum = valid ? (v.x + v.y) + (v.z + v.w) : 0.f;
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off, kWave);
  if (row < M && lig == 0) put_softmax_stats(st, row, mx, sum);
  const float inv = 1.0f / sum;
  if (valid) __builtin_nontemporal_store(v * inv, y + row * n4 + lig);
}

// The same for short rows of any length and alignment (N <= 128, 4-byte accesses): G lanes per
// row, up to 4 elements per lane, lane l holding elements l, l + G, l + 2G, l + 3G (N = 31 ran
// at 10% of HBM peak with a wave per row).
template <int G>
__global__ __launch_bounds__(256) void softmax_rows_f32_grouped_any(const float* __restrict__ x, float* __restrict__ y,
                                                                    int64_t M, int64_t N, SoftmaxStats st) {
  const int lig = threadIdx.x & (G - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (256 / G) + threadIdx.x / G;
  const float ninf = -__builtin_inff();
  const float* xr = x + row * N;
  float v[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = row < M && lig + k * G < N ? xr[lig + k * G] : ninf;
  float mx = max_nan(max_nan(v[0], v[1]), max_nan(v[2], v[3]));
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) mx = max_nan(mx, __shfl_xor(mx, off, kWave));
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    v[k] = exp_nonpos(v[k] - mx);
    if (lig + k * G < N) sum += v[k];
  }
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off, kWave);
  if (row < M && lig == 0) put_softmax_stats(st, row, mx, sum);
  const float inv = 1.0f / sum;
  if (row < M) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (lig + k * G < N) y[row * N + lig + k * G] = v[k] * inv;
  }
}

// ---------------------------------------------------------------- LDS-staged short rows
// A block of consecutive short rows is one contiguous run of n elements in memory, whatever the
// row length.  stage_in copies it to LDS with 16-byte loads: element e goes to dst[h + e], where
// h = (address of src & 127) / sizeof(T) (stage_offset), so src's 128-byte lines fall on 128-byte
// boundaries of dst: a wave's 1 KiB of vectors covers whole lines, and every whole vector moves
// with one load and one ds_write_b128 (a plain copy whose 1 KiB store runs start 16 bytes past a
// line boundary ran 17% slower than an aligned one: the lines split between two stores are
// written twice).  Vectors wholly outside the run are skipped; the at most two partial vectors at
// its ends move element by element.  stage_out is the reverse.  src and dst must be aligned to
// their element size; dst (src for stage_out) holds at least kStageSlack<T> elements past the run.
constexpr int kStageAlign = 128;
template <typename T>
constexpr int kStageSlack = kStageAlign / sizeof(T) + 16 / sizeof(T);
template <typename T>
__device__ __forceinline__ int stage_offset(const T* p) {
  return static_cast<int>((reinterpret_cast<uintptr_t>(p) & (kStageAlign - 1)) / sizeof(T));
}
template <typename T, int kT>
__device__ __forceinline__ void stage_in(const T* __restrict__ src, int n, T* dst, int h) {
  constexpr int kE = 16 / sizeof(T);
  const u32x4* base =
      reinterpret_cast<const u32x4*>(reinterpret_cast<uintptr_t>(src) & ~uintptr_t{kStageAlign - 1});
  const int nv = (h + n + kE - 1) / kE;
  for (int v = threadIdx.x; v < nv; v += kT) {
    const int e0 = v * kE - h;
    if (e0 >= 0 && e0 + kE <= n) {
      reinterpret_cast<u32x4*>(dst)[v] = __builtin_nontemporal_load(base + v);
    } else if (e0 + kE > 0) {  // every load issued before the first is used: clamped indices, no branches
      T t[kE];
#pragma unroll
      for (int k = 0; k < kE; ++k) t[k] = src[min(max(e0 + k, 0), n - 1)];
#pragma unroll
      for (int k = 0; k < kE; ++k)
        if (e0 + k >= 0 && e0 + k < n) dst[v * kE + k] = t[k];
    }
  }
}

template <typename T, int kT>
__device__ __forceinline__ void stage_out(const T* src, int h, int n, T* __restrict__ dst) {
  constexpr int kE = 16 / sizeof(T);
  u32x4* base = reinterpret_cast<u32x4*>(reinterpret_cast<uintptr_t>(dst) & ~uintptr_t{kStageAlign - 1});
  const int nv = (h + n + kE - 1) / kE;
  for (int v = threadIdx.x; v < nv; v += kT) {
    const int e0 = v * kE - h;
    if (e0 >= 0 && e0 + kE <= n) {
      __builtin_nontemporal_store(reinterpret_cast<const u32x4*>(src)[v], base + v);
    } else if (e0 + kE > 0) {  // the slot's LDS words read together (v * kE + kE <= the buffer's size)
      T t[kE];
#pragma unroll
      for (int k = 0; k < kE; ++k) t[k] = src[v * kE + k];
#pragma unroll
      for (int k = 0; k < kE; ++k)
        if (e0 + k >= 0 && e0 + k < n) dst[e0 + k] = t[k];
    }
  }
}

// Rows per workgroup of the LDS-staged short-row kernels: kShortRpt (softmax) or kLnShortRpt
// (LayerNorm) rows per group of G lanes.
constexpr int kShortRpt = 2;
constexpr int kLnShortRpt = 4;

// Short rows of any length (N <= 128) with x and y 4-byte aligned: the rows of a workgroup
// (kShortRpt * 256 / G of them, at most 8 KiB) are staged through LDS with 16-byte accesses
// (softmax_rows_f32_grouped_any's per-element 4-byte accesses of rows that straddle vectors
// ran at 55-66% of HBM peak), then each group of G lanes takes a row with
// softmax_rows_f32_grouped_any's element mapping and arithmetic, so the results are identical.
// y goes back into the same LDS slots when x and y share their offset modulo 128 bytes (each
// lane rewrites only the slots it read), after a barrier otherwise.
template <int G>
__global__ __launch_bounds__(256) void softmax_rows_f32_short_lds(const float* __restrict__ x, float* __restrict__ y,
                                                                  int64_t M, int N, SoftmaxStats st) {
  constexpr int kRows = kShortRpt * (256 / G);
  __shared__ __align__(16) float buf[kRows * 4 * G + kStageSlack<float>];
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kRows;
  const int rows = static_cast<int>(M - r0 < kRows ? M - r0 : kRows);
  const int n = rows * N;
  const float* xb = x + r0 * N;
  float* yb = y + r0 * N;
  const int hx = stage_offset(xb);
  const int hy = stage_offset(yb);
  stage_in<float, 256>(xb, n, buf, hx);
  __syncthreads();
  const int lig = threadIdx.x & (G - 1);
  const float ninf = -__builtin_inff();
  float v[kShortRpt][4];
  float inv[kShortRpt];
#pragma unroll
  for (int rr = 0; rr < kShortRpt; ++rr) {
    const int lr = rr * (256 / G) + static_cast<int>(threadIdx.x) / G;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      // read unconditionally (index < hx + kRows * N <= the buffer's size), so that the reads
      // are not serialised behind one branch each
      const float t = buf[hx + lr * N + lig + k * G];
      v[rr][k] = lr < rows && lig + k * G < N ? t : ninf;
    }
    float mx = max_nan(max_nan(v[rr][0], v[rr][1]), max_nan(v[rr][2], v[rr][3]));
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) mx = max_nan(mx, __shfl_xor(mx, off, kWave));
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[rr][k] = exp_nonpos(v[rr][k] - mx);
      if (lig + k * G < N) sum += v[rr][k];
    }
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off, kWave);
    if (lr < rows && lig == 0) put_softmax_stats(st, r0 + lr, mx, sum);
    inv[rr] = 1.0f / sum;
  }
  if (hx != hy) __syncthreads();  // uniform over the workgroup
#pragma unroll
  for (int rr = 0; rr < kShortRpt; ++rr) {
    const int lr = rr * (256 / G) + static_cast<int>(threadIdx.x) / G;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (lr < rows && lig + k * G < N) buf[hy + lr * N + lig + k * G] = v[rr][k] * inv[rr];
  }
  __syncthreads();
  stage_out<float, 256>(buf, hy, n, yb);
}

static void launch_softmax_short_lds(const float* x, float* y, int64_t M, int N, const SoftmaxStats& st,
                                     hipStream_t s) {
  int g = 1;
  while (4 * g < N) g *= 2;
  const int rows = kShortRpt * (256 / g);
  const dim3 grid(static_cast<unsigned>((M + rows - 1) / rows)), block(256);
  switch (g) {
    case 1: softmax_rows_f32_short_lds<1><<<grid, block, 0, s>>>(x, y, M, N, st); break;
    case 2: softmax_rows_f32_short_lds<2><<<grid, block, 0, s>>>(x, y, M, N, st); break;
    case 4: softmax_rows_f32_short_lds<4><<<grid, block, 0, s>>>(x, y, M, N, st); break;
    case 8: softmax_rows_f32_short_lds<8><<<grid, block, 0, s>>>(x, y, M, N, st); break;
    case 16: softmax_rows_f32_short_lds<16><<<grid, block, 0, s>>>(x, y, M, N, st); break;
    default: softmax_rows_f32_short_lds<32><<<grid, block, 0, s>>>(x, y, M, N, st); break;
  }
}

static void launch_softmax_grouped_any(const float* x, float* y, int64_t M, int64_t N, const SoftmaxStats& st,
                                      hipStream_t s) {
  int g = 1;
  while (4 * g < N) g *= 2;
  const dim3 grid(static_cast<unsigned>((M * g + 255) / 256)), block(256);
  switch (g) {
    case 1: softmax_rows_f32_grouped_any<1><<<grid, block, 0, s>>>(x, y, M, N, st); break;
    case 2: softmax_rows_f32_grouped_any<2><<<grid, block, 0, s>>>(x, y, M, N, st); break;
    case 4: softmax_rows_f32_grouped_any<4><<<grid, block, 0, s>>>(x, y, M, N, st); break;
    case 8: softmax_rows_f32_grouped_any<8><<<grid, block, 0, s>>>(x, y, M, N, st); break;
    case 16: softmax_rows_f32_grouped_any<16><<<grid, block, 0, s>>>(x, y, M, N, st); break;
    default: softmax_rows_f32_grouped_any<32><<<grid, block, 0, s>>>(x, y, M, N, st); break;
  }
}

static void launch_softmax_grouped(const f32x4* x4, f32x4* y4, int64_t M, int n4, const SoftmaxStats& st,
                                   hipStream_t s) {
  int g = 1;
  while (g < n4) g *= 2;
  const dim3 grid(static_cast<unsigned>((M * g + 255) / 256)), block(256);
  switch (g) {
    case 1: softmax_rows_f32_grouped<1><<<grid, block, 0, s>>>(x4, y4, M, n4, st); break;
    case 2: softmax_rows_f32_grouped<2><<<grid, block, 0, s>>>(x4, y4, M, n4, st); break;
    case 4: softmax_rows_f32_grouped<4><<<grid, block, 0, s>>>(x4, y4, M, n4, st); break;
    case 8: softmax_rows_f32_grouped<8><<<grid, block, 0, s>>>(x4, y4, M, n4, st); break;
    case 16: softmax_rows_f32_grouped<16><<<grid, block, 0, s>>>(x4, y4, M, n4, st); break;
    default: softmax_rows_f32_grouped<32><<<grid, block, 0, s>>>(x4, y4, M, n4, st); break;
  }
}

template <int kVpl, bool kFull, int kWaves>
static void launch_softmax_reg_waves(const f32x4* x4, f32x4* y4, int64_t M, int n4, const SoftmaxStats& st,
                                     hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((M + kWaves - 1) / kWaves));
  softmax_rows_f32_reg<kVpl, kFull, 1, kWaves><<<grid, dim3(64 * kWaves), 0, s>>>(x4, y4, M, n4, st);
}

// rows: rows per workgroup, 1, 2 or 4, or 0 (automatic).  Four rows of at most 1024 floats run
// as two waves of two rows each, otherwise one wave per row.  The automatic choice
// (`kernel_runner --sweep softmax-rows`, graph replays, us against the next best): rows of
// exactly 1024 floats run as four waves of two rows each, eight rows per workgroup (23.7
// against 24.0); rows of at most 256 floats as two waves of two rows (N = 200: 19.9 against
// 20.6 for eight); the other rows of at most 1024 floats as two waves of one row (N = 512: 23.2
// against 24.7 for eight, N = 768: 23.7 against 25.8; with a lane's last vector partly past
// the row, two rows per wave lose more than they gain); longer rows four waves of one row.
template <int kVpl>
static void launch_softmax_reg(const f32x4* x4, f32x4* y4, int64_t M, int n4, int rows, const SoftmaxStats& st,
                               hipStream_t s) {
  const bool full = n4 == kVpl * kWave;
  if (kVpl == 4 && full && rows == 0) {
    softmax_rows_f32_reg<kVpl, true, 2, 4><<<dim3(static_cast<unsigned>((M + 7) / 8)), dim3(256), 0, s>>>(x4, y4, M, n4,
                                                                                                         st);
    return;
  }
  if (kVpl == 1 && rows == 0) rows = 4;
  if (kVpl <= 4 && rows == 0) rows = 2;
  if (rows == 0) rows = 4;
  if (kVpl <= 4 && rows == 4) {
    const dim3 grid(static_cast<unsigned>((M + 3) / 4));
    if (full)
      softmax_rows_f32_reg<kVpl, true, 2, 2><<<grid, dim3(128), 0, s>>>(x4, y4, M, n4, st);
    else
      softmax_rows_f32_reg<kVpl, false, 2, 2><<<grid, dim3(128), 0, s>>>(x4, y4, M, n4, st);
    return;
  }
  switch (rows) {
    case 1:
      full ? launch_softmax_reg_waves<kVpl, true, 1>(x4, y4, M, n4, st, s)
           : launch_softmax_reg_waves<kVpl, false, 1>(x4, y4, M, n4, st, s);
      break;
    case 2:
      full ? launch_softmax_reg_waves<kVpl, true, 2>(x4, y4, M, n4, st, s)
           : launch_softmax_reg_waves<kVpl, false, 2>(x4, y4, M, n4, st, s);
      break;
    default:
      full ? launch_softmax_reg_waves<kVpl, true, 4>(x4, y4, M, n4, st, s)
           : launch_softmax_reg_waves<kVpl, false, 4>(x4, y4, M, n4, st, s);
      break;
  }
}

// True when launch_softmax_rows_f32 runs the one-wave-per-row form, the only form with a
// choice of rows per workgroup (every other form is one row per workgroup).
bool softmax_rows_per_wg_form(const float* x, const float* y, int64_t N) {
  const bool vec = (N % 4 == 0) && (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15) == 0);
  return vec && N / 4 <= 1024;
}

// rows_per_wg: 0 = automatic (4), else 1, 2 or 4 for the one-wave-per-row form.  part: workspace
// of 2 * M * softmax_split_plan(M, N).S floats, or null: rows longer than 65536 floats are then
// split over several workgroups each (16-byte aligned rows, or rows at the same offset modulo 16
// bytes in x and y), else they take the workgroup-per-row kernel.  row_max, row_sum: per-row
// outputs of the maximum and of the sum of exp(x - max), or null (every form writes them).
hipError_t launch_softmax_rows_f32(const float* x, float* y, int64_t M, int64_t N, int rows_per_wg, hipStream_t s,
                                   float* part, float* row_max, float* row_sum) {
  if (M == 0 || N == 0) return hipSuccess;  // (statistics of empty rows are rejected by the caller)
  const SoftmaxStats st{row_max, row_sum};
  if (part != nullptr) {
    const SoftmaxSplit p = softmax_split_plan(M, N);
    const uintptr_t xa = reinterpret_cast<uintptr_t>(x), ya = reinterpret_cast<uintptr_t>(y);
    if (p.S > 0 && N % 4 == 0 && ((xa | ya) & 15) == 0) {
      launch_softmax_split<false>(x, y, M, N, p, part, st, s);
      return hipGetLastError();
    }
    if (p.S > 0 && ((xa | ya) & 3) == 0 && ((xa ^ ya) & 15) == 0) {
      launch_softmax_split<true>(x, y, M, N, p, part, st, s);
      return hipGetLastError();
    }
  }
  const int rows = rows_per_wg > 0 ? rows_per_wg : 0;  // 0: the register kernels choose
  if (M > 0x7fffffffLL) return hipErrorInvalidValue;  // grid.x limit of the row-per-workgroup fallback
  const bool vec = (N % 4 == 0) && (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15) == 0);
  // rows of a non-vector shape split at the same 16-byte boundaries in x and y
  const bool skew = !vec && (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 3) == 0) &&
                    (((reinterpret_cast<uintptr_t>(x) ^ reinterpret_cast<uintptr_t>(y)) & 15) == 0);
  const int64_t n4 = N / 4;
  const f32x4* x4 = reinterpret_cast<const f32x4*>(x);
  f32x4* y4 = reinterpret_cast<f32x4*>(y);
  const int n4i = static_cast<int>(n4 < 0x7fffffff ? n4 : 0x7fffffff);
  if (vec && n4 <= 32 && rows_per_wg == 0)  // short rows: several per wave (a rows knob keeps a wave per row)
    launch_softmax_grouped(x4, y4, M, n4i, st, s);
  else if (vec && n4 <= 64)
    launch_softmax_reg<1>(x4, y4, M, n4i, rows, st, s);
  else if (vec && n4 <= 128)
    launch_softmax_reg<2>(x4, y4, M, n4i, rows, st, s);
  else if (vec && n4 <= 256)
    launch_softmax_reg<4>(x4, y4, M, n4i, rows, st, s);
  else if (vec && n4 <= 512)
    launch_softmax_reg<8>(x4, y4, M, n4i, rows, st, s);
  else if (vec && n4 <= 1024)
    launch_softmax_reg<16>(x4, y4, M, n4i, rows, st, s);
  else if (vec && n4 <= 2048)
    softmax_rows_f32_multi<16, 2><<<dim3(static_cast<unsigned>(M)), dim3(128), 0, s>>>(x4, y4, M, n4i, st);
  else if (vec && n4 <= 4096)
    softmax_rows_f32_multi<16, 4><<<dim3(static_cast<unsigned>(M)), dim3(256), 0, s>>>(x4, y4, M, n4i, st);
  else if (vec && n4 <= 8192)
    softmax_rows_f32_multi<16, 8><<<dim3(static_cast<unsigned>(M)), dim3(512), 0, s>>>(x4, y4, M, n4i, st);
  else if (vec && n4 <= 16384)
    softmax_rows_f32_multi<16, 16><<<dim3(static_cast<unsigned>(M)), dim3(1024), 0, s>>>(x4, y4, M, n4i, st);
  else if (!vec && N <= 128 && rows_per_wg == 0 &&
           ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 3) == 0)
    launch_softmax_short_lds(x, y, M, static_cast<int>(N), st, s);  // short rows at any length: staged in LDS
  else if (!vec && N <= 128 && rows_per_wg == 0)  // short rows at any alignment: several per wave
    launch_softmax_grouped_any(x, y, M, N, st, s);
  else if (!vec && N <= 64 * 16)
    softmax_rows_f32_regs<16, 1><<<dim3(static_cast<unsigned>(M)), dim3(64), 0, s>>>(x, y, M, N, st);
  else if (skew && N <= 4096)
    softmax_rows_f32_skew<16, 1><<<dim3(static_cast<unsigned>(M)), dim3(64), 0, s>>>(x, y, M, N, st);
  else if (skew && N <= 4096 * 2)
    softmax_rows_f32_skew<16, 2><<<dim3(static_cast<unsigned>(M)), dim3(128), 0, s>>>(x, y, M, N, st);
  else if (skew && N <= 4096 * 4)
    softmax_rows_f32_skew<16, 4><<<dim3(static_cast<unsigned>(M)), dim3(256), 0, s>>>(x, y, M, N, st);
  else if (skew && N <= 4096 * 8)
    softmax_rows_f32_skew<16, 8><<<dim3(static_cast<unsigned>(M)), dim3(512), 0, s>>>(x, y, M, N, st);
  else if (skew && N <= 4096 * 16)
    softmax_rows_f32_skew<16, 16><<<dim3(static_cast<unsigned>(M)), dim3(1024), 0, s>>>(x, y, M, N, st);
  else if (!vec && N <= 64 * 64)
    softmax_rows_f32_regs<64, 1><<<dim3(static_cast<unsigned>(M)), dim3(64), 0, s>>>(x, y, M, N, st);
  else if (!vec && N <= 64 * 64 * 2)
    softmax_rows_f32_regs<64, 2><<<dim3(static_cast<unsigned>(M)), dim3(128), 0, s>>>(x, y, M, N, st);
  else if (!vec && N <= 64 * 64 * 4)
    softmax_rows_f32_regs<64, 4><<<dim3(static_cast<unsigned>(M)), dim3(256), 0, s>>>(x, y, M, N, st);
  else if (!vec && N <= 64 * 64 * 8)
    softmax_rows_f32_regs<64, 8><<<dim3(static_cast<unsigned>(M)), dim3(512), 0, s>>>(x, y, M, N, st);
  else if (!vec && N <= 64 * 64 * 16)
    softmax_rows_f32_regs<64, 16><<<dim3(static_cast<unsigned>(M)), dim3(1024), 0, s>>>(x, y, M, N, st);
  else if (vec && n4 >= kResVpl * kResT && n4 <= kResMaxVecs)  // vocabulary-width rows, read once
    softmax_rows_f32_resident<true><<<dim3(static_cast<unsigned>(M)), dim3(kResT), 0, s>>>(x4, y4, n4i, st);
  else if (vec && n4 <= kResMaxVecs)
    softmax_rows_f32_resident<false><<<dim3(static_cast<unsigned>(M)), dim3(kResT), 0, s>>>(x4, y4, n4i, st);
  else if (skew || vec)
    softmax_rows_f32_online<true><<<dim3(static_cast<unsigned>(M)), dim3(1024), 0, s>>>(x, y, N, st);
  else
    softmax_rows_f32_online<false><<<dim3(static_cast<unsigned>(M)), dim3(1024), 0, s>>>(x, y, N, st);
  return hipGetLastError();
}

// ============================================================== LayerNorm forward (f16)
// Op order of the reference LayerNorm IR (pipeline/tilelang/core.py:1322-1384):
//   mean = sum(x)/N; d = x - mean; var = sum(d*d)/N; rstd = 1/sqrt(var + eps);
//   y = (d*rstd)*w + b, rounded to f16 (RNE).
// Statistics are accumulated in f32 from the exact f16 values.  The vector kernel
// uses gfx950's mixed-precision instructions so a row costs ~7 VALU per element:
// v_dot2_f32_f16 for sum(x), v_fma_mix_f32 (f16 operand, f32 math) for
// d = x*1 - mean and for d*rstd*w + b, and v_cvt_pk_f16_f32 for the packed store.
// The last step is one fused multiply-add instead of a multiply and an add
// (a difference of at most one f32 rounding before the f16 rounding).
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

// One wave per row, kLnRows rows per workgroup.  The row is held in registers (kVpl
// 16-byte vectors per lane) and read from HBM once; w and b are staged in LDS once per
// workgroup instead of being read by every row (16 KiB of L1/L2 traffic per 8 KiB row), and
// the row's loads are issued before the staging loads.  The centred values are recomputed
// in the last pass rather than kept live (the same FMA, so the same bits).
// Measured on [8192, 4096]: 24.9 us with 4 rows per workgroup and w/b read per row, 22.6 us
// like this (a plain copy of the same bytes takes 22.4 us).  The kernel must stay within 64
// VGPRs so that two workgroups fit on a CU (at one per CU it ran ~12% slower): the row loads
// share one base address, and the arithmetic runs on every lane with only the stores
// predicated (with the arithmetic inside the store branch the compiler kept f32 copies of x
// live across the reduction).  kExact (n8 == 64 * kVpl and M % kLnRows == 0) drops the tail
// masks.
constexpr int kLnRows = 16;
// Argument order: what the first loads need comes first (the first 56 bytes of arguments arrive
// preloaded in SGPRs), rstd_out and eps, needed last, after.
template <int kVpl, bool kExact>
__global__ __launch_bounds__(64 * kLnRows) void layernorm_rows_f16_wave(
    const u32x4* __restrict__ x, const u32x4* __restrict__ w, const u32x4* __restrict__ b, u32x4* __restrict__ y,
    int n8, int N, int64_t M, float* __restrict__ mean_out, float* __restrict__ rstd_out, float eps) {
  static_assert(kVpl * kWave <= 64 * kLnRows, "one staging load per thread");
  __shared__ u32x4 w_lds[kVpl * kWave], b_lds[kVpl * kWave];
  const int lane = threadIdx.x & 63;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kLnRows + (threadIdx.x >> 6);
  // Waves past the last row read row M-1 (M > 0), stage w/b, pass the barrier and store nothing.
  const bool live = kExact || row0 < M;
  const int64_t row = live ? row0 : M - 1;
  // The address is written base + lane + i*kWave so that every load shares one base register
  // and takes i*1 KiB as an immediate offset; with the index precomputed, each load got its
  // own 64-bit address (+16 VGPRs, which cost the second workgroup per CU).
  const u32x4* xr = x + row * n8 + lane;
  f16x8_t xv[kVpl];
#pragma unroll
  for (int i = 0; i < kVpl; ++i)
    xv[i] = __builtin_bit_cast(f16x8_t, (kExact || lane + i * kWave < n8) ? __builtin_nontemporal_load(xr + i * kWave)
                                                                         : u32x4(0u));
  if (threadIdx.x < (kExact ? kVpl * kWave : n8)) {
    const u32x4 wt = w[threadIdx.x], bt = b[threadIdx.x];
    w_lds[threadIdx.x] = wt;
    b_lds[threadIdx.x] = bt;
  }
  float s = 0.f;
  const f16x2_t one = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
#pragma unroll
  for (int i = 0; i < kVpl; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f16x2_t p = {xv[i][2 * j], xv[i][2 * j + 1]};
      s = __builtin_amdgcn_fdot2(p, one, s, false);  // padding lanes hold +0
    }
  const float mean = wave_sum(s) / static_cast<float>(N);
  float q = 0.f;
  // 1.0 the compiler cannot fold away, so x*unit - mean stays one v_fma_mix_f32
  // (f16 operand widened inside the instruction) instead of a convert and a subtract.
  float unit;
  asm volatile("v_mov_b32 %0, 1.0" : "=v"(unit));
#pragma unroll
  for (int i = 0; i < kVpl; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float d = __builtin_fmaf(static_cast<float>(xv[i][j]), unit, -mean);
      q = __builtin_fmaf(d, (kExact || (lane + i * kWave) < n8) ? d : 0.f, q);
    }
  const float var = wave_sum(q) / static_cast<float>(N);
  const float rstd = 1.0f / sqrtf(var + eps);
  float unit2;  // a second opaque 1.0: d is recomputed below, not kept live across the reduction
  asm volatile("v_mov_b32 %0, 1.0" : "=v"(unit2));
  __syncthreads();  // w/b staged
  u32x4* yr = y + row * n8;
#pragma unroll
  for (int i = 0; i < kVpl; ++i) {
    const int idx = lane + i * kWave;  // lanes past n8 read LDS entries never staged and store nothing
    const f16x8_t wv = __builtin_bit_cast(f16x8_t, w_lds[idx]);
    const f16x8_t bv = __builtin_bit_cast(f16x8_t, b_lds[idx]);
    f16x8_t o;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float d = __builtin_fmaf(static_cast<float>(xv[i][j]), unit2, -mean);
      o[j] = static_cast<_Float16>(__builtin_fmaf(d * rstd, static_cast<float>(wv[j]), static_cast<float>(bv[j])));
    }
    if (kExact || (live && idx < n8)) __builtin_nontemporal_store(__builtin_bit_cast(u32x4, o), yr + idx);
  }
  if ((kExact || live) && lane == 0) {  // null statistics pointers: not wanted, not written
    if (mean_out != nullptr) mean_out[row] = mean;
    if (rstd_out != nullptr) rstd_out[row] = rstd;
  }
}

// Rows longer than one wave holds (N > 4096): kW waves share a row, kWaves / kW rows per
// workgroup of kWaves waves.  Wave v of a row holds the 16-byte vectors (v*64 + lane) + i*64*kW,
// i < kVpl, in registers (the row is read from HBM once, as in the one-wave kernel); the
// wave sums are exchanged through LDS, and every wave adds the kW partials in the same order,
// so all waves of a row hold the same mean and rstd.  w and b are read from global memory
// (L2-resident, shared by all rows) rather than staged: a row of 64K halves would need 256 KiB.
template <int kVpl, int kW, int kWaves>
__global__ __launch_bounds__(64 * kWaves) void layernorm_rows_f16_multi(
    const u32x4* __restrict__ x, const u32x4* __restrict__ w, const u32x4* __restrict__ b, u32x4* __restrict__ y,
    float* __restrict__ mean_out, float* __restrict__ rstd_out, int64_t M, int n8, int N, float eps) {
  constexpr int kRows = kWaves / kW;
  static_assert(kRows * kW == kWaves, "whole rows per workgroup");
  __shared__ float part_s[kRows][kW], part_q[kRows][kW];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6, r = wave / kW, v = wave % kW;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kRows + r;
  const bool live = row0 < M;  // waves past the last row read row M-1 and store nothing
  const int64_t row = live ? row0 : M - 1;
  const u32x4* xr = x + row * n8 + v * kWave + lane;
  f16x8_t xv[kVpl];
#pragma unroll
  for (int i = 0; i < kVpl; ++i)
    xv[i] = __builtin_bit_cast(f16x8_t, v * kWave + lane + i * kWave * kW < n8
                                            ? __builtin_nontemporal_load(xr + i * kWave * kW)
                                            : u32x4(0u));
  float s = 0.f;
  const f16x2_t one = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
#pragma unroll
  for (int i = 0; i < kVpl; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f16x2_t p = {xv[i][2 * j], xv[i][2 * j + 1]};
      s = __builtin_amdgcn_fdot2(p, one, s, false);  // padding lanes hold +0
    }
  s = wave_sum(s);
  if (lane == 0) part_s[r][v] = s;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < kW; ++k) tot += part_s[r][k];
  const float mean = tot / static_cast<float>(N);
  float unit;  // an opaque 1.0, as in the one-wave kernel: x*unit - mean is one v_fma_mix_f32
  asm volatile("v_mov_b32 %0, 1.0" : "=v"(unit));
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < kVpl; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float d = __builtin_fmaf(static_cast<float>(xv[i][j]), unit, -mean);
      q = __builtin_fmaf(d, v * kWave + lane + i * kWave * kW < n8 ? d : 0.f, q);
    }
  q = wave_sum(q);
  if (lane == 0) part_q[r][v] = q;
  __syncthreads();
  float qt = 0.f;
#pragma unroll
  for (int k = 0; k < kW; ++k) qt += part_q[r][k];
  const float rstd = 1.0f / sqrtf(qt / static_cast<float>(N) + eps);
  float unit2;
  asm volatile("v_mov_b32 %0, 1.0" : "=v"(unit2));
  u32x4* yr = y + row * n8;
#pragma unroll
  for (int i = 0; i < kVpl; ++i) {
    const int idx = v * kWave + lane + i * kWave * kW;
    const bool in = idx < n8;
    const f16x8_t wv = __builtin_bit_cast(f16x8_t, in ? w[idx] : u32x4(0u));
    const f16x8_t bv = __builtin_bit_cast(f16x8_t, in ? b[idx] : u32x4(0u));
    f16x8_t o;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float d = __builtin_fmaf(static_cast<float>(xv[i][j]), unit2, -mean);
      o[j] = static_cast<_Float16>(__builtin_fmaf(d * rstd, static_cast<float>(wv[j]), static_cast<float>(bv[j])));
    }
    if (live && in) __builtin_nontemporal_store(__builtin_bit_cast(u32x4, o), yr + idx);
  }
  if (live && v == 0 && lane == 0) {
    if (mean_out != nullptr) mean_out[row] = mean;
    if (rstd_out != nullptr) rstd_out[row] = rstd;
  }
}

// Halves h .. h+7 (h < 8) of the 16 halves in (lo, hi), branch-free: dword q + i of the eight
// (q = h / 2) is selected in two stages (offset by 2 dwords when q & 2, then by 1 when q & 1;
// h is uniform per row, so the selects are too), and adjacent dwords are joined with
// v_alignbit by 16 bits when h is odd (by 0 bits, i.e. unchanged, when it is even).
// (Named scalars, not an array: with an array the compiler indexed it in scratch memory.)
__device__ __forceinline__ u32x4 halves_from(const u32x4& lo, const u32x4& hi, int h) {
  const bool by2 = (h & 4) != 0, by1 = (h & 2) != 0;
  const uint32_t e0 = by2 ? lo.z : lo.x, e1 = by2 ? lo.w : lo.y, e2 = by2 ? hi.x : lo.z;
  const uint32_t e3 = by2 ? hi.y : lo.w, e4 = by2 ? hi.z : hi.x, e5 = by2 ? hi.w : hi.y;
  const uint32_t f0 = by1 ? e1 : e0, f1 = by1 ? e2 : e1, f2 = by1 ? e3 : e2, f3 = by1 ? e4 : e3, f4 = by1 ? e5 : e4;
  const uint32_t r = (h & 1) ? 16u : 0u;
  return u32x4{__builtin_amdgcn_alignbit(f1, f0, r), __builtin_amdgcn_alignbit(f2, f1, r),
               __builtin_amdgcn_alignbit(f3, f2, r), __builtin_amdgcn_alignbit(f4, f3, r)};
}

// Elements e0 .. e0+7 of a 16-byte aligned f16 vector v of n elements, e0 = 8k + h (h < 8), read
// as the aligned 16-byte vectors k and k+1 (the second only when h > 0; element-wise past n).
__device__ __forceinline__ f16x8_t f16x8_at(const uint16_t* __restrict__ v, int64_t n, int64_t k, int h) {
  const u32x4* v8 = reinterpret_cast<const u32x4*>(v);
  const u32x4 lo = v8[k];
  if (h == 0) return __builtin_bit_cast(f16x8_t, lo);
  u32x4 hi;
  if (8 * k + 16 <= n) {
    hi = v8[k + 1];
  } else {
    uint16_t e[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) e[j] = 8 * k + 8 + j < n ? v[8 * k + 8 + j] : uint16_t(0);
    hi = u32x4{e[0] | (uint32_t(e[1]) << 16), e[2] | (uint32_t(e[3]) << 16), e[4] | (uint32_t(e[5]) << 16),
               e[6] | (uint32_t(e[7]) << 16)};
  }
  return __builtin_bit_cast(f16x8_t, halves_from(lo, hi, h));
}

// Rows that do not all start 16-byte aligned (N % 8 != 0), N <= 4096 * kW, with x and y
// sharing their alignment modulo 16 bytes: one row per workgroup of kW waves.  Each row splits
// into a head of h < 8 halves (up to its first 16-byte boundary), nb 16-byte aligned vectors
// held in registers (vector k on wave k / 64 % kW, as in the multi-wave form) and a tail of
// t < 8 halves; thread j < h holds head element j, thread j < t tail element j, so the row is
// read from HBM once.  w and b stay in L2, shared by every row: kAlignedWB (w and b 16-byte aligned) reads them as aligned 16-byte vectors
// realigned to the row's head (f16x8_at), otherwise element by element.  Same op order and
// precision as the vector forms: f32 statistics, two-pass centred variance,
// y = (d * rstd) * w + b as one FMA, rounded to f16.  Every access is bounded by the row: body
// vector k < nb covers elements h + 8k .. h + 8k + 7 < h + 8nb <= N.
template <int kVpl, int kW, bool kAlignedWB>
__global__ __launch_bounds__(64 * kW) void layernorm_rows_f16_skew(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const uint16_t* __restrict__ b,
    uint16_t* __restrict__ y, float* __restrict__ mean_out, float* __restrict__ rstd_out, int64_t M, int64_t N,
    float eps) {
  __shared__ float part_s[kW], part_q[kW];
  const int lane = threadIdx.x & 63, v = threadIdx.x >> 6, tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  if (row >= M) return;  // uniform per workgroup
  const uint16_t* xr = x + row * N;
  uint16_t* yr = y + row * N;
  const int64_t to_edge = (8 - ((reinterpret_cast<uintptr_t>(xr) >> 1) & 7)) & 7;
  const int64_t head = to_edge < N ? to_edge : N;
  const int64_t nb = (N - head) >> 3;
  const int64_t tail = N - head - 8 * nb;
  const int64_t first = v * kWave + lane;  // this lane's first body vector
  const u32x4* xb = reinterpret_cast<const u32x4*>(xr + head) + first;
  u32x4* yb = reinterpret_cast<u32x4*>(yr + head) + first;
  f16x8_t xv[kVpl];
#pragma unroll
  for (int i = 0; i < kVpl; ++i)
    xv[i] = __builtin_bit_cast(f16x8_t, first + i * kWave * kW < nb ? __builtin_nontemporal_load(xb + i * kWave * kW)
                                                                    : u32x4(0u));
  const float hx = tid < head ? f16_to_f32(xr[tid]) : 0.0f;
  const float tx = tid < tail ? f16_to_f32(xr[head + 8 * nb + tid]) : 0.0f;
  float s = hx + tx;  // padding is +0
#pragma unroll
  for (int i = 0; i < kVpl; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) s += static_cast<float>(xv[i][j]);
  s = wave_sum(s);
  if (kW > 1) {
    if (lane == 0) part_s[v] = s;
    __syncthreads();
    s = 0.f;
#pragma unroll
    for (int k = 0; k < kW; ++k) s += part_s[k];
  }
  const float mean = s / static_cast<float>(N);
  float q = 0.f;
  if (tid < head) q = (hx - mean) * (hx - mean);
  if (tid < tail) q = __builtin_fmaf(tx - mean, tx - mean, q);
#pragma unroll
  for (int i = 0; i < kVpl; ++i) {
    const bool in = first + i * kWave * kW < nb;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float d = static_cast<float>(xv[i][j]) - mean;
      q = __builtin_fmaf(d, in ? d : 0.f, q);
    }
  }
  q = wave_sum(q);
  if (kW > 1) {
    if (lane == 0) part_q[v] = q;
    __syncthreads();
    q = 0.f;
#pragma unroll
    for (int k = 0; k < kW; ++k) q += part_q[k];
  }
  const float rstd = 1.0f / sqrtf(q / static_cast<float>(N) + eps);
#pragma unroll
  for (int i = 0; i < kVpl; ++i) {
    const int64_t k = first + i * kWave * kW;
    if (k < nb) {
      f16x8_t wv, bv;
      if (kAlignedWB) {
        wv = f16x8_at(w, N, k, static_cast<int>(head));
        bv = f16x8_at(b, N, k, static_cast<int>(head));
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          wv[j] = __builtin_bit_cast(_Float16, w[head + 8 * k + j]);
          bv[j] = __builtin_bit_cast(_Float16, b[head + 8 * k + j]);
        }
      }
      f16x8_t o;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float d = static_cast<float>(xv[i][j]) - mean;
        o[j] = static_cast<_Float16>(__builtin_fmaf(d * rstd, static_cast<float>(wv[j]), static_cast<float>(bv[j])));
      }
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4, o), yb + i * kWave * kW);
    }
  }
  if (tid < head) yr[tid] = f32_to_f16_rne(__builtin_fmaf((hx - mean) * rstd, f16_to_f32(w[tid]), f16_to_f32(b[tid])));
  if (tid < tail) {
    const int64_t e = head + 8 * nb + tid;
    yr[e] = f32_to_f16_rne(__builtin_fmaf((tx - mean) * rstd, f16_to_f32(w[e]), f16_to_f32(b[e])));
  }
  if (tid == 0) {
    if (mean_out != nullptr) mean_out[row] = mean;
    if (rstd_out != nullptr) rstd_out[row] = rstd;
  }
}

// Rows of at most 4096 + 7 halves that do not all start 16-byte aligned, one wave per row, as
// in layernorm_rows_f16_skew<8, 1, .>, with w and b realigned once per workgroup instead of per
// row: the rows r = c, c + 8, c + 16, ... start at the same offset modulo 16 bytes (8 rows are
// 8N halves = 16N bytes apart), so they share the head and the shift that brings w and b to
// the body's 16-byte vectors.  Workgroup g takes class c = g % 8; its kWaves waves take that
// class's rows t = g / 8 + J (kWaves i + wave) (J = gridDim.x / 8), after staging w and b,
// shifted by the class's head, in LDS (8 KiB each).  The body arithmetic is the aligned
// one-wave kernel's (v_dot2_f32_f16 for the sum, v_fma_mix_f32 for x - mean, recomputed in
// the output pass), which keeps a row at half the registers of layernorm_rows_f16_skew (that
// kernel converts all 64 halves of a lane to f32 once and keeps them: 127 VGPRs, 4 waves per
// SIMD, 46% of HBM peak at [8192, 4099]).
constexpr int kLnLdsWaves = 4;
constexpr int kLnLdsMaxVec = 512;  // body vectors of a row of N <= 4096 + 7
// kVpl body vectors per lane: rows of at most 512 kVpl + 7 halves.
template <int kVpl, bool kAlignedWB>
__global__ __launch_bounds__(64 * kLnLdsWaves) __attribute__((amdgpu_waves_per_eu(6, 6))) void layernorm_rows_f16_skew_lds(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const uint16_t* __restrict__ b,
    uint16_t* __restrict__ y, float* __restrict__ mean_out, float* __restrict__ rstd_out, int64_t M, int64_t N,
    float eps) {
  static_assert(kVpl * kWave <= kLnLdsMaxVec, "w and b staging");
  __shared__ u32x4 w_s[kLnLdsMaxVec], b_s[kLnLdsMaxVec];
  const int lane = threadIdx.x & 63, v = threadIdx.x >> 6;
  const int64_t c = blockIdx.x % 8, j = blockIdx.x / 8, J = gridDim.x / 8;
  if (c >= M) return;  // uniform per workgroup
  // N <= 4096 + 7: head, body and tail counts fit 32 bits
  const int n = static_cast<int>(N);
  const int to_edge = static_cast<int>((8 - ((reinterpret_cast<uintptr_t>(x + c * N) >> 1) & 7)) & 7);
  const int head = to_edge < n ? to_edge : n;
  const int nb = (n - head) >> 3;
  const int tail = n - head - 8 * nb;
  for (int k = threadIdx.x; k < nb; k += 64 * kLnLdsWaves) {
    f16x8_t wv, bv;
    if (kAlignedWB) {
      wv = f16x8_at(w, N, k, head);
      bv = f16x8_at(b, N, k, head);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        wv[e] = __builtin_bit_cast(_Float16, w[head + 8 * k + e]);
        bv[e] = __builtin_bit_cast(_Float16, b[head + 8 * k + e]);
      }
    }
    w_s[k] = __builtin_bit_cast(u32x4, wv);
    b_s[k] = __builtin_bit_cast(u32x4, bv);
  }
  __syncthreads();
  // head and tail w, b of this lane (the same for every row of the class)
  const float hw = lane < head ? f16_to_f32(w[lane]) : 0.0f, hb = lane < head ? f16_to_f32(b[lane]) : 0.0f;
  const int te = head + 8 * nb + lane;
  const float tw = lane < tail ? f16_to_f32(w[te]) : 0.0f, tb = lane < tail ? f16_to_f32(b[te]) : 0.0f;
  for (int64_t t = j + J * v;; t += J * kLnLdsWaves) {
    const int64_t row = c + 8 * t;
    if (row >= M) break;  // uniform per wave: waves take their own rows, no barrier below
    const uint16_t* xr = x + row * N;
    uint16_t* yr = y + row * N;
    const u32x4* xb = reinterpret_cast<const u32x4*>(xr + head) + lane;
    u32x4* yb = reinterpret_cast<u32x4*>(yr + head) + lane;
    f16x8_t xv[kVpl];
#pragma unroll
    for (int i = 0; i < kVpl; ++i)
      xv[i] = __builtin_bit_cast(f16x8_t, lane + i * kWave < nb ? __builtin_nontemporal_load(xb + i * kWave)
                                                                 : u32x4(0u));
    const float hx = lane < head ? f16_to_f32(xr[lane]) : 0.0f;
    const float tx = lane < tail ? f16_to_f32(xr[te]) : 0.0f;
    float s = hx + tx;  // padding is +0
    const f16x2_t one = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
#pragma unroll
    for (int i = 0; i < kVpl; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f16x2_t pr = {xv[i][2 * e], xv[i][2 * e + 1]};
        s = __builtin_amdgcn_fdot2(pr, one, s, false);
      }
    s = wave_sum(s);
    const float mean = s / static_cast<float>(N);
    // an opaque 1.0: x * unit - mean stays one v_fma_mix_f32 (f16 operand widened inside)
    float unit;
    asm volatile("v_mov_b32 %0, 1.0" : "=v"(unit));
    float q = 0.f;
    if (lane < head) q = (hx - mean) * (hx - mean);
    if (lane < tail) q = __builtin_fmaf(tx - mean, tx - mean, q);
#pragma unroll
    for (int i = 0; i < kVpl; ++i) {
      const bool in = lane + i * kWave < nb;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = __builtin_fmaf(static_cast<float>(xv[i][e]), unit, -mean);
        q = __builtin_fmaf(d, in ? d : 0.f, q);
      }
    }
    q = wave_sum(q);
    const float rstd = 1.0f / sqrtf(q / static_cast<float>(N) + eps);
    float unit2;  // a second opaque 1.0: d is recomputed below, not kept across the reduction
    asm volatile("v_mov_b32 %0, 1.0" : "=v"(unit2));
#pragma unroll
    for (int i = 0; i < kVpl; ++i) {
      const int k = lane + i * kWave;
      if (k < nb) {
        const f16x8_t wv = __builtin_bit_cast(f16x8_t, w_s[k]), bv = __builtin_bit_cast(f16x8_t, b_s[k]);
        f16x8_t o;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = __builtin_fmaf(static_cast<float>(xv[i][e]), unit2, -mean);
          o[e] = static_cast<_Float16>(__builtin_fmaf(d * rstd, static_cast<float>(wv[e]), static_cast<float>(bv[e])));
        }
        // an ordinary store: the row's 128-byte lines are shared with the stores of the next
        // instruction and of the neighbouring rows, which the L2 can then merge (2.5% faster
        // than non-temporal stores at [8192, 4099])
        yb[i * kWave] = __builtin_bit_cast(u32x4, o);
      }
    }
    if (lane < head) yr[lane] = f32_to_f16_rne(__builtin_fmaf((hx - mean) * rstd, hw, hb));
    if (lane < tail) yr[te] = f32_to_f16_rne(__builtin_fmaf((tx - mean) * rstd, tw, tb));
    if (lane == 0) {
      if (mean_out != nullptr) mean_out[row] = mean;
      if (rstd_out != nullptr) rstd_out[row] = rstd;
    }
  }
}

// Rows no other form holds (longer than 65543 halves, x and y at different offsets modulo 16
// bytes, bases not 2-byte aligned): one workgroup per row (kT threads: 1024, or 256 for rows of
// at most 16384 halves, which leave a larger one idle) and the reference's three
// passes (sum; sum of squared deviations from the mean; the output), in f32 with the IR's op
// order and no contraction.  kVec: N % 8 == 0 and x, y, w, b 16-byte aligned, 16-byte accesses
// (8 halves), two per thread in flight; otherwise 2-byte accesses.  Between passes the row is
// read again, mostly from L2 (a 64K-half row is 128 KiB).
__device__ __forceinline__ float sum_f16x8(const u32x4& v) {
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k)
    s += f16_to_f32(static_cast<uint16_t>(v[k] & 0xffffu)) + f16_to_f32(static_cast<uint16_t>(v[k] >> 16));
  return s;
}

__device__ __forceinline__ float sq_dev_f16x8(const u32x4& v, float mean) {
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float a = f16_to_f32(static_cast<uint16_t>(v[k] & 0xffffu)) - mean;
    const float c = f16_to_f32(static_cast<uint16_t>(v[k] >> 16)) - mean;
    q += a * a + c * c;
  }
  return q;
}

__device__ __forceinline__ uint16_t ln_out(uint16_t xh, uint16_t wh, uint16_t bh, float mean, float rstd) {
  const float d = f16_to_f32(xh) - mean;
  const float xhat = d * rstd;
  const float scaled = xhat * f16_to_f32(wh);
  return f32_to_f16_rne(scaled + f16_to_f32(bh));
}

template <bool kVec, int kT>
__global__ __launch_bounds__(kT) void layernorm_rows_f16_long(const uint16_t* __restrict__ x,
                                                                const uint16_t* __restrict__ w,
                                                                const uint16_t* __restrict__ b, uint16_t* __restrict__ y,
                                                                float* __restrict__ mean_out,
                                                                float* __restrict__ rstd_out, int64_t N, float eps) {
#pragma clang fp contract(off)
  __shared__ float scratch[kT / kWave];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * N;
  uint16_t* yr = y + row * N;
  const int64_t n8 = N / 8;
  const u32x4* x8 = reinterpret_cast<const u32x4*>(xr);
  float s = 0.f;
  if constexpr (kVec) {
    for (int64_t i = tid; i < n8; i += 2 * kT) {
      const u32x4 v0 = x8[i];
      const u32x4 v1 = i + kT < n8 ? x8[i + kT] : u32x4(0u);
      s += sum_f16x8(v0) + sum_f16x8(v1);
    }
  } else {
    for (int64_t i = tid; i < N; i += kT) s += f16_to_f32(xr[i]);
  }
  const float mean = block_sum(s, scratch) / static_cast<float>(N);
  float q = 0.f;
  if constexpr (kVec) {
    for (int64_t i = tid; i < n8; i += 2 * kT) {
      const u32x4 v0 = x8[i];
      q += sq_dev_f16x8(v0, mean);
      if (i + kT < n8) q += sq_dev_f16x8(x8[i + kT], mean);
    }
  } else {
    for (int64_t i = tid; i < N; i += kT) {
      const float d = f16_to_f32(xr[i]) - mean;
      q += d * d;
    }
  }
  const float var = block_sum(q, scratch) / static_cast<float>(N);
  const float rstd = 1.0f / sqrtf(var + eps);
  if constexpr (kVec) {
    const u32x4* w8 = reinterpret_cast<const u32x4*>(w);
    const u32x4* b8 = reinterpret_cast<const u32x4*>(b);
    u32x4* y8 = reinterpret_cast<u32x4*>(yr);
    for (int64_t i = tid; i < n8; i += kT) {
      const u32x4 v = __builtin_nontemporal_load(x8 + i), wv = w8[i], bv = b8[i];
      u32x4 o;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t lo = ln_out(static_cast<uint16_t>(v[k] & 0xffffu), static_cast<uint16_t>(wv[k] & 0xffffu),
                                   static_cast<uint16_t>(bv[k] & 0xffffu), mean, rstd);
        const uint32_t hi = ln_out(static_cast<uint16_t>(v[k] >> 16), static_cast<uint16_t>(wv[k] >> 16),
                                   static_cast<uint16_t>(bv[k] >> 16), mean, rstd);
        o[k] = lo | (hi << 16);
      }
      __builtin_nontemporal_store(o, y8 + i);
    }
  } else {
    for (int64_t i = tid; i < N; i += kT) yr[i] = ln_out(xr[i], w[i], b[i], mean, rstd);
  }
  if (tid == 0) {
    if (mean_out != nullptr) mean_out[row] = mean;
    if (rstd_out != nullptr) rstd_out[row] = rstd;
  }
}

// Short rows (N % 8 == 0, at most 32 16-byte vectors, every tensor 16-byte aligned): G lanes per
// row, one vector of 8 halves per lane, 64 / G rows per wave (a wave per row left most lanes
// idle: N = 32 ran at 6% of HBM peak, 128 at 22%).  The wave kernel's arithmetic, with the two
// sums reduced over the group by xor shuffles; w and b read per lane (L1/L2 hits).  Each group
// takes kLnGroupedRows rows with both loads in flight together and the divisions done once per
// row on one lane (2 rows: 62-64% -> 68-71% of HBM peak at N = 32-256; 4 measured the same as 2).
constexpr int kLnGroupedRows = 2;  // rows per group of G lanes

template <int G, int kR>
__global__ __launch_bounds__(256) void layernorm_rows_f16_grouped(const u32x4* __restrict__ x,
                                                                  const u32x4* __restrict__ w,
                                                                  const u32x4* __restrict__ b, u32x4* __restrict__ y,
                                                                  float* __restrict__ mean_out,
                                                                  float* __restrict__ rstd_out, int64_t M, int n8, int N,
                                                                  float eps) {
  const int lig = threadIdx.x & (G - 1);
  // kR rows per group, 256 / G rows apart; every row's load issued before the first is used
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * (256 / G) * kR + threadIdx.x / G;
  f16x8_t xv[kR];
  bool valid[kR];
#pragma unroll
  for (int rr = 0; rr < kR; ++rr) {
    const int64_t row = row0 + rr * (256 / G);
    valid[rr] = row < M && lig < n8;  // no early return: the group's shuffles need every lane
    xv[rr] = __builtin_bit_cast(f16x8_t, valid[rr] ? __builtin_nontemporal_load(x + row * n8 + lig) : u32x4(0u));
  }
  const f16x8_t wv = __builtin_bit_cast(f16x8_t, lig < n8 ? w[lig] : u32x4(0u));
  const f16x8_t bv = __builtin_bit_cast(f16x8_t, lig < n8 ? b[lig] : u32x4(0u));
  // a row's divisions and square root are the same on the G lanes of its group: with kR > 1 and
  // G >= kR, lane rr of the group computes them for row rr and broadcasts the result
  constexpr bool kOneLane = kR > 1 && G >= kR;
  const int lead = (static_cast<int>(threadIdx.x) & (kWave - 1)) & ~(G - 1);
  const f16x2_t one = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
  float mean[kR], rstd[kR], sq[kR];
#pragma unroll
  for (int rr = 0; rr < kR; ++rr) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f16x2_t p = {xv[rr][2 * j], xv[rr][2 * j + 1]};
      s = __builtin_amdgcn_fdot2(p, one, s, false);  // padding lanes hold +0
    }
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) s += __shfl_xor(s, off, kWave);
    sq[rr] = s;
  }
  if constexpr (kOneLane) {
    float sel = sq[0];
#pragma unroll
    for (int rr = 1; rr < kR; ++rr) sel = lig == rr ? sq[rr] : sel;
    const float m = sel / static_cast<float>(N);
#pragma unroll
    for (int rr = 0; rr < kR; ++rr) mean[rr] = __shfl(m, lead + rr, kWave);
  } else {
#pragma unroll
    for (int rr = 0; rr < kR; ++rr) mean[rr] = sq[rr] / static_cast<float>(N);
  }
  float unit;  // 1.0 the compiler cannot fold away: x*unit - mean stays one v_fma_mix_f32
  asm volatile("v_mov_b32 %0, 1.0" : "=v"(unit));
#pragma unroll
  for (int rr = 0; rr < kR; ++rr) {
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float d = __builtin_fmaf(static_cast<float>(xv[rr][j]), unit, -mean[rr]);
      q = __builtin_fmaf(d, valid[rr] ? d : 0.f, q);
    }
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) q += __shfl_xor(q, off, kWave);
    sq[rr] = q;
  }
  if constexpr (kOneLane) {
    float sel = sq[0];
#pragma unroll
    for (int rr = 1; rr < kR; ++rr) sel = lig == rr ? sq[rr] : sel;
    const float r = 1.0f / sqrtf(sel / static_cast<float>(N) + eps);
#pragma unroll
    for (int rr = 0; rr < kR; ++rr) rstd[rr] = __shfl(r, lead + rr, kWave);
  } else {
#pragma unroll
    for (int rr = 0; rr < kR; ++rr) rstd[rr] = 1.0f / sqrtf(sq[rr] / static_cast<float>(N) + eps);
  }
#pragma unroll
  for (int rr = 0; rr < kR; ++rr) {
    const int64_t row = row0 + rr * (256 / G);
    if (valid[rr]) {
      f16x8_t o;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float d = __builtin_fmaf(static_cast<float>(xv[rr][j]), unit, -mean[rr]);
        o[j] = static_cast<_Float16>(__builtin_fmaf(d * rstd[rr], static_cast<float>(wv[j]), static_cast<float>(bv[j])));
      }
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4, o), y + row * n8 + lig);
    }
    if (row < M && lig == 0) {  // null statistics pointers: not wanted, not written
      if (mean_out != nullptr) mean_out[row] = mean[rr];
      if (rstd_out != nullptr) rstd_out[row] = rstd[rr];
    }
  }
}

// Short rows of any length and alignment (N <= 256 halves, 2-byte accesses): G lanes per row, up
// to 8 elements per lane, lane l holding elements l + kG, k < 8 (N = 33 ran at 3.5% of HBM peak
// with the per-class kernel); mean, centred variance and the output as in the other forms.
template <int G>
__global__ __launch_bounds__(256) void layernorm_rows_f16_grouped_any(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const uint16_t* __restrict__ b,
    uint16_t* __restrict__ y, float* __restrict__ mean_out, float* __restrict__ rstd_out, int64_t M, int64_t N,
    float eps) {
  const int lig = threadIdx.x & (G - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (256 / G) + threadIdx.x / G;
  const uint16_t* xr = x + row * N;
  float v[8];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    v[k] = row < M && lig + k * G < N ? f16_to_f32(xr[lig + k * G]) : 0.f;
    s += v[k];
  }
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) s += __shfl_xor(s, off, kWave);
  const float mean = s / static_cast<float>(N);
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float d = v[k] - mean;
    if (lig + k * G < N) q = __builtin_fmaf(d, d, q);
  }
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) q += __shfl_xor(q, off, kWave);
  const float rstd = 1.0f / sqrtf(q / static_cast<float>(N) + eps);
  if (row < M) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int64_t i = lig + k * G;
      if (i < N)
        y[row * N + i] = f32_to_f16_rne(__builtin_fmaf((v[k] - mean) * rstd, f16_to_f32(w[i]), f16_to_f32(b[i])));
    }
    if (lig == 0) {  // null statistics pointers: not wanted, not written
      if (mean_out != nullptr) mean_out[row] = mean;
      if (rstd_out != nullptr) rstd_out[row] = rstd;
    }
  }
}

// Short rows of any length (N <= 256 halves) with x and y 2-byte aligned: the rows of a workgroup
// (kShortRpt * 256 / G of them, at most 8 KiB) are staged through LDS with 16-byte accesses, w and
// b once per workgroup (three 2-byte loads per element held layernorm_rows_f16_grouped_any to
// 18-25% of HBM peak), then each group of G lanes takes a row with that kernel's element mapping
// and arithmetic, so the results are identical.  y goes back into the same LDS slots as in the
// staged softmax.
template <int G, int K>
__global__ __launch_bounds__(256) void layernorm_rows_f16_short_lds(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, const uint16_t* __restrict__ b,
    uint16_t* __restrict__ y, float* __restrict__ mean_out, float* __restrict__ rstd_out, int64_t M, int N, float eps) {
  constexpr int kRows = kLnShortRpt * (256 / G);
  __shared__ __align__(16) uint16_t buf[kRows * K * G + kStageSlack<uint16_t>];
  __shared__ float wl[8 * G], bl[8 * G];
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kRows;
  const int rows = static_cast<int>(M - r0 < kRows ? M - r0 : kRows);
  const int n = rows * N;
  const uint16_t* xb = x + r0 * N;
  uint16_t* yb = y + r0 * N;
  const int hx = stage_offset(xb);
  const int hy = stage_offset(yb);
  if (static_cast<int>(threadIdx.x) < N) {  // N <= 256 = blockDim.x
    wl[threadIdx.x] = f16_to_f32(w[threadIdx.x]);
    bl[threadIdx.x] = f16_to_f32(b[threadIdx.x]);
  }
  stage_in<uint16_t, 256>(xb, n, buf, hx);
  __syncthreads();
  const int lig = threadIdx.x & (G - 1);
  float v[kLnShortRpt][K];
  float mean[kLnShortRpt], rstd[kLnShortRpt];
  // Each row's divisions and square root (about 30 VALU instructions) are the same on all G lanes
  // of its group: with G >= kLnShortRpt, lane rr of a group computes them for its row rr and
  // broadcasts the result, one set of instructions for all the thread's rows.
  constexpr bool kOneLane = G >= kLnShortRpt;
  const int lead = (static_cast<int>(threadIdx.x) & (kWave - 1)) & ~(G - 1);
  float sum[kLnShortRpt];
#pragma unroll
  for (int rr = 0; rr < kLnShortRpt; ++rr) {
    const int lr = rr * (256 / G) + static_cast<int>(threadIdx.x) / G;
    sum[rr] = 0.f;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const float t = f16_to_f32(buf[hx + lr * N + lig + k * G]);  // in the buffer: read unconditionally
      v[rr][k] = lr < rows && lig + k * G < N ? t : 0.f;
      sum[rr] += v[rr][k];
    }
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) sum[rr] += __shfl_xor(sum[rr], off, kWave);
  }
  if constexpr (kOneLane) {
    float sel = sum[0];
#pragma unroll
    for (int rr = 1; rr < kLnShortRpt; ++rr) sel = lig == rr ? sum[rr] : sel;
    const float m = sel / static_cast<float>(N);
#pragma unroll
    for (int rr = 0; rr < kLnShortRpt; ++rr) mean[rr] = __shfl(m, lead + rr, kWave);
  } else {
#pragma unroll
    for (int rr = 0; rr < kLnShortRpt; ++rr) mean[rr] = sum[rr] / static_cast<float>(N);
  }
  float q[kLnShortRpt];
#pragma unroll
  for (int rr = 0; rr < kLnShortRpt; ++rr) {
    q[rr] = 0.f;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const float d = v[rr][k] - mean[rr];
      if (lig + k * G < N) q[rr] = __builtin_fmaf(d, d, q[rr]);
    }
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) q[rr] += __shfl_xor(q[rr], off, kWave);
  }
  if constexpr (kOneLane) {
    float sel = q[0];
#pragma unroll
    for (int rr = 1; rr < kLnShortRpt; ++rr) sel = lig == rr ? q[rr] : sel;
    const float r = 1.0f / sqrtf(sel / static_cast<float>(N) + eps);
#pragma unroll
    for (int rr = 0; rr < kLnShortRpt; ++rr) rstd[rr] = __shfl(r, lead + rr, kWave);
  } else {
#pragma unroll
    for (int rr = 0; rr < kLnShortRpt; ++rr) rstd[rr] = 1.0f / sqrtf(q[rr] / static_cast<float>(N) + eps);
  }
  if (hx != hy) __syncthreads();  // uniform over the workgroup
#pragma unroll
  for (int rr = 0; rr < kLnShortRpt; ++rr) {
    const int lr = rr * (256 / G) + static_cast<int>(threadIdx.x) / G;
    if (lr < rows) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int c = lig + k * G;
        if (c < N)
          buf[hy + lr * N + c] = f32_to_f16_rne(__builtin_fmaf((v[rr][k] - mean[rr]) * rstd[rr], wl[c], bl[c]));
      }
      if (lig == 0) {  // null statistics pointers: not wanted, not written
        if (mean_out != nullptr) mean_out[r0 + lr] = mean[rr];
        if (rstd_out != nullptr) rstd_out[r0 + lr] = rstd[rr];
      }
    }
  }
  __syncthreads();
  stage_out<uint16_t, 256>(buf, hy, n, yb);
}

static void launch_layernorm_short_lds(const uint16_t* x, const uint16_t* w, const uint16_t* b, uint16_t* y,
                                       float* mean, float* rstd, int64_t M, int N, float eps, hipStream_t s) {
  int g = 1;
  while (8 * g < N) g *= 2;
  const int rows = kLnShortRpt * (256 / g);
  const dim3 grid(static_cast<unsigned>((M + rows - 1) / rows)), block(256);
  // up to 5 or 8 elements per lane: rows of 4G + 1 .. 5G elements leave fewer idle slots with 5
#define IHIP_LN_SHORT(G)                                                                         \
  if (N <= 5 * (G))                                                                              \
    layernorm_rows_f16_short_lds<G, 5><<<grid, block, 0, s>>>(x, w, b, y, mean, rstd, M, N, eps); \
  else                                                                                           \
    layernorm_rows_f16_short_lds<G, 8><<<grid, block, 0, s>>>(x, w, b, y, mean, rstd, M, N, eps)
  switch (g) {
    case 1: IHIP_LN_SHORT(1); break;
    case 2: IHIP_LN_SHORT(2); break;
    case 4: IHIP_LN_SHORT(4); break;
    case 8: IHIP_LN_SHORT(8); break;
    case 16: IHIP_LN_SHORT(16); break;
    default: IHIP_LN_SHORT(32); break;
  }
#undef IHIP_LN_SHORT
}

static void launch_layernorm_grouped_any(const uint16_t* x, const uint16_t* w, const uint16_t* b, uint16_t* y,
                                         float* mean, float* rstd, int64_t M, int64_t N, float eps, hipStream_t s) {
  int g = 1;
  while (8 * g < N) g *= 2;
  const dim3 grid(static_cast<unsigned>((M * g + 255) / 256)), block(256);
  switch (g) {
    case 1: layernorm_rows_f16_grouped_any<1><<<grid, block, 0, s>>>(x, w, b, y, mean, rstd, M, N, eps); break;
    case 2: layernorm_rows_f16_grouped_any<2><<<grid, block, 0, s>>>(x, w, b, y, mean, rstd, M, N, eps); break;
    case 4: layernorm_rows_f16_grouped_any<4><<<grid, block, 0, s>>>(x, w, b, y, mean, rstd, M, N, eps); break;
    case 8: layernorm_rows_f16_grouped_any<8><<<grid, block, 0, s>>>(x, w, b, y, mean, rstd, M, N, eps); break;
    case 16: layernorm_rows_f16_grouped_any<16><<<grid, block, 0, s>>>(x, w, b, y, mean, rstd, M, N, eps); break;
    default: layernorm_rows_f16_grouped_any<32><<<grid, block, 0, s>>>(x, w, b, y, mean, rstd, M, N, eps); break;
  }
}

static void launch_layernorm_grouped(const u32x4* x8, const u32x4* w8, const u32x4* b8, u32x4* y8, float* mean,
                                     float* rstd, int64_t M, int n8, int N, float eps, hipStream_t s) {
  int g = 1;
  while (g < n8) g *= 2;
  constexpr int kR = kLnGroupedRows;
  const dim3 grid(static_cast<unsigned>((M * g + 256 * kR - 1) / (256 * kR))), block(256);
  switch (g) {
    case 1: layernorm_rows_f16_grouped<1, kR><<<grid, block, 0, s>>>(x8, w8, b8, y8, mean, rstd, M, n8, N, eps); break;
    case 2: layernorm_rows_f16_grouped<2, kR><<<grid, block, 0, s>>>(x8, w8, b8, y8, mean, rstd, M, n8, N, eps); break;
    case 4: layernorm_rows_f16_grouped<4, kR><<<grid, block, 0, s>>>(x8, w8, b8, y8, mean, rstd, M, n8, N, eps); break;
    case 8: layernorm_rows_f16_grouped<8, kR><<<grid, block, 0, s>>>(x8, w8, b8, y8, mean, rstd, M, n8, N, eps); break;
    case 16: layernorm_rows_f16_grouped<16, kR><<<grid, block, 0, s>>>(x8, w8, b8, y8, mean, rstd, M, n8, N, eps); break;
    default: layernorm_rows_f16_grouped<32, kR><<<grid, block, 0, s>>>(x8, w8, b8, y8, mean, rstd, M, n8, N, eps); break;
  }
}

template <int kVpl>
static void launch_layernorm_wave(const u32x4* x8, const u32x4* w8, const u32x4* b8, u32x4* y8, float* mean, float* rstd,
                                  int64_t M, int n8, int N, float eps, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((M + kLnRows - 1) / kLnRows)), block(64 * kLnRows);
  if (n8 == kVpl * kWave && M % kLnRows == 0)
    layernorm_rows_f16_wave<kVpl, true><<<grid, block, 0, s>>>(x8, w8, b8, y8, n8, N, M, mean, rstd, eps);
  else
    layernorm_rows_f16_wave<kVpl, false><<<grid, block, 0, s>>>(x8, w8, b8, y8, n8, N, M, mean, rstd, eps);
}

template <int kVpl, int kW, int kWaves>
static void launch_layernorm_multi(const u32x4* x8, const u32x4* w8, const u32x4* b8, u32x4* y8, float* mean,
                                   float* rstd, int64_t M, int n8, int N, float eps, hipStream_t s) {
  constexpr int kRows = kWaves / kW;
  const dim3 grid(static_cast<unsigned>((M + kRows - 1) / kRows)), block(64 * kWaves);
  layernorm_rows_f16_multi<kVpl, kW, kWaves><<<grid, block, 0, s>>>(x8, w8, b8, y8, mean, rstd, M, n8, N, eps);
}

// kW waves per row for rows of at most 4096 * kW + 7 halves: a body of nb <= 512 * kW vectors
// (8 per lane) plus a head and tail of < 8 each.
template <bool kAlignedWB>
static void launch_layernorm_skew(const uint16_t* x, const uint16_t* w, const uint16_t* b, uint16_t* y, float* mean,
                                  float* rstd, int64_t M, int64_t N, float eps, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(M));
  if (N <= 4096 + 7)
    layernorm_rows_f16_skew<8, 1, kAlignedWB><<<grid, dim3(64), 0, s>>>(x, w, b, y, mean, rstd, M, N, eps);
  else if (N <= 8192 + 7)
    layernorm_rows_f16_skew<8, 2, kAlignedWB><<<grid, dim3(128), 0, s>>>(x, w, b, y, mean, rstd, M, N, eps);
  else if (N <= 16384 + 7)
    layernorm_rows_f16_skew<8, 4, kAlignedWB><<<grid, dim3(256), 0, s>>>(x, w, b, y, mean, rstd, M, N, eps);
  else if (N <= 32768 + 7)
    layernorm_rows_f16_skew<8, 8, kAlignedWB><<<grid, dim3(512), 0, s>>>(x, w, b, y, mean, rstd, M, N, eps);
  else
    layernorm_rows_f16_skew<8, 16, kAlignedWB><<<grid, dim3(1024), 0, s>>>(x, w, b, y, mean, rstd, M, N, eps);
}

hipError_t launch_layernorm_rows_f16(const uint16_t* x, const uint16_t* w, const uint16_t* b, uint16_t* y, float* mean,
                                     float* rstd, int64_t M, int64_t N, float eps, hipStream_t s) {
  if (M == 0) return hipSuccess;
  if (M > 0x7fffffffLL) return hipErrorInvalidValue;  // grid.x limit of the row-per-workgroup fallback
  const uintptr_t al = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                       reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(y);
  const bool vec = N > 0 && (N % 8 == 0) && ((al & 15) == 0) && N <= 65536;
  // rows split at the same 16-byte boundaries in x and y (torch allocations are 16-byte aligned,
  // so any N qualifies); w and b are read per element
  const bool skew = !vec && N > 0 && N <= 65536 + 7 && (al & 1) == 0 &&
                    ((reinterpret_cast<uintptr_t>(x) ^ reinterpret_cast<uintptr_t>(y)) & 15) == 0;
  if (!vec && N > 0 && N <= 256) {  // short rows: several per wave
    if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 1) == 0)
      launch_layernorm_short_lds(x, w, b, y, mean, rstd, M, static_cast<int>(N), eps, s);  // staged in LDS
    else
      launch_layernorm_grouped_any(x, w, b, y, mean, rstd, M, N, eps, s);
    return hipGetLastError();
  }
  if (skew) {
    const bool wb16 = ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(b)) & 15) == 0;
    if (N <= 4096 + 7) {
      // 8 row classes x J workgroups of kLnLdsWaves waves (J <= 128: 4 workgroups per CU,
      // which measured 2-8% ahead of 8), then more rows per wave
      const int64_t per_class = (M + 7) / 8;
      const int64_t J = std::min<int64_t>(128, (per_class + kLnLdsWaves - 1) / kLnLdsWaves);
      const dim3 grid(static_cast<unsigned>(8 * J)), block(64 * kLnLdsWaves);
      const auto go = [&](auto vpl) {
        constexpr int kV = decltype(vpl)::value;
        if (wb16)
          layernorm_rows_f16_skew_lds<kV, true><<<grid, block, 0, s>>>(x, w, b, y, mean, rstd, M, N, eps);
        else
          layernorm_rows_f16_skew_lds<kV, false><<<grid, block, 0, s>>>(x, w, b, y, mean, rstd, M, N, eps);
      };
      if (N <= 1024 + 7)
        go(std::integral_constant<int, 2>{});
      else if (N <= 2048 + 7)
        go(std::integral_constant<int, 4>{});
      else
        go(std::integral_constant<int, 8>{});
    } else if (wb16) {
      launch_layernorm_skew<true>(x, w, b, y, mean, rstd, M, N, eps, s);
    } else {
      launch_layernorm_skew<false>(x, w, b, y, mean, rstd, M, N, eps, s);
    }
    return hipGetLastError();
  }
  if (!vec) {
    const dim3 grid(static_cast<unsigned>(M));
    if (N % 8 == 0 && (al & 15) == 0)  // N > 65536
      layernorm_rows_f16_long<true, 1024><<<grid, dim3(1024), 0, s>>>(x, w, b, y, mean, rstd, N, eps);
    else if (N > 16384)
      layernorm_rows_f16_long<false, 1024><<<grid, dim3(1024), 0, s>>>(x, w, b, y, mean, rstd, N, eps);
    else
      layernorm_rows_f16_long<false, 256><<<grid, dim3(256), 0, s>>>(x, w, b, y, mean, rstd, N, eps);
    return hipGetLastError();
  }
  const int n8 = static_cast<int>(N / 8);
  const u32x4* x8 = reinterpret_cast<const u32x4*>(x);
  const u32x4* w8 = reinterpret_cast<const u32x4*>(w);
  const u32x4* b8 = reinterpret_cast<const u32x4*>(b);
  u32x4* y8 = reinterpret_cast<u32x4*>(y);
  if (n8 <= 32)  // short rows: several per wave
    launch_layernorm_grouped(x8, w8, b8, y8, mean, rstd, M, n8, static_cast<int>(N), eps, s);
  else if (n8 <= 64)
    launch_layernorm_wave<1>(x8, w8, b8, y8, mean, rstd, M, n8, static_cast<int>(N), eps, s);
  else if (n8 <= 128)
    launch_layernorm_wave<2>(x8, w8, b8, y8, mean, rstd, M, n8, static_cast<int>(N), eps, s);
  else if (n8 <= 256)
    launch_layernorm_wave<4>(x8, w8, b8, y8, mean, rstd, M, n8, static_cast<int>(N), eps, s);
  else if (n8 <= 512)
    launch_layernorm_wave<8>(x8, w8, b8, y8, mean, rstd, M, n8, static_cast<int>(N), eps, s);
  // Multi-wave forms, by measured rate on 64 MiB (1 << 25 halves) of rows: up to 8K halves, 2 waves
  // per row and 8 rows per 1024-thread workgroup (74-75% of peak); longer rows, one row per
  // workgroup with 16 vectors per lane (16K: 73%, 32K and 64K: 70-71%).  Shapes with 8 vectors
  // per lane and 4 or more waves per row reached 60-62%: fewer bytes in flight per SIMD.
  else if (n8 <= 1024)
    launch_layernorm_multi<8, 2, 16>(x8, w8, b8, y8, mean, rstd, M, n8, static_cast<int>(N), eps, s);
  else if (n8 <= 2048)
    launch_layernorm_multi<16, 2, 2>(x8, w8, b8, y8, mean, rstd, M, n8, static_cast<int>(N), eps, s);
  else if (n8 <= 4096)
    launch_layernorm_multi<16, 4, 4>(x8, w8, b8, y8, mean, rstd, M, n8, static_cast<int>(N), eps, s);
  else
    launch_layernorm_multi<16, 8, 8>(x8, w8, b8, y8, mean, rstd, M, n8, static_cast<int>(N), eps, s);
  return hipGetLastError();
}

}  // namespace ihip
