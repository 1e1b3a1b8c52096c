// C = act(op(A) @ op(B) + bias) in float32 throughout: A [M, K] (or [K, M] with transpose_a),
// B [K, N] (or [N, K] with transpose_b), bias f32 [N] or null, C f32 [M, N], on gfx950's fp32
// matrix cores (v_mfma_f32_32x32x2_f32: exact f32 products, f32 accumulation; no reduced-
// precision inputs).  Any M, N, K and any alignment.
//
// Schedule (one MFMA instruction is 32x32x2 = 4096 flops in 16 passes, so a CU needs only
// 8 bytes of operands per clock at full rate: the kernel stages through registers and is
// built to keep the matrix pipe fed, not to save copy instructions):
//  * workgroup tile TB x TB (TB = 128, or 64 when 128-tiles would leave most CUs idle), k step
//    32; 256 threads = 4 waves in a 2x2 grid, each owning (TB/2)^2 = (TB/64)^2 blocks of 32x32;
//  * LDS double buffer, one barrier per k step; the next step's global loads are issued before
//    the current step's MFMAs so their latency hides behind ~4096 cycles of matrix work;
//  * each operand is copied into LDS in its own memory order with 16-byte accesses: a
//    K-contiguous operand (A as [M, K], B as [N, K]) as [row][k] rows of 36 floats, a
//    row-contiguous one (A as [K, M], B as [K, N]) as [k][row] rows of TB + 8 floats.  Both
//    paddings keep the MFMA operand reads free of bank conflicts;
//  * k order: within each 8-k slab, lane half h (lane / 32) feeds k = 4h + t to the t-th MFMA
//    (t < 4), so a lane's four k values are contiguous in a [row][k] tile (one 16-byte read)
//    and four rows apart in a [k][row] tile;
//  * the MFMA computes C^T (B as the first operand), so each lane ends with 4 consecutive
//    columns of one C row: 16-byte stores in the epilogue, which adds bias and applies ReLU
//    (numpy's maximum(x, 0): NaN and -0.0 pass through);
//  * tiles are ordered XCD-contiguously, then grouped 8 tile-rows at a time (L2 reuse).
// Edges: a 16-byte chunk that lies wholly inside the operand (and whose row stride allows it)
// is one vector load; any other chunk is loaded element by element with zeros outside, so
// ragged M, N, K and unaligned operands need no copies and no second kernel.
#include "common.hpp"

namespace ihip {

typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kF32Bk = 32;   // k per LDS tile
constexpr int kF32GroupM = 8;  // tile-rows per raster group

// LDS tile of one operand: kKMajor = [k][row] (row-contiguous operand), else [row][k].
template <int TB, bool kKMajor>
struct F32Tile {
  static constexpr int kPitch = kKMajor ? TB + 8 : kF32Bk + 4;
  static constexpr int kFloats = kKMajor ? kF32Bk * kPitch : TB * kPitch;
  static constexpr int kChunks = TB * kF32Bk / 4 / 256;  // 16-byte chunks per thread
};

// Chunk i of this thread for the tile at (row r0, k k0) of an operand with `rows` rows and K
// columns of k, stored in memory as [rows][K] (kKMajor = false) or [K][rows] (true) with
// leading dimension ld.  vec: rows of the memory layout start 16-byte aligned.
template <int TB, bool kKMajor>
__device__ __forceinline__ void f32_load_tile(const float* __restrict__ X, int64_t rows, int64_t K, int64_t ld,
                                              int64_t r0, int64_t k0, bool vec, int tid,
                                              f32x4 (&v)[F32Tile<TB, kKMajor>::kChunks]) {
#pragma unroll
  for (int i = 0; i < F32Tile<TB, kKMajor>::kChunks; ++i) {
    const int c = tid + 256 * i;
    int64_t outer, inner, outer_lim, inner_lim;
    if (kKMajor) {  // memory [K][rows]: a chunk is 4 consecutive rows at one k
      outer = k0 + c / (TB / 4);
      inner = r0 + (c % (TB / 4)) * 4;
      outer_lim = K;
      inner_lim = rows;
    } else {  // memory [rows][K]: a chunk is 4 consecutive k of one row
      outer = r0 + c / (kF32Bk / 4);
      inner = k0 + (c % (kF32Bk / 4)) * 4;
      outer_lim = rows;
      inner_lim = K;
    }
    const float* p = X + outer * ld + inner;
    if (vec && outer < outer_lim && inner + 4 <= inner_lim) {
      v[i] = *reinterpret_cast<const f32x4*>(p);
    } else {
      f32x4 t = {0.f, 0.f, 0.f, 0.f};
      if (outer < outer_lim) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (inner + e < inner_lim) t[e] = p[e];
      }
      v[i] = t;
    }
  }
}

template <int TB, bool kKMajor>
__device__ __forceinline__ void f32_store_tile(float* lds, int tid, const f32x4 (&v)[F32Tile<TB, kKMajor>::kChunks]) {
  constexpr int P = F32Tile<TB, kKMajor>::kPitch;
#pragma unroll
  for (int i = 0; i < F32Tile<TB, kKMajor>::kChunks; ++i) {
    const int c = tid + 256 * i;
    const int off = kKMajor ? (c / (TB / 4)) * P + (c % (TB / 4)) * 4 : (c / (kF32Bk / 4)) * P + (c % (kF32Bk / 4)) * 4;
    *reinterpret_cast<f32x4*>(lds + off) = v[i];
  }
}

// The four k values (4h + t, t < 4, of slab kk) of row `r` of the tile for this lane.
template <int TB, bool kKMajor>
__device__ __forceinline__ f32x4 f32_frag(const float* lds, int r, int kk, int h) {
  constexpr int P = F32Tile<TB, kKMajor>::kPitch;
  if (kKMajor) {
    const float* p = lds + (kk * 8 + 4 * h) * P + r;
    return f32x4{p[0], p[P], p[2 * P], p[3 * P]};
  }
  return *reinterpret_cast<const f32x4*>(lds + r * P + kk * 8 + 4 * h);
}

__device__ __forceinline__ float relu_keep_nan(float v) { return v < 0.0f ? 0.0f : v; }

template <int TB, bool kTA, bool kTB>
__global__ __launch_bounds__(256) void gemm_f32_bias_relu_kernel(const float* __restrict__ A,
                                                                 const float* __restrict__ B,
                                                                 const float* __restrict__ bias, float* __restrict__ C,
                                                                 int64_t M, int64_t N, int64_t K, int relu,
                                                                 int tiles_m, int tiles_n, int flags) {
  static_assert(TB == 128 || TB == 64, "tile extents");
  using TA = F32Tile<TB, kTA>;  // A as [K, M] is row-contiguous: a [k][m] tile
  using TBt = F32Tile<TB, !kTB>;  // B as [K, N] is row-contiguous: a [k][n] tile
  constexpr int kBlk = TB / 64;
  __shared__ __attribute__((aligned(16))) float lds[2 * (TA::kFloats + TBt::kFloats)];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1, h = lane >> 5;
  const bool vec_a = flags & 1, vec_b = flags & 2, vec_c = flags & 4;

  const int bid = xcd_contiguous(blockIdx.x, gridDim.x);
  const int per_group = kF32GroupM * tiles_n;
  const int g = bid / per_group, first_m = g * kF32GroupM;
  const int gsz = (tiles_m - first_m) < kF32GroupM ? (tiles_m - first_m) : kF32GroupM;
  const int tm = first_m + (bid % per_group) % gsz, tn = (bid % per_group) / gsz;
  const int64_t m0 = static_cast<int64_t>(tm) * TB, n0 = static_cast<int64_t>(tn) * TB;
  const int64_t lda = kTA ? M : K, ldb = kTB ? K : N;

  f32x16_t acc[kBlk][kBlk];
#pragma unroll
  for (int i = 0; i < kBlk; ++i)
#pragma unroll
    for (int j = 0; j < kBlk; ++j) acc[i][j] = f32x16_t{};

  const int KT = static_cast<int>((K + kF32Bk - 1) / kF32Bk);
  f32x4 ra[TA::kChunks], rb[TBt::kChunks];
  if (KT > 0) {
    f32_load_tile<TB, kTA>(A, M, K, lda, m0, 0, vec_a, tid, ra);
    f32_load_tile<TB, !kTB>(B, N, K, ldb, n0, 0, vec_b, tid, rb);
    f32_store_tile<TB, kTA>(lds, tid, ra);
    f32_store_tile<TB, !kTB>(lds + TA::kFloats, tid, rb);
  }
  __syncthreads();

  const int ra0 = wm * (TB / 2) + (lane & 31), rb0 = wn * (TB / 2) + (lane & 31);
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < KT;
    if (more) {
      const int64_t k1 = static_cast<int64_t>(kt + 1) * kF32Bk;
      f32_load_tile<TB, kTA>(A, M, K, lda, m0, k1, vec_a, tid, ra);
      f32_load_tile<TB, !kTB>(B, N, K, ldb, n0, k1, vec_b, tid, rb);
    }
    const float* la = lds + cur * (TA::kFloats + TBt::kFloats);
    const float* lb = la + TA::kFloats;
#pragma unroll
    for (int kk = 0; kk < kF32Bk / 8; ++kk) {
      f32x4 af[kBlk], bf[kBlk];
#pragma unroll
      for (int i = 0; i < kBlk; ++i) {
        af[i] = f32_frag<TB, kTA>(la, ra0 + i * 32, kk, h);
        bf[i] = f32_frag<TB, !kTB>(lb, rb0 + i * 32, kk, h);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int ni = 0; ni < kBlk; ++ni)
#pragma unroll
          for (int mi = 0; mi < kBlk; ++mi)
            acc[ni][mi] = __builtin_amdgcn_mfma_f32_32x32x2f32(bf[ni][t], af[mi][t], acc[ni][mi], 0, 0, 0);
    }
    if (more) {
      float* nxt = lds + (cur ^ 1) * (TA::kFloats + TBt::kFloats);
      f32_store_tile<TB, kTA>(nxt, tid, ra);
      f32_store_tile<TB, !kTB>(nxt + TA::kFloats, tid, rb);
    }
    __syncthreads();
  }

  // ---- epilogue: lane holds C[m][n..n+3], m = lane & 31 (+block), n = 8*g4 + 4*h (+block)
#pragma unroll
  for (int ni = 0; ni < kBlk; ++ni) {
#pragma unroll
    for (int mi = 0; mi < kBlk; ++mi) {
      const int64_t m = m0 + wm * (TB / 2) + mi * 32 + (lane & 31);
      if (m >= M) continue;
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int64_t n = n0 + wn * (TB / 2) + ni * 32 + g4 * 8 + h * 4;
        f32x4 v;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float t = acc[ni][mi][g4 * 4 + q];
          if (bias != nullptr && n + q < N) t = t + bias[n + q];
          v[q] = relu ? relu_keep_nan(t) : t;
        }
        float* p = C + m * N + n;
        if (vec_c && n + 4 <= N) {
          *reinterpret_cast<f32x4*>(p) = v;
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (n + q < N) p[q] = v[q];
        }
      }
    }
  }
}

// 128x128 tiles, or 64x64 when fewer than 256 tiles of 128x128 (the CU count) would run.
int gemm_f32_tile_extent(int64_t M, int64_t N) {
  const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
  return t128 < 256 ? 64 : 128;
}

template <int TB, bool kTA, bool kTB>
static hipError_t launch_f32_tb(const float* A, const float* B, const float* bias, float* C, int64_t M, int64_t N,
                                int64_t K, int relu, int flags, hipStream_t s) {
  const int64_t tm = (M + TB - 1) / TB, tn = (N + TB - 1) / TB;
  if (tm * tn > 0x7fffffffLL) return hipErrorInvalidValue;
  gemm_f32_bias_relu_kernel<TB, kTA, kTB><<<dim3(static_cast<unsigned>(tm * tn)), dim3(256), 0, s>>>(
      A, B, bias, C, M, N, K, relu, static_cast<int>(tm), static_cast<int>(tn), flags);
  return hipGetLastError();
}

template <int TB>
static hipError_t launch_f32_layout(const float* A, const float* B, const float* bias, float* C, int64_t M, int64_t N,
                                    int64_t K, bool ta, bool tb, int relu, int flags, hipStream_t s) {
  if (!ta && !tb) return launch_f32_tb<TB, false, false>(A, B, bias, C, M, N, K, relu, flags, s);
  if (!ta) return launch_f32_tb<TB, false, true>(A, B, bias, C, M, N, K, relu, flags, s);
  if (!tb) return launch_f32_tb<TB, true, false>(A, B, bias, C, M, N, K, relu, flags, s);
  return launch_f32_tb<TB, true, true>(A, B, bias, C, M, N, K, relu, flags, s);
}

static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// tile: 0 = automatic (gemm_f32_tile_extent), else 64 or 128.  Results do not depend on the
// tile: every C element sums its k in the same order (8-k slabs in ascending order, each
// slab as four MFMAs in the same lane pairing).
hipError_t launch_gemm_f32_bias_relu(const float* A, const float* B, const float* bias, float* C, int64_t M,
                                     int64_t N, int64_t K, bool ta, bool tb, int relu, int tile, hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  const int64_t lda = ta ? M : K, ldb = tb ? K : N;
  const int flags = ((lda % 4 == 0 && al16(A)) ? 1 : 0) | ((ldb % 4 == 0 && al16(B)) ? 2 : 0) |
                    ((N % 4 == 0 && al16(C)) ? 4 : 0);
  const int tb_ext = tile != 0 ? tile : gemm_f32_tile_extent(M, N);
  return tb_ext == 64 ? launch_f32_layout<64>(A, B, bias, C, M, N, K, ta, tb, relu, flags, s)
                      : launch_f32_layout<128>(A, B, bias, C, M, N, K, ta, tb, relu, flags, s);
}

}  // namespace ihip
