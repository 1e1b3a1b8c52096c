// C = relu?(op(A) @ op(B) + bias?) with A [M,K] (or [K,M] transposed) and B [K,N] (or
// [N,K] transposed), bf16 row-major, bias f32 [N], f32 accumulation on CDNA4 MFMA,
// C bf16 (RNE) — any shape.
//
// Entry point of the GEMM family: shapes whose rows all start 16-byte aligned (N % 8 == 0,
// K % 8 == 0, M % 8 == 0 for a transposed A) with 16-byte aligned operands go to
// gemm_fast.hip, for any M, N and K; every other shape runs the guarded kernel below, which
// stages operands through registers:
//  * workgroup tile TB(M) x TB(N), TB = 256, or 128 for grids of at most 128 tiles of 256x256
//    (half the CUs; as in gemm_fast.hip), K step 64; 256 threads = 4 waves in a 2x2 grid,
//    each wave owning a TB/2 x TB/2 sub-tile = (TB/64)^2 blocks of v_mfma_f32_32x32x16_bf16;
//    both tile extents accumulate every C element in the same k order (identical results);
//  * LDS double buffer: A tile as [m][k] and B tile transposed to [n][k] (rows padded
//    to 144 B) so both MFMA operands are 16-byte reads of 8 consecutive k;
//  * B is transposed on the way into LDS: each thread loads an 8(k) x 8(n) block and
//    writes eight 16-byte [n][k] rows;
//  * loads are element-wise with zero fill outside [M, N, K] and stores element-wise,
//    so any M, N, K and any alignment are handled;
//  * a transposed operand swaps roles: A given as [K,M] is loaded like B and transposed into
//    the [m][k] tile, B given as [N,K] is loaded like A straight into the [n][k] tile.
#include "common.hpp"

namespace ihip {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;
constexpr int kLdsRow = 72;                      // halves per LDS row (64 + 8 pad)
constexpr int kGroupM = 8;                       // tile-rows per raster group
// One operand tile of TB rows, and the LDS of {A, Bt} x double buffer (147456 B for TB = 256).
template <int TB> constexpr int tile_halves() { return TB * kLdsRow; }
template <int TB> constexpr int lds_halves() { return 2 * 2 * tile_halves<TB>(); }

__device__ __forceinline__ uint32_t dw(const uint4& v, int q) {
  return q == 0 ? v.x : q == 1 ? v.y : q == 2 ? v.z : v.w;
}
__device__ __forceinline__ uint32_t lo_pair(uint32_t a, uint32_t b) { return (a & 0xffffu) | (b << 16); }
__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) { return (a >> 16) | (b & 0xffff0000u); }

// TB rows x 64 k as 16-byte chunks, TB/32 per thread.
template <bool kGuard, int TB>
__device__ __forceinline__ void load_a(const uint16_t* __restrict__ A, int64_t M, int64_t K, int64_t m0, int64_t k0,
                                       int tid, uint4 (&ra)[8]) {
#pragma unroll
  for (int i = 0; i < TB / 32; ++i) {
    const int c = tid + 256 * i;
    const int64_t gm = m0 + (c >> 3), gk = k0 + (c & 7) * 8;
    if (!kGuard) {
      ra[i] = *reinterpret_cast<const uint4*>(A + gm * K + gk);
    } else {
      uint16_t h[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) h[e] = (gm < M && gk + e < K) ? A[gm * K + gk + e] : uint16_t(0);
      ra[i] = make_uint4(h[0] | (uint32_t(h[1]) << 16), h[2] | (uint32_t(h[3]) << 16), h[4] | (uint32_t(h[5]) << 16),
                         h[6] | (uint32_t(h[7]) << 16));
    }
  }
}

template <int TB>
__device__ __forceinline__ void store_a(uint16_t* lds_a, int tid, const uint4 (&ra)[8]) {
#pragma unroll
  for (int i = 0; i < TB / 32; ++i) {
    const int c = tid + 256 * i;
    *reinterpret_cast<uint4*>(lds_a + (c >> 3) * kLdsRow + (c & 7) * 8) = ra[i];
  }
}

// Thread t < TB owns the 8(k) x 8(n) block (kb = t & 7, nb = t >> 3) of the 64 x TB B tile
// (with TB = 128 the last two waves own none: the callers skip them, a uniform branch).
template <bool kGuard>
__device__ __forceinline__ void load_b(const uint16_t* __restrict__ B, int64_t K, int64_t N, int64_t k0, int64_t n0,
                                       int tid, uint4 (&rb)[8]) {
  const int kb = tid & 7, nb = tid >> 3;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int64_t gk = k0 + kb * 8 + r, gn = n0 + nb * 8;
    if (!kGuard) {
      rb[r] = *reinterpret_cast<const uint4*>(B + gk * N + gn);
    } else {
      uint16_t h[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) h[e] = (gk < K && gn + e < N) ? B[gk * N + gn + e] : uint16_t(0);
      rb[r] = make_uint4(h[0] | (uint32_t(h[1]) << 16), h[2] | (uint32_t(h[3]) << 16), h[4] | (uint32_t(h[5]) << 16),
                         h[6] | (uint32_t(h[7]) << 16));
    }
  }
}

__device__ __forceinline__ void store_bt(uint16_t* lds_b, int tid, const uint4 (&rb)[8]) {
  const int kb = tid & 7, nb = tid >> 3;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int q = j >> 1;
    uint4 o;
    if ((j & 1) == 0) {
      o.x = lo_pair(dw(rb[0], q), dw(rb[1], q));
      o.y = lo_pair(dw(rb[2], q), dw(rb[3], q));
      o.z = lo_pair(dw(rb[4], q), dw(rb[5], q));
      o.w = lo_pair(dw(rb[6], q), dw(rb[7], q));
    } else {
      o.x = hi_pair(dw(rb[0], q), dw(rb[1], q));
      o.y = hi_pair(dw(rb[2], q), dw(rb[3], q));
      o.z = hi_pair(dw(rb[4], q), dw(rb[5], q));
      o.w = hi_pair(dw(rb[6], q), dw(rb[7], q));
    }
    *reinterpret_cast<uint4*>(lds_b + (nb * 8 + j) * kLdsRow + kb * 8) = o;
  }
}

__device__ __forceinline__ float relu_np(float v) { return v < 0.0f ? 0.0f : v; }  // keeps -0.0 and NaN

// One K slice of both operands into registers, then into the [m][k] / [n][k] LDS tiles.
template <bool kGuard, bool kTA, bool kTB, int TB>
__device__ __forceinline__ void load_slice(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, int64_t M,
                                           int64_t N, int64_t K, int64_t m0, int64_t n0, int64_t k0, int tid,
                                           uint4 (&ra)[8], uint4 (&rb)[8]) {
  const bool blk = tid < TB;  // owns an 8x8 block of a K-major operand
  if (!kTA) load_a<kGuard, TB>(A, M, K, m0, k0, tid, ra);
  else if (blk) load_b<kGuard>(A, K, M, k0, m0, tid, ra);
  if (!kTB) {
    if (blk) load_b<kGuard>(B, K, N, k0, n0, tid, rb);
  } else {
    load_a<kGuard, TB>(B, N, K, n0, k0, tid, rb);
  }
}

template <bool kTA, bool kTB, int TB>
__device__ __forceinline__ void store_slice(uint16_t* lds_a, uint16_t* lds_b, int tid, const uint4 (&ra)[8],
                                            const uint4 (&rb)[8]) {
  const bool blk = tid < TB;
  if (!kTA) store_a<TB>(lds_a, tid, ra);
  else if (blk) store_bt(lds_a, tid, ra);
  if (!kTB) {
    if (blk) store_bt(lds_b, tid, rb);
  } else {
    store_a<TB>(lds_b, tid, rb);
  }
}

template <bool kGuard, bool kTA, bool kTB, int TB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_bf16_bias_relu_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                                const float* __restrict__ bias, uint16_t* __restrict__ C, int64_t M, int64_t N,
                                int64_t K, int relu, int tiles_m, int tiles_n) {
  static_assert(TB == 256 || TB == 128, "tile extents");
  constexpr int kBlk = TB / 64;  // 32x32 blocks per wave and dimension
  constexpr int kTileHalves = tile_halves<TB>();
  __shared__ __attribute__((aligned(16))) uint16_t lds[lds_halves<TB>()];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;

  // ---- tile schedule: XCD-contiguous, then grouped raster inside each XCD's range
  const int bid = xcd_contiguous(blockIdx.x, gridDim.x);
  const int per_group = kGroupM * tiles_n;
  const int g = bid / per_group, first_m = g * kGroupM;
  const int gsz = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int tm = first_m + (bid % per_group) % gsz, tn = (bid % per_group) / gsz;
  const int64_t m0 = static_cast<int64_t>(tm) * TB, n0 = static_cast<int64_t>(tn) * TB;

  f32x16_t acc[kBlk][kBlk];
#pragma unroll
  for (int i = 0; i < kBlk; ++i)
#pragma unroll
    for (int j = 0; j < kBlk; ++j) acc[i][j] = f32x16_t{};

  const int KT = static_cast<int>((K + kBK - 1) / kBK);
  uint4 ra[8], rb[8];
  if (KT > 0) {
    load_slice<kGuard, kTA, kTB, TB>(A, B, M, N, K, m0, n0, 0, tid, ra, rb);
    store_slice<kTA, kTB, TB>(lds, lds + kTileHalves, tid, ra, rb);
  }
  __syncthreads();

  const int a_off = (wm * (TB / 2) + (lane & 31)) * kLdsRow + (lane >> 5) * 8;
  const int b_off = (wn * (TB / 2) + (lane & 31)) * kLdsRow + (lane >> 5) * 8;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < KT;
    if (more)
      load_slice<kGuard, kTA, kTB, TB>(A, B, M, N, K, m0, n0, static_cast<int64_t>(kt + 1) * kBK, tid, ra, rb);
    const uint16_t* la = lds + cur * 2 * kTileHalves + a_off;
    const uint16_t* lb = lds + cur * 2 * kTileHalves + kTileHalves + b_off;
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      bf16x8_t af[kBlk], bf[kBlk];
#pragma unroll
      for (int i = 0; i < kBlk; ++i) {
        af[i] = *reinterpret_cast<const bf16x8_t*>(la + i * 32 * kLdsRow + kk * 16);
        bf[i] = *reinterpret_cast<const bf16x8_t*>(lb + i * 32 * kLdsRow + kk * 16);
      }
#pragma unroll
      for (int ni = 0; ni < kBlk; ++ni)
#pragma unroll
        for (int mi = 0; mi < kBlk; ++mi)
          acc[ni][mi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[ni], af[mi], acc[ni][mi], 0, 0, 0);
    }
    if (more) {
      uint16_t* nxt = lds + (cur ^ 1) * 2 * kTileHalves;
      store_slice<kTA, kTB, TB>(nxt, nxt + kTileHalves, tid, ra, rb);
    }
    __syncthreads();
  }

  // ---- epilogue: lane holds C[m][n..n+3] for m = lane&31 (+block), n = 8*g + 4*(lane>>5) (+block)
#pragma unroll
  for (int ni = 0; ni < kBlk; ++ni) {
#pragma unroll
    for (int mi = 0; mi < kBlk; ++mi) {
      const int64_t m = m0 + wm * (TB / 2) + mi * 32 + (lane & 31);
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int64_t n = n0 + wn * (TB / 2) + ni * 32 + g4 * 8 + (lane >> 5) * 4;
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float t = acc[ni][mi][g4 * 4 + q];
          if (bias != nullptr && (!kGuard || n + q < N)) t = t + bias[n + q];
          v[q] = relu ? relu_np(t) : t;
        }
        if (!kGuard) {
          uint2 pk;
          pk.x = f32_to_bf16_rne(v[0]) | (uint32_t(f32_to_bf16_rne(v[1])) << 16);
          pk.y = f32_to_bf16_rne(v[2]) | (uint32_t(f32_to_bf16_rne(v[3])) << 16);
          *reinterpret_cast<uint2*>(C + m * N + n) = pk;
        } else if (m < M) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (n + q < N) C[m * N + n + q] = f32_to_bf16_rne(v[q]);
        }
      }
    }
  }
}

bool gemm_fast_fits(int64_t M, int64_t N, int64_t K, bool transpose_a, bool transpose_b, const void* A, const void* B,
                    const void* C);
hipError_t launch_gemm_fast(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M, int64_t N,
                            int64_t K, bool transpose_a, bool transpose_b, int relu, int tile, hipStream_t s,
                            bool c_unaligned);
hipError_t launch_gemm_packed(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                              int64_t N, int64_t K, bool ta, bool tb, int relu, int tile, void* ws, int64_t ws_bytes,
                              hipStream_t s);
hipError_t launch_gemm_split(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                             int64_t N, int64_t K, bool ta, bool tb, int relu, int tile, int splits, void* ws,
                             int64_t ws_bytes, hipStream_t s);

template <bool kTA, bool kTB, int TB>
static hipError_t launch_guarded(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                                 int64_t N, int64_t K, int relu, hipStream_t s) {
  const int64_t tm = (M + TB - 1) / TB, tn = (N + TB - 1) / TB;
  if (tm * tn > 0x7fffffffLL) return hipErrorInvalidValue;
  gemm_bf16_bias_relu_kernel<true, kTA, kTB, TB><<<dim3(static_cast<unsigned>(tm * tn)), dim3(256), 0, s>>>(
      A, B, bias, C, M, N, K, relu, static_cast<int>(tm), static_cast<int>(tn));
  return hipGetLastError();
}

template <int TB>
static hipError_t launch_guarded_tb(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                                    int64_t N, int64_t K, bool transpose_a, bool transpose_b, int relu, hipStream_t s) {
  if (!transpose_a && !transpose_b) return launch_guarded<false, false, TB>(A, B, bias, C, M, N, K, relu, s);
  if (!transpose_a) return launch_guarded<false, true, TB>(A, B, bias, C, M, N, K, relu, s);
  if (!transpose_b) return launch_guarded<true, false, TB>(A, B, bias, C, M, N, K, relu, s);
  return launch_guarded<true, true, TB>(A, B, bias, C, M, N, K, relu, s);
}

int gemm_fast_tile_extent(int64_t M, int64_t N);

// tile: 0 = automatic (256x256 tiles, 128x128 for grids of at most 128 256x256 tiles), else
// 128 or 256; the same rule and choice for the tiled and the guarded kernel.
hipError_t launch_gemm_bf16_bias_relu(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                                      int64_t N, int64_t K, bool transpose_a, bool transpose_b, int relu, int tile,
                                      hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  if (gemm_fast_fits(M, N, K, transpose_a, transpose_b, A, B, C))
    return launch_gemm_fast(A, B, bias, C, M, N, K, transpose_a, transpose_b, relu, tile, s, false);
  const int tb = tile != 0 ? tile : gemm_fast_tile_extent(M, N);
  return tb == 128 ? launch_guarded_tb<128>(A, B, bias, C, M, N, K, transpose_a, transpose_b, relu, s)
                   : launch_guarded_tb<256>(A, B, bias, C, M, N, K, transpose_a, transpose_b, relu, s);
}

// The same with a workspace (ws, ws_bytes; may be null / 0): operands the tiled kernel cannot
// read in place are packed into it and the tiled kernel runs on the copies, and a grid of too
// few tiles is split along K with f32 partials in it (gemm_pack.hip); without a large enough
// workspace the unsplit tiled kernel or the guarded kernel runs, as above.
hipError_t launch_gemm_bf16_bias_relu_ws(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C,
                                         int64_t M, int64_t N, int64_t K, bool transpose_a, bool transpose_b, int relu,
                                         int tile, void* ws, int64_t ws_bytes, hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  // split-K by the split rule when the workspace holds the partials, else unsplit
  hipError_t e = launch_gemm_split(A, B, bias, C, M, N, K, transpose_a, transpose_b, relu, tile, 0, ws, ws_bytes, s);
  if (e != hipErrorNotSupported) return e;
  if (!gemm_fast_fits(M, N, K, transpose_a, transpose_b, A, B, C)) {
    e = launch_gemm_packed(A, B, bias, C, M, N, K, transpose_a, transpose_b, relu, tile, ws, ws_bytes, s);
    if (e != hipErrorNotSupported) return e;
  }
  return launch_gemm_bf16_bias_relu(A, B, bias, C, M, N, K, transpose_a, transpose_b, relu, tile, s);
}

}  // namespace ihip
