// C = relu?(A @ B + bias?) with A [M,K] bf16, B [K,N] bf16 (both row-major),
// bias f32 [N], f32 accumulation on CDNA4 MFMA, C bf16 (RNE).
//
// Tiling (gfx950):
//  * workgroup tile 256(M) x 256(N), K step 64; 256 threads = 4 waves in a 2x2
//    grid, each wave owning a 128x128 sub-tile = 4x4 blocks of
//    v_mfma_f32_32x32x16_bf16 (256 f32 accumulators per lane);
//  * LDS double buffer: A tile as [m][k] and B tile transposed to [n][k] so both
//    MFMA operands are 16-byte ds_read_b128 of 8 consecutive k; rows padded to
//    144 B so 16 consecutive rows land on distinct bank groups;
//  * B is transposed on the way into LDS: each thread loads an 8(k) x 8(n) block
//    with eight 16-byte loads and writes eight 16-byte [n][k] rows;
//  * the next K tile's global loads are issued before the current tile's MFMAs
//    and written to the other LDS buffer after them: one barrier per K step;
//  * the MFMA is issued as D = Bt * At, so each lane's accumulators hold four
//    consecutive n of one m: the epilogue adds bias, applies ReLU and stores
//    8 bytes per lane;
//  * tiles are remapped so each of the 8 XCDs (private L2) works on one
//    contiguous, grouped region of C, concurrently sharing A rows and B columns.
// Tiles that do not fit the shape (M, N not multiples of 256, K not a multiple
// of 64, or unaligned pointers) use the guarded instantiation, which loads
// element-wise with zero fill and stores element-wise.
#include "common.hpp"

namespace ihip {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kLdsRow = 72;                      // halves per LDS row (64 + 8 pad)
constexpr int kTileHalves = 256 * kLdsRow;       // one operand tile
constexpr int kLdsHalves = 2 * 2 * kTileHalves;  // {A, Bt} x double buffer = 147456 B
constexpr int kGroupM = 8;                       // tile-rows per raster group

__device__ __forceinline__ uint32_t dw(const uint4& v, int q) {
  return q == 0 ? v.x : q == 1 ? v.y : q == 2 ? v.z : v.w;
}
__device__ __forceinline__ uint32_t lo_pair(uint32_t a, uint32_t b) { return (a & 0xffffu) | (b << 16); }
__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) { return (a >> 16) | (b & 0xffff0000u); }

template <bool kGuard>
__device__ __forceinline__ void load_a(const uint16_t* __restrict__ A, int64_t M, int64_t K, int64_t m0, int64_t k0,
                                       int tid, uint4 (&ra)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
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

__device__ __forceinline__ void store_a(uint16_t* lds_a, int tid, const uint4 (&ra)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = tid + 256 * i;
    *reinterpret_cast<uint4*>(lds_a + (c >> 3) * kLdsRow + (c & 7) * 8) = ra[i];
  }
}

// Thread t owns the 8(k) x 8(n) block (kb = t & 7, nb = t >> 3) of the 64 x 256 B tile.
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

template <bool kGuard>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_bf16_bias_relu_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                                const float* __restrict__ bias, uint16_t* __restrict__ C, int64_t M, int64_t N,
                                int64_t K, int relu, int tiles_m, int tiles_n) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[kLdsHalves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;

  // ---- tile schedule: XCD-contiguous, then grouped raster inside each XCD's range
  int bid = blockIdx.x;
  const int T = gridDim.x;
  if (T % kNumXcd == 0) bid = (bid % kNumXcd) * (T / kNumXcd) + bid / kNumXcd;
  const int per_group = kGroupM * tiles_n;
  const int g = bid / per_group, first_m = g * kGroupM;
  const int gsz = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int tm = first_m + (bid % per_group) % gsz, tn = (bid % per_group) / gsz;
  const int64_t m0 = static_cast<int64_t>(tm) * kBM, n0 = static_cast<int64_t>(tn) * kBN;

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16_t{};

  const int KT = static_cast<int>((K + kBK - 1) / kBK);
  uint4 ra[8], rb[8];
  if (KT > 0) {
    load_a<kGuard>(A, M, K, m0, 0, tid, ra);
    load_b<kGuard>(B, K, N, 0, n0, tid, rb);
    store_a(lds, tid, ra);
    store_bt(lds + kTileHalves, tid, rb);
  }
  __syncthreads();

  const int a_off = (wm * 128 + (lane & 31)) * kLdsRow + (lane >> 5) * 8;
  const int b_off = (wn * 128 + (lane & 31)) * kLdsRow + (lane >> 5) * 8;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < KT;
    if (more) {
      load_a<kGuard>(A, M, K, m0, static_cast<int64_t>(kt + 1) * kBK, tid, ra);
      load_b<kGuard>(B, K, N, static_cast<int64_t>(kt + 1) * kBK, n0, tid, rb);
    }
    const uint16_t* la = lds + cur * 2 * kTileHalves + a_off;
    const uint16_t* lb = lds + cur * 2 * kTileHalves + kTileHalves + b_off;
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      bf16x8_t af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        af[i] = *reinterpret_cast<const bf16x8_t*>(la + i * 32 * kLdsRow + kk * 16);
        bf[i] = *reinterpret_cast<const bf16x8_t*>(lb + i * 32 * kLdsRow + kk * 16);
      }
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
          acc[ni][mi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[ni], af[mi], acc[ni][mi], 0, 0, 0);
    }
    if (more) {
      uint16_t* nxt = lds + (cur ^ 1) * 2 * kTileHalves;
      store_a(nxt, tid, ra);
      store_bt(nxt + kTileHalves, tid, rb);
    }
    __syncthreads();
  }

  // ---- epilogue: lane holds C[m][n..n+3] for m = lane&31 (+block), n = 8*g + 4*(lane>>5) (+block)
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) {
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      const int64_t m = m0 + wm * 128 + mi * 32 + (lane & 31);
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int64_t n = n0 + wn * 128 + ni * 32 + g4 * 8 + (lane >> 5) * 4;
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

// ============================================================================
// Fast path for full tiles: operands stream straight into LDS.
//
// Both operand tiles are copied with gfx950's direct-to-LDS loads
// (global_load_lds_dwordx4): lane l of a wave writes its 16 bytes to
// LDS base + 16*l, so no VGPRs hold tile data and the copy of tile k+1 runs
// under the MFMAs of tile k.  The LDS placement is fixed by the lane number,
// so bank conflicts are avoided by choosing which global chunk each lane
// fetches (XOR swizzles below), not by padding.
//
//  A stage: [256 m][64 k] bf16, 128 B rows, 16-B chunk p of row r holds logical
//           k-chunk p ^ (r & 7): the 8 rows a ds_read_b128 phase touches hit 8
//           different chunk columns.
//  B stage: [64 k][256 n] bf16, 512 B rows, 16-B chunk p of row k holds logical
//           n-chunk p ^ (2*(k & 3)): the 4 rows one ds_read_b64_tr_b16 lane group
//           touches land on 4 different 32-B bank windows.
//  B fragments are read with ds_read_b64_tr_b16: lanes 4t+q of a 16-lane group
//  address row k0+t, columns n0+4q..4q+3, and lane i receives column n0+i for
//  rows k0..k0+3 — the k-contiguous layout the MFMA operand needs, with no VALU
//  transposition.
// ============================================================================
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x8_t __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
typedef __attribute__((address_space(3))) char lds_char_t;

constexpr int kStageA = 256 * 64 * 2;  // bytes
constexpr int kStageB = 64 * 256 * 2;  // bytes
constexpr int kStage = kStageA + kStageB;

// Per-lane byte offsets of the direct-to-LDS copies (the same for every
// instruction and every K step; the uniform part of each address is scalar).
struct DmaLane {
  uint32_t a;  // byte offset inside the A tile, relative to its wave-instruction base row
  uint32_t b;  // byte offset inside the B tile, relative to its wave-instruction base row
};

__device__ __forceinline__ DmaLane dma_lane(int64_t N, int64_t K, int wave, int lane) {
  // A chunk s = 64*j + lane with j = 4*i + wave: row r = 32*i + 8*wave + (lane >> 3), slot p = lane & 7,
  // logical chunk p ^ (r & 7) = (lane & 7) ^ (lane >> 3)  (r & 7 == lane >> 3).
  // B chunk s = 64*j + lane: row k = 8*i + 2*wave + (lane >> 5), slot p = lane & 31,
  // logical chunk p ^ 2*(k & 3) with k & 3 == (2*wave + (lane >> 5)) & 3.
  DmaLane d;
  d.a = 2u * static_cast<uint32_t>((lane >> 3) * K + (((lane & 7) ^ (lane >> 3)) * 8));
  d.b = 2u * static_cast<uint32_t>((lane >> 5) * N + (((lane & 31) ^ (((2 * wave + (lane >> 5)) & 3) << 1)) * 8));
  return d;
}

// global_load_lds_dwordx4: each lane copies 16 B from sbase + voff to LDS
// address m0 + 16*lane.  Written as inline asm so the compiler does not treat
// the copy as an LDS store it must wait for before every later LDS read; the
// kernel waits for the copies itself (vmcnt(0) + barrier) before reading a stage.
__device__ __forceinline__ void dma16(const uint16_t* sbase, uint32_t voff, uint32_t lds_addr) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_addr) : "memory");
}

__device__ __forceinline__ void dma_tile(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, int64_t N,
                                         int64_t K, int64_t m0, int64_t n0, int64_t k0, uint32_t stage, int wave,
                                         const DmaLane& d) {
#pragma unroll
  for (int i = 0; i < 8; ++i)  // A: wave-instruction j = 4i + wave fills LDS [1 KiB * j, +1 KiB) = rows 8j..8j+7
    dma16(A + (m0 + 32 * i + 8 * wave) * K + k0, d.a, stage + (4 * i + wave) * 1024);
#pragma unroll
  for (int i = 0; i < 8; ++i)  // B: wave-instruction j fills k-rows 2j, 2j+1 (512 B each)
    dma16(B + (k0 + 8 * i + 2 * wave) * N + n0, d.b, stage + kStageA + (4 * i + wave) * 1024);
}

struct Frags {
  bf16x8_t a[4], b[4];
};

// Per-lane LDS byte offsets of the fragment reads.  The wave covers A rows
// wm*128 + mi*32 + (lane & 31) and B columns wn*32 + ni*64 + (lane & 31), so mi
// and ni (and, for B, kk and the half t) become immediate offsets.
struct FragLane {
  int a[4];  // per kk
  int b;
};

__device__ __forceinline__ FragLane frag_lane(int wm, int wn, int lane) {
  FragLane f;
  const int r = wm * 128 + (lane & 31);
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) f.a[kk] = r * 128 + (((2 * kk + (lane >> 5)) ^ (lane & 7)) * 16);
  const int g = lane >> 4, i = lane & 15;
  const int khalf = g >> 1, nsub = g & 1;
  const int k = khalf * 8 + (i >> 2);                       // + 16*kk + 4*t
  const int n = wn * 32 + nsub * 16 + 4 * (i & 3);          // + 64*ni
  const int p = (n >> 3) ^ ((i >> 2) << 1);                 // k & 3 == i >> 2
  f.b = kStageA + k * 512 + p * 16 + (n & 7) * 2;
  return f;
}

__device__ __forceinline__ void read_frags(const lds_char_t* stage, int kk, const FragLane& fl, Frags& f) {
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
    f.a[mi] = *reinterpret_cast<const __attribute__((address_space(3))) bf16x8_t*>(stage + fl.a[kk] + mi * 32 * 128);
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) {
    i16x4_t part[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
      part[t] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_i16x4_t*)(stage + fl.b + (kk * 16 + t * 4) * 512 + ni * 128));
    const i16x8_t both = {part[0][0], part[0][1], part[0][2], part[0][3], part[1][0], part[1][1], part[1][2], part[1][3]};
    f.b[ni] = __builtin_bit_cast(bf16x8_t, both);
  }
}

__device__ __forceinline__ void mfma_stage(const lds_char_t* cur, const FragLane& fl, f32x16_t (&acc)[4][4]) {
  Frags f[2];
  read_frags(cur, 0, fl, f[0]);
#pragma unroll
  for (int kk = 0; kk < kBK / 16; ++kk) {
    if (kk + 1 < kBK / 16) read_frags(cur, kk + 1, fl, f[(kk + 1) & 1]);
    const Frags& fc = f[kk & 1];
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
        acc[ni][mi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fc.b[ni], fc.a[mi], acc[ni][mi], 0, 0, 0);
  }
}

// Waits for this wave's outstanding direct-to-LDS copies, then for every wave.
__device__ __forceinline__ void stage_barrier() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_bf16_dma_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, const float* __restrict__ bias,
                          uint16_t* __restrict__ C, int64_t N, int64_t K, int relu, int tiles_m, int tiles_n) {
  __shared__ __attribute__((aligned(1024))) char lds_raw[2 * kStage];
  const lds_char_t* lds = (const lds_char_t*)lds_raw;
  const uint32_t lds_addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar address math
  const int wm = wave & 1, wn = wave >> 1;

  int bid = blockIdx.x;
  const int T = gridDim.x;
  if (T % kNumXcd == 0) bid = (bid % kNumXcd) * (T / kNumXcd) + bid / kNumXcd;
  const int per_group = kGroupM * tiles_n;
  const int g = bid / per_group, first_m = g * kGroupM;
  const int gsz = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int tm = first_m + (bid % per_group) % gsz, tn = (bid % per_group) / gsz;
  const int64_t m0 = static_cast<int64_t>(tm) * kBM, n0 = static_cast<int64_t>(tn) * kBN;

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16_t{};

  const DmaLane dl = dma_lane(N, K, wave, lane);
  const FragLane fl = frag_lane(wm, wn, lane);
  const int KT = static_cast<int>(K / kBK);
  if (KT > 0) dma_tile(A, B, N, K, m0, n0, 0, lds_addr, wave, dl);
  stage_barrier();
  for (int kt = 0; kt < KT; ++kt) {
    if (kt + 1 < KT)
      dma_tile(A, B, N, K, m0, n0, static_cast<int64_t>(kt + 1) * kBK, lds_addr + ((kt + 1) & 1) * kStage, wave, dl);
    mfma_stage(lds + (kt & 1) * kStage, fl, acc);
    stage_barrier();
  }

  // Epilogue, one 32x32 block at a time (the empty asm keeps the compiler from
  // pulling all 256 accumulators into VGPRs at once).
  const bool has_bias = bias != nullptr;
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) {
    float bv[4][4];
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int64_t n = n0 + wn * 32 + ni * 64 + g4 * 8 + (lane >> 5) * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) bv[g4][q] = has_bias ? bias[n + q] : 0.0f;
    }
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      const int64_t m = m0 + wm * 128 + mi * 32 + (lane & 31);
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int64_t n = n0 + wn * 32 + ni * 64 + g4 * 8 + (lane >> 5) * 4;
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float t = acc[ni][mi][g4 * 4 + q];
          if (has_bias) t = t + bv[g4][q];
          v[q] = relu ? relu_np(t) : t;
        }
        uint2 pk;
        pk.x = f32_to_bf16_rne(v[0]) | (uint32_t(f32_to_bf16_rne(v[1])) << 16);
        pk.y = f32_to_bf16_rne(v[2]) | (uint32_t(f32_to_bf16_rne(v[3])) << 16);
        *reinterpret_cast<uint2*>(C + m * N + n) = pk;
      }
      asm volatile("" ::: "memory");
    }
  }
}

hipError_t launch_gemm_bf16_bias_relu(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                                      int64_t N, int64_t K, int relu, hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  const int64_t tm = (M + kBM - 1) / kBM, tn = (N + kBN - 1) / kBN;
  if (tm * tn > 0x7fffffffLL) return hipErrorInvalidValue;
  const uintptr_t al = reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B) | reinterpret_cast<uintptr_t>(C);
  const bool fast = (M % kBM == 0) && (N % kBN == 0) && (K % kBK == 0) && ((al & 15) == 0);
  const dim3 grid(static_cast<unsigned>(tm * tn)), block(256);
  if (fast)
    gemm_bf16_dma_kernel<<<grid, block, 0, s>>>(A, B, bias, C, N, K, relu, static_cast<int>(tm), static_cast<int>(tn));
  else
    gemm_bf16_bias_relu_kernel<true><<<grid, block, 0, s>>>(A, B, bias, C, M, N, K, relu, static_cast<int>(tm),
                                                            static_cast<int>(tn));
  return hipGetLastError();
}

}  // namespace ihip
