// bf16 GEMM for whole 256x256 tiles with 64-k slices in two LDS stages (C = act(A @ B + bias),
// A [M, K] row-major, B [K, N] or, transposed, [N, K]; f32 accumulation on
// v_mfma_f32_32x32x16_bf16; C bf16, round to nearest even).
//
// Why a second tiled kernel: with one wave per SIMD (the 256 f32 accumulators of a 128x128
// wave tile fill the register file), every workgroup barrier leaves the matrix pipe idle while
// the wave waits.  gemm_fast.hip keeps a ring of 32-k slices and passes one barrier per slice,
// 1024 cycles of MFMA work.  Here a slice is 64 k (2048 MFMA cycles): the LDS holds three
// slices of A and two of B (5 x 32 KiB), one barrier per slice.  A slice's stage is free once
// the barrier that closes the slice has passed (every wave has read its fragments), and is
// refilled with the slice two ahead: A (whose 256 row panels miss L2 more often than B's
// columns) during the first quarter of the following slice, B right after the barrier.
//
// Shapes: M % 256 == 0, N % 256 == 0, K % 64 == 0 (K >= 64), A, B and C 16-byte aligned, and
// the 32-bit per-lane copy offsets in range (K * 512 and N * 128 below 2^32); the dispatcher
// sends everything else to gemm_fast.hip.  The k order of every C element is that of
// gemm_fast.hip (16-k MFMA steps in ascending k), so both kernels give identical results.
//
// Layout in a stage: A as [256 rows][64 k], 128-byte rows; B given as [K, N] as [64 k][256 n],
// 512-byte rows; B given as [N, K] as [256 n][64 k] like A.  Copies are gfx950 direct-to-LDS
// loads (global_load_lds_dwordx4: lane l of a wave writes 16 bytes at m0 + 16 l), so bank
// conflicts are avoided by choosing which global chunk a lane fetches (XOR swizzles over the
// 64 banks): a 128-byte row r holds logical 16-byte chunk c in slot c ^ ((r / 2) % 8); a 512-byte
// k-row holds logical n-chunk c in slot c ^ 2 (k & 3) ^ 8 ((c / 2) & 1), so that one
// ds_read_b64_tr_b16 cycle (4 k-rows x 2 column groups) lands on 8 distinct 32-byte windows.
// Fragments: A (and a K-contiguous B) with ds_read_b128, a K-major B with two
// ds_read_b64_tr_b16 per block (lane i of a 16-lane group receives column i of 4 k-rows).
#include "common.hpp"

#include <type_traits>

namespace ihip {
namespace db {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
typedef __attribute__((address_space(3))) bf16x8_t lds_bf16x8_t;
typedef __attribute__((address_space(3))) char lds_char_t;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2_t;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4_t;

constexpr int kTile = 256;
constexpr int kDK = 64;
constexpr int kOpBytes = kTile * kDK * 2;     // one operand's slice: 32 KiB
constexpr int kRegionsA = 3;                  // A slices in LDS (ring of three)
constexpr int kStagesB = 2;                   // B slices in LDS (double buffer)
constexpr int kOffB = kRegionsA * kOpBytes;   // B stages after the A regions
constexpr int kRing = kOffB + kStagesB * kOpBytes;
constexpr int kCopies = kOpBytes / 1024 / 4;  // copy instructions per wave per operand per slice: 8
constexpr int kGroupRows = 8;                 // tile-rows per raster group
constexpr int kCPitch = kTile * 2 + 16;       // bytes per staged C row
constexpr int kLdsBytes = kTile * kCPitch + kTile * 4 > kRing ? kTile * kCPitch + kTile * 4 : kRing;
static_assert(kLdsBytes <= 160 * 1024, "LDS");

// Slot of logical 16-byte chunk c in 128-byte row r, and of logical n-chunk c in k-row k.
__device__ __forceinline__ int row_slot(int c, int r) { return c ^ ((r >> 1) & 7); }
__device__ __forceinline__ int kmaj_slot(int c, int k) { return c ^ ((k & 3) << 1) ^ (((c >> 1) & 1) << 3); }
// Inverse of kmaj_slot in c for a fixed k.
__device__ __forceinline__ int kmaj_logical(int p, int k) {
  const int x = p ^ ((k & 3) << 1);
  return x ^ (((x >> 1) & 1) << 3);
}

__device__ __forceinline__ void dma16(const uint16_t* sbase, uint32_t voff, uint32_t lds_addr) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_addr) : "memory");
}

template <int n>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory");
}

// Per-lane byte offsets of one operand's 8 copy instructions (from the slice's scalar base).
// Instruction j = 4i + wave copies 1 KiB: 8 rows of a K-contiguous operand (leading dim ld = K)
// or 2 k-rows of a K-major one (leading dim ld = N).  The swizzle term depends on j only
// through j & 1 = wave & 1 (K-contiguous) or through (2j) & 3 = 2 (wave & 1) (K-major).
template <bool kKMajor>
__device__ __forceinline__ void copy_offsets(int64_t ld, int wave, int lane, uint32_t (&off)[kCopies]) {
#pragma unroll
  for (int i = 0; i < kCopies; ++i) {
    const int j = 4 * i + wave;
    if (!kKMajor) {
      const int r = j * 8 + lane / 8;
      const int c = row_slot(lane % 8, r);  // row_slot is its own inverse in c
      off[i] = 2u * static_cast<uint32_t>(r * ld + c * 8);
    } else {
      const int k = j * 2 + lane / 32;
      off[i] = 2u * static_cast<uint32_t>(k * ld + kmaj_logical(lane % 32, k) * 8);
    }
  }
}

// Fragment LDS offsets (within an operand's slice).  K-contiguous: per 16-k step kk, block 0 of
// rows base + (lane & 31), chunk 2 kk + lane / 32 (blocks `step` rows apart share the swizzle
// term since step / 2 % 8 == 0).  K-major: per block, the tr-read address of k-row
// (g / 2) * 8 + i / 4 (k-step 0), columns base + blk * step + (g & 1) * 16 + 4 (i & 3).
template <bool kKMajor>
__device__ __forceinline__ void frag_offsets(int base, int step, int lane, int (&o)[4]) {
  if (!kKMajor) {
    const int r = base + (lane & 31);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) o[kk] = r * 128 + row_slot(2 * kk + (lane >> 5), r) * 16;
  } else {
    const int g = lane >> 4, i = lane & 15;
    const int k = (g >> 1) * 8 + (i >> 2);
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const int x = base + blk * step + (g & 1) * 16 + 4 * (i & 3);
      o[blk] = k * (kTile * 2) + kmaj_slot(x >> 3, k) * 16 + (x & 7) * 2;
    }
  }
}

struct Frag {
  bf16x8_t a[4], b[4];
};

// LDS read `slot` of one 16-k step: A's 4 ds_read_b128 first, then B's (4 ds_read_b128, or
// 8 ds_read_b64_tr_b16: two per block, the low and high 4 k).
template <bool BKM>
__device__ __forceinline__ void read_slot(const lds_char_t* sa, const lds_char_t* sb, int kk, const int (&oa)[4],
                                          const int (&ob)[4], Frag& f, int slot) {
  if (slot < 4) {
    f.a[slot] = *(const lds_bf16x8_t*)(sa + oa[kk] + slot * 32 * 128);
  } else if (!BKM) {
    const int blk = slot - 4;
    f.b[blk] = *(const lds_bf16x8_t*)(sb + ob[kk] + blk * 64 * 128);
  } else {
    const int blk = (slot - 4) >> 1, half = (slot - 4) & 1;
    const i16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_i16x4_t*)(sb + ob[blk] + (kk * 16 + half * 4) * (kTile * 2)));
    i16x8_t w = __builtin_bit_cast(i16x8_t, f.b[blk]);
    if (half == 0) {
      w[0] = v[0], w[1] = v[1], w[2] = v[2], w[3] = v[3];
    } else {
      w[4] = v[0], w[5] = v[1], w[6] = v[2], w[7] = v[3];
    }
    f.b[blk] = __builtin_bit_cast(bf16x8_t, w);
  }
}

template <bool BKM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_bf16_db64_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                           const float* __restrict__ bias, uint16_t* __restrict__ C, int64_t M, int64_t N, int64_t K,
                           int relu, int tiles_m, int tiles_n) {
  constexpr int kSlots = BKM ? 12 : 8;  // LDS reads per 16-k step
  constexpr int kPerQ = kSlots / 4;     // ... per quarter (4 MFMAs)
  constexpr int kPre = 1;               // MFMAs issued before the slice's closing barrier
  __shared__ __attribute__((aligned(1024))) char lds_raw[kLdsBytes];
  const lds_char_t* lds = (const lds_char_t*)lds_raw;
  const uint32_t lds_addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));

  // tile schedule: XCD-contiguous, then 8 tile-rows at a time, column by column
  const int bid = xcd_contiguous(blockIdx.x, gridDim.x);
  const int per_group = kGroupRows * tiles_n;
  const int grp = bid / per_group, first_m = grp * kGroupRows;
  const int gsz = (tiles_m - first_m) < kGroupRows ? (tiles_m - first_m) : kGroupRows;
  const int tm = first_m + (bid % per_group) % gsz, tn = (bid % per_group) / gsz;
  const int64_t m0 = static_cast<int64_t>(tm) * kTile, n0 = static_cast<int64_t>(tn) * kTile;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const float bias_v = threadIdx.x < kTile && bias != nullptr ? bias[n0 + threadIdx.x] : 0.0f;

  uint32_t ca[kCopies], cb[kCopies];
  copy_offsets<false>(K, wave, lane, ca);
  copy_offsets<BKM>(BKM ? N : K, wave, lane, cb);
  int oa[4], ob[4];
  frag_offsets<false>(wm * 128, 32, lane, oa);
  frag_offsets<BKM>(wn * 32, 64, lane, ob);

  const uint16_t* const a_rows = A + m0 * K;
  const uint16_t* const b_base = BKM ? B + n0 : B + n0 * K;
  // copy instruction c (0 .. 7) of A slice s into region ra, of B slice s into stage s & 1
  auto copy_a = [&](int s, int ra, int c) {
    dma16(a_rows + static_cast<int64_t>(s) * kDK, ca[c], lds_addr + ra * kOpBytes + (4 * c + wave) * 1024);
  };
  auto copy_b = [&](int s, int c) {
    const int64_t k0 = static_cast<int64_t>(s) * kDK;
    dma16(BKM ? b_base + k0 * N : b_base + k0, cb[c], lds_addr + kOffB + (s & 1) * kOpBytes + (4 * c + wave) * 1024);
  };

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16_t{};

  // Copy schedule: one copy instruction per quarter of 4 MFMAs, so that the LDS writes of the
  // copies never pile onto the fragment reads.  Quarters 0-15 of slice kt (4 per 16-k step):
  //   0-3:   B slice kt+1, its second half (the first half went right after slice kt-1 closed);
  //   4-11:  A slice kt+2, into the A region slice kt-1 used;
  //   12-15: B slice kt+2, its first half, into the B stage slice kt used, after the barrier
  //          that closes slice kt (quarter 12).
  // That barrier waits for A and B of slice kt+1: copies complete in issue order, and only A
  // slice kt+2's 8 instructions were issued after them.
  const int KT = static_cast<int>(K / kDK);
  // prologue: slice 0, then A of slice 1 and the first half of B of slice 1
#pragma unroll
  for (int c = 0; c < kCopies; ++c) copy_a(0, 0, c);
#pragma unroll
  for (int c = 0; c < kCopies; ++c) copy_b(0, c);
  if (KT > 1) {
#pragma unroll
    for (int c = 0; c < kCopies; ++c) copy_a(1, 1, c);
#pragma unroll
    for (int c = 0; c < kCopies / 2; ++c) copy_b(1, c);
    wait_vm<kCopies + kCopies / 2>();
  } else {
    wait_vm<0>();
  }
  __syncthreads();
  Frag f[2];
#pragma unroll
  for (int sl = 0; sl < kSlots; ++sl) read_slot<BKM>(lds, lds + kOffB, 0, oa, ob, f[0], sl);

  // One 64-k slice.  ra: its A region (kt % 3).  kMore: slice kt+1 exists (the slice closes with
  // the barrier and reads slice kt+1's first fragments); kMore2: slice kt+2 exists (the slice
  // copies it).  Straight-line code per slice keeps the MFMA / LDS-read interleave in one region.
  auto slice = [&](int kt, int ra, auto more_tag, auto more2_tag) {
    constexpr bool kMore = decltype(more_tag)::value;
    constexpr bool kMore2 = decltype(more2_tag)::value;
    const int ra1 = ra == kRegionsA - 1 ? 0 : ra + 1, ra2 = ra1 == kRegionsA - 1 ? 0 : ra1 + 1;
    const lds_char_t* sa = lds + ra * kOpBytes;
    const lds_char_t* sb = lds + kOffB + (kt & 1) * kOpBytes;
    const lds_char_t* na = lds + ra1 * kOpBytes;
    const lds_char_t* nb = lds + kOffB + ((kt + 1) & 1) * kOpBytes;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      Frag& cur = f[kk & 1];
      Frag& nxt = f[(kk & 1) ^ 1];
      const bool last = kk == 3;
      const bool rd = !last || kMore;  // a next step exists
      const lds_char_t* rda = last ? na : sa;
      const lds_char_t* rdb = last ? nb : sb;
      const int rk = last ? 0 : kk + 1;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        __builtin_amdgcn_sched_barrier(0);
        const bool pre = last && q == 0 && kMore;
        if (pre) {  // close the slice: this wave's copies of slice kt+1 have landed, then the barrier
#pragma unroll
          for (int mi = 0; mi < kPre; ++mi)
            acc[0][mi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur.b[0], cur.a[mi], acc[0][mi], 0, 0, 0);
          if constexpr (kMore2)
            wait_vm<kCopies>();
          else
            wait_vm<0>();
          __syncthreads();
          __builtin_amdgcn_sched_barrier(0);
        }
        const int from = pre ? kPre : 0;
        if (rd) {
#pragma unroll
          for (int r = 0; r < kPerQ; ++r) read_slot<BKM>(rda, rdb, rk, oa, ob, nxt, q * kPerQ + r);
        }
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
          if (mi >= from)
            acc[q][mi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur.b[q], cur.a[mi], acc[q][mi], 0, 0, 0);
        if (rd) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (j < 4 - from) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            if (j < kPerQ) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     // one LDS read
          }
        }
        const int qi = kk * 4 + q;
        if (kMore && qi < 4) {  // B slice kt+1, second half
          __builtin_amdgcn_sched_barrier(0);
          copy_b(kt + 1, kCopies / 2 + qi);
        } else if (kMore2 && qi < 12) {  // A slice kt+2
          __builtin_amdgcn_sched_barrier(0);
          copy_a(kt + 2, ra2, qi - 4);
        } else if (kMore2) {  // B slice kt+2, first half (after the barrier of quarter 12)
          __builtin_amdgcn_sched_barrier(0);
          copy_b(kt + 2, qi - 12);
        }
      }
    }
  };
  int kt = 0, ra = 0;
  for (; kt + 2 < KT; ++kt) {
    slice(kt, ra, std::true_type{}, std::true_type{});
    ra = ra == kRegionsA - 1 ? 0 : ra + 1;
  }
  if (kt + 1 < KT) {
    slice(kt, ra, std::true_type{}, std::false_type{});
    ++kt;
    ra = ra == kRegionsA - 1 ? 0 : ra + 1;
  }
  slice(kt, ra, std::false_type{}, std::false_type{});

  // epilogue: bias + activation, the tile staged in LDS as bf16 rows, written out in 512-byte rows
  __syncthreads();
  float* bias_lds = reinterpret_cast<float*>(lds_raw + kTile * kCPitch);
  if (threadIdx.x < kTile) bias_lds[threadIdx.x] = bias_v;
  __syncthreads();
  typedef __attribute__((address_space(3))) char lds_wchar_t;
  lds_wchar_t* ct = (lds_wchar_t*)lds_raw;
  const float floor_v = relu ? 0.0f : -__builtin_inff();
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) {
    f32x4_t bv[4];
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4)
      bv[g4] = *reinterpret_cast<const f32x4_t*>(&bias_lds[wn * 32 + ni * 64 + g4 * 8 + (lane >> 5) * 4]);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      const int ml = wm * 128 + mi * 32 + (lane & 31);
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int nl = wn * 32 + ni * 64 + g4 * 8 + (lane >> 5) * 4;
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = __builtin_elementwise_maximum(acc[ni][mi][g4 * 4 + q] + bv[g4][q], floor_v);
        const bf16x2_t lo = {static_cast<__bf16>(v[0]), static_cast<__bf16>(v[1])};
        const bf16x2_t hi = {static_cast<__bf16>(v[2]), static_cast<__bf16>(v[3])};
        const u32x2 pk = {__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
        *(lds_u32x2_t*)(ct + ml * kCPitch + nl * 2) = pk;
      }
      asm volatile("" ::: "memory");
    }
  }
  __syncthreads();
  constexpr int kLanesPerRow = kTile / 8, kRowsPerStore = 64 / kLanesPerRow;
  const int chunk = lane % kLanesPerRow;
#pragma unroll 4
  for (int i = 0; i < kTile / (4 * kRowsPerStore); ++i) {
    const int row = (i * 4 + wave) * kRowsPerStore + lane / kLanesPerRow;
    const u32x4 v = *(const lds_u32x4_t*)(ct + row * kCPitch + chunk * 16);
    *reinterpret_cast<u32x4*>(C + (m0 + row) * N + n0 + chunk * 8) = v;
  }
}

}  // namespace db

// True when the double-buffered kernel takes this launch: whole tiles, K a multiple of 64, A
// given as [M, K], 16-byte aligned tensors, 32-bit copy offsets.
bool gemm_db64_fits(int64_t M, int64_t N, int64_t K, bool transpose_a, const void* A, const void* B, const void* C) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B) | reinterpret_cast<uintptr_t>(C);
  const int64_t lim = int64_t(1) << 32;
  return !transpose_a && M > 0 && N > 0 && K >= db::kDK && M % db::kTile == 0 && N % db::kTile == 0 &&
         K % db::kDK == 0 && (al & 15) == 0 && K * 512 < lim && N * 128 < lim &&
         (M / db::kTile) * (N / db::kTile) <= 0x7fffffffLL;
}

hipError_t launch_gemm_db64(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M, int64_t N,
                            int64_t K, bool transpose_b, int relu, hipStream_t s) {
  const int tm = static_cast<int>(M / db::kTile), tn = static_cast<int>(N / db::kTile);
  const dim3 grid(static_cast<unsigned>(tm) * static_cast<unsigned>(tn)), block(256);
  if (transpose_b)
    db::gemm_bf16_db64_kernel<false><<<grid, block, 0, s>>>(A, B, bias, C, M, N, K, relu, tm, tn);
  else
    db::gemm_bf16_db64_kernel<true><<<grid, block, 0, s>>>(A, B, bias, C, M, N, K, relu, tm, tn);
  return hipGetLastError();
}

}  // namespace ihip
