// bf16 GEMM in 256x256 tiles on v_mfma_f32_16x16x32_bf16 (C = act(A @ B + bias),
// A [M, K] row-major, B [K, N] or, transposed, [N, K]; f32 accumulation; C bf16, round to
// nearest even).
//
// Why 16x16x32 MFMAs: on random operands the chip runs at its power limit, so the clock, and
// with it the throughput, follows the energy per FLOP.  The 16x16x32 form reads 4 accumulator
// registers per 16 cycles where the 32x32x16 form reads 16 per 32 cycles (half the accumulator
// traffic per FLOP): register-only MFMA loops on random bf16 data run at about 2.1 GHz against
// 1.83 GHz, and this kernel at 1.89 GHz against 1.65 GHz for the same tile schedule with the
// 32x32x16 form (`rocm-smi -c` during back-to-back launches).  The sums come out bit-identical
// to the 32x32x16 kernels' (same k order over 16-k halves, f32 accumulation).
//
// Tile schedule: 256x256 tiles, each computed by a workgroup of four waves (2 x 2), each wave a
// 128x128 block held as 8 x 8 accumulators of 16x16 (256 AGPRs, one wave per SIMD).  The grid
// is persistent, one workgroup per CU taking tiles in turn (a tile's stores drain while the
// next tile's first slices load, and no workgroup is launched per tile).  K runs in 64-k
// slices; LDS holds three A slices and two B slices (5 x 32 KiB); one barrier per slice.
// A slice is two 32-k steps of 64 MFMAs; a step's fragments (8 A blocks, 8 B blocks) are read
// during the previous step, in its first six quarters (a quarter = 8 MFMAs), so that the last
// read has landed before the barrier that opens the next slice.
//
// Shapes: any M, N % 8 == 0, K % 64 == 0 (K >= 64), A, B and C 16-byte aligned, and the 32-bit
// per-lane copy offsets in range (K * 512 and N * 128 below 2^32); the dispatcher sends
// everything else to gemm_fast.hip.  M or N not a multiple of 256 leaves edge tiles, which copy
// through range-checked descriptors and mask their stores (the EDGE kernel below).
//
// Layout in a stage: A as [256 rows][64 k], 128-byte rows; B given as [K, N] as [64 k][256 n],
// 512-byte rows; B given as [N, K] as [256 n][64 k] like A.  Copies are gfx950 direct-to-LDS
// loads (global_load_lds_dwordx4: lane l of a wave writes 16 bytes at m0 + 16 l), so bank
// conflicts are avoided by choosing which global chunk a lane fetches (XOR swizzles over the
// 64 banks): a 128-byte row r holds logical 16-byte chunk c in slot c ^ ((r / 2) % 8); a 512-byte
// k-row holds logical n-chunk c in slot c ^ 2 (k & 3) ^ 8 ((c / 2) & 1) ^ 8 ((k / 8) & 1).
// Fragments of 16x16x32: lane l holds row (or column) l & 15 and k 8 (l >> 4) .. +7 of a 32-k
// step; A (and a K-contiguous B) with ds_read_b128, a K-major B with two ds_read_b64_tr_b16 per
// block (each 16-lane group reads a 4 k x 16 n block; lane i receives column i).
// The MFMAs are issued as inline assembly with the accumulator pinned in AGPRs: through the
// builtin the register allocator moves some of the 64 accumulators through VGPRs
// (v_accvgpr_read/write pairs and wait states inside the loop).
#include "common.hpp"

#include <atomic>
#include <type_traits>

namespace ihip {
namespace m16 {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
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
constexpr int kOpBytes = kTile * kDK * 2;
constexpr int kRegionsA = 3;
constexpr int kStagesB = 2;
constexpr int kOffB = kRegionsA * kOpBytes;
constexpr int kRing = kOffB + kStagesB * kOpBytes;
constexpr int kCopies = kOpBytes / 1024 / 4;  // copy instructions per wave per operand per slice: 8
constexpr int kGroupRows = 8;
constexpr int kCPitch = kTile * 2 + 16;
constexpr int kLdsBytes = kTile * kCPitch + kTile * 4 > kRing ? kTile * kCPitch + kTile * 4 : kRing;
static_assert(kLdsBytes <= 160 * 1024, "LDS");

__device__ __forceinline__ int row_slot(int c, int r) { return c ^ ((r >> 1) & 7); }
// K-major slot: bit 3 also follows bit 3 of k, so that the two 16-lane groups one tr read
// serves together (k rows 8 apart, same columns) land on different halves of the banks.
__device__ __forceinline__ int kmaj_slot(int c, int k) {
  return c ^ ((k & 3) << 1) ^ (((c >> 1) & 1) << 3) ^ (((k >> 3) & 1) << 3);
}
// Inverse of kmaj_slot in c for a fixed k.
__device__ __forceinline__ int kmaj_logical(int p, int k) {
  const int x = p ^ ((k & 3) << 1) ^ (((k >> 3) & 1) << 3);
  return x ^ (((x >> 1) & 1) << 3);
}

__device__ __forceinline__ void dma16(const uint16_t* sbase, uint32_t voff, uint32_t lds_addr) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_addr) : "memory");
}

// Raw buffer descriptor over [base, end): loads at byte offsets past end - base return zero.
__device__ __forceinline__ i32x4_t rsrc_of(const uint16_t* base, const uint16_t* end) {
  const int64_t left = (end - base) * 2;
  const uint32_t records = left <= 0 ? 0u : left >= 0xffffffffll ? 0xffffffffu : static_cast<uint32_t>(left);
  const uint64_t addr = reinterpret_cast<uint64_t>(base);
  // word1: base address bits 47:32, stride 0; word3: 32-bit data format, raw (untyped) access
  return i32x4_t{static_cast<int>(addr & 0xffffffffu), static_cast<int>((addr >> 32) & 0xffffu),
                 static_cast<int>(records), 0x00020000};
}

// The direct-to-LDS copy through a descriptor, for tiles that reach past a tensor's last row.
__device__ __forceinline__ void dma16(const i32x4_t& rsrc, uint32_t voff, uint32_t lds_addr) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "{m0}"(lds_addr) : "memory");
}

template <int n>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory");
}

// Per-lane byte offsets of one operand's 8 copy instructions (from the slice's scalar base).
// Instruction j = 4i + wave copies 1 KiB: 8 rows of a K-contiguous operand (leading dim ld = K)
// or 2 k-rows of a K-major one (leading dim ld = N), each lane fetching the chunk its LDS slot
// holds under the swizzle.
template <bool kKMajor>
__device__ __forceinline__ void copy_offsets(int64_t ld, int wave, int lane, uint32_t (&off)[kCopies]) {
#pragma unroll
  for (int i = 0; i < kCopies; ++i) {
    const int j = 4 * i + wave;
    if (!kKMajor) {
      const int r = j * 8 + lane / 8;
      const int c = row_slot(lane % 8, r);
      off[i] = 2u * static_cast<uint32_t>(r * ld + c * 8);
    } else {
      const int k = j * 2 + lane / 32;
      off[i] = 2u * static_cast<uint32_t>(k * ld + kmaj_logical(lane % 32, k) * 8);
    }
  }
}

// One MFMA with the accumulator pinned in AGPRs (the register allocator otherwise moves some
// of the 64 accumulators through VGPRs).
__device__ __forceinline__ void mfma16(f32x4_t& acc, const bf16x8_t& a, const bf16x8_t& b) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// Orders AGPR reads after the MFMAs that write them: the compiler sees the inline-asm MFMA as a
// one-cycle instruction and would read an accumulator right behind it.  Redefining the
// accumulators here (after 24 wait states) makes every later read use the value this defines.
template <bool kWait>
__device__ __forceinline__ void acc_fence(f32x4_t (&a)[8]) {
  if constexpr (kWait)
    asm volatile("s_nop 7\n s_nop 7\n s_nop 7"
                 : "+a"(a[0]), "+a"(a[1]), "+a"(a[2]), "+a"(a[3]), "+a"(a[4]), "+a"(a[5]), "+a"(a[6]), "+a"(a[7]));
  else
    asm volatile(""
                 : "+a"(a[0]), "+a"(a[1]), "+a"(a[2]), "+a"(a[3]), "+a"(a[4]), "+a"(a[5]), "+a"(a[6]), "+a"(a[7]));
}

struct Frag {
  bf16x8_t a[8], b[8];
};

// LDS offsets of a wave's fragments.  K-contiguous operand, rows base + 16 blk + (lane & 15),
// k group g = lane >> 4 (8 k): step s reads chunk 4 s + g; blocks are 2048 bytes apart.
__device__ __forceinline__ void kc_offsets(int base, int lane, int (&o)[2]) {
  const int r = base + (lane & 15), g = lane >> 4;
#pragma unroll
  for (int s = 0; s < 2; ++s) o[s] = r * 128 + row_slot(4 * s + g, r) * 16;
}
// K-major B: block q, the tr read of k rows 8 g + 4 h + (i >> 2) (+32 s), columns
// base + 16 q + 4 (i & 3) .. +3, i = lane & 15.
__device__ __forceinline__ void km_offsets(int base, int lane, int (&o)[8]) {
  const int g = lane >> 4, i = lane & 15;
  const int k = 8 * g + (i >> 2);
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int x = base + 16 * q + 4 * (i & 3);
    o[q] = k * (kTile * 2) + kmaj_slot(x >> 3, k) * 16 + (x & 7) * 2;
  }
}

// Read slot `slot` of the fragments of 32-k step s (offsets from kc_offsets / km_offsets).  Order: B blocks first (the next step's
// first MFMAs need all of them), then A blocks.
template <bool BKM>
__device__ __forceinline__ void read_slot(const lds_char_t* sa, const lds_char_t* sb, int s, const int (&oa)[2],
                                          const int (&obc)[2], const int (&obk)[8], Frag& f, int slot) {
  constexpr int kB = BKM ? 16 : 8;
  if (slot >= kB) {
    const int blk = slot - kB;
    f.a[blk] = *(const lds_bf16x8_t*)(sa + oa[s] + blk * 2048);
  } else if (!BKM) {
    f.b[slot] = *(const lds_bf16x8_t*)(sb + obc[s] + slot * 2048);
  } else {
    const int q = slot >> 1, h = slot & 1;
    const i16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_i16x4_t*)(sb + obk[q] + (32 * s + 4 * h) * (kTile * 2)));
    i16x8_t w = __builtin_bit_cast(i16x8_t, f.b[q]);
    if (h == 0) {
      w[0] = v[0], w[1] = v[1], w[2] = v[2], w[3] = v[3];
    } else {
      w[4] = v[0], w[5] = v[1], w[6] = v[2], w[7] = v[3];
    }
    f.b[q] = __builtin_bit_cast(bf16x8_t, w);
  }
}

// EDGE: M or N not a multiple of 256.  Tiles that reach past the last row or column copy A and B
// through descriptors that end at the tensor (rows past it read zeros; B columns past N, within
// the tensor, read other columns' values, which only reach outputs that are not stored) and
// mask their stores; the other tiles run the plain copies.
template <bool BKM, bool RELU, bool EDGE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_bf16_m16_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                          const float* __restrict__ bias, uint16_t* __restrict__ C, int64_t M, int64_t N, int64_t K,
                          int tiles_m, int tiles_n) {
  constexpr int kSlots = BKM ? 24 : 16;  // LDS reads per 32-k step
  constexpr int kReadQ = 6;              // the reads go in the first 6 of a step's 8 quarters
  constexpr int kPre = 2;
  __shared__ __attribute__((aligned(1024))) char lds_raw[kLdsBytes];
  const lds_char_t* lds = (const lds_char_t*)lds_raw;
  const uint32_t lds_addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave & 1, wn = wave >> 1;

  uint32_t ca[kCopies], cb[kCopies];
  copy_offsets<false>(K, wave, lane, ca);
  copy_offsets<BKM>(BKM ? N : K, wave, lane, cb);
  int oa[2], obc[2], obk[8];
  kc_offsets(wm * 128, lane, oa);
  if constexpr (BKM)
    km_offsets(wn * 128, lane, obk);
  else
    kc_offsets(wn * 128, lane, obc);

  // Persistent grid: workgroup b takes virtual tiles b, b + G, b + 2G, ...; a virtual tile v runs
  // on XCD v % 8 as a non-persistent launch's block v would, and maps to the same tile.
  const int tiles = tiles_m * tiles_n;
  for (int v = blockIdx.x; v < tiles; v += gridDim.x) {
    const int bid = xcd_contiguous(v, tiles);
    const int per_group = kGroupRows * tiles_n;
    const int grp = bid / per_group, first_m = grp * kGroupRows;
    const int gsz = (tiles_m - first_m) < kGroupRows ? (tiles_m - first_m) : kGroupRows;
    const int tm = first_m + (bid % per_group) % gsz, tn = (bid % per_group) / gsz;
    const int64_t m0 = static_cast<int64_t>(tm) * kTile, n0 = static_cast<int64_t>(tn) * kTile;
    const float bias_v = threadIdx.x < kTile && bias != nullptr && (!EDGE || n0 + threadIdx.x < N)
                             ? bias[n0 + threadIdx.x]
                             : 0.0f;

    const uint16_t* const a_rows = A + m0 * K;
    const uint16_t* const b_base = BKM ? B + n0 : B + n0 * K;
    auto tile = [&](auto edge_tag) {
      constexpr bool kEdge = decltype(edge_tag)::value;
      auto copy_a = [&](int s, int ra, int c) {
        const uint16_t* const base = a_rows + static_cast<int64_t>(s) * kDK;
        const uint32_t dst = lds_addr + ra * kOpBytes + (4 * c + wave) * 1024;
        if constexpr (kEdge)
          dma16(rsrc_of(base, A + M * K), ca[c], dst);
        else
          dma16(base, ca[c], dst);
      };
      auto copy_b = [&](int s, int c) {
        const int64_t k0 = static_cast<int64_t>(s) * kDK;
        const uint16_t* const base = BKM ? b_base + k0 * N : b_base + k0;
        const uint32_t dst = lds_addr + kOffB + (s & 1) * kOpBytes + (4 * c + wave) * 1024;
        if constexpr (kEdge)
          dma16(rsrc_of(base, B + K * N), cb[c], dst);
        else
          dma16(base, cb[c], dst);
      };

      f32x4_t acc[8][8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = f32x4_t{};
      acc_fence<true>(acc[0]);
#pragma unroll
      for (int i = 1; i < 8; ++i) acc_fence<false>(acc[i]);

      const int KT = static_cast<int>(K / kDK);
#pragma unroll
      for (int c = 0; c < kCopies; ++c) copy_a(0, 0, c);
#pragma unroll
      for (int c = 0; c < kCopies; ++c) copy_b(0, c);
      if (KT > 1) {
#pragma unroll
        for (int c = 0; c < kCopies; ++c) copy_a(1, 1, c);
#pragma unroll
        for (int c = 0; c < kCopies; ++c) copy_b(1, c);
        wait_vm<2 * kCopies>();
      } else {
        wait_vm<0>();
      }
      __syncthreads();
      Frag f[2];
#pragma unroll
      for (int sl = 0; sl < kSlots; ++sl) read_slot<BKM>(lds, lds + kOffB, 0, oa, obc, obk, f[0], sl);

      // Copy schedule per slice kt (16 quarters of 8 MFMAs): quarters 0-7 copy A slice kt+2 into
      // the region slice kt-1 used; quarters 8-15, after the barrier that closes slice kt (start of
      // quarter 8), copy B slice kt+2 into the stage slice kt used.  The barrier waits for A and B
      // of slice kt+1 (issued during slice kt-1): only A slice kt+2's copies were issued since.
      auto slice = [&](int kt, int ra, auto more_tag, auto more2_tag) {
        constexpr bool kMore = decltype(more_tag)::value;
        constexpr bool kMore2 = decltype(more2_tag)::value;
        const int ra1 = ra == kRegionsA - 1 ? 0 : ra + 1, ra2 = ra1 == kRegionsA - 1 ? 0 : ra1 + 1;
        const lds_char_t* sa = lds + ra * kOpBytes;
        const lds_char_t* sb = lds + kOffB + (kt & 1) * kOpBytes;
        const lds_char_t* na = lds + ra1 * kOpBytes;
        const lds_char_t* nb = lds + kOffB + ((kt + 1) & 1) * kOpBytes;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          Frag& cur = f[s];
          Frag& nxt = f[s ^ 1];
          const bool last = s == 1;
          const bool rd = !last || kMore;
          const lds_char_t* rda = last ? na : sa;
          const lds_char_t* rdb = last ? nb : sb;
          const int rs = last ? 0 : 1;
#pragma unroll
          for (int mi = 0; mi < 8; ++mi) {
            __builtin_amdgcn_sched_barrier(0);
            const bool pre = last && mi == 0 && kMore;
            if (pre) {
#pragma unroll
              for (int q = 0; q < kPre; ++q)
                mfma16(acc[mi][q], cur.b[q], cur.a[mi]);
              if constexpr (kMore2)
                wait_vm<kCopies>();
              else
                wait_vm<0>();
              __syncthreads();
              __builtin_amdgcn_sched_barrier(0);
            }
            const int from = pre ? kPre : 0;
            // fixed order: MFMA, LDS read, MFMA, LDS read, ..., each fenced so that the scheduler
            // keeps one live range per accumulator
#pragma unroll
            for (int q = 0; q < 8; ++q) {
              if (q >= from) {
                mfma16(acc[mi][q], cur.b[q], cur.a[mi]);
                __builtin_amdgcn_sched_barrier(0);
              }
              const int r = q - from;
              const int lo = mi < kReadQ ? mi * kSlots / kReadQ : kSlots;
              const int hi = mi < kReadQ ? (mi + 1) * kSlots / kReadQ : kSlots;
              if (rd && r >= 0 && lo + r < hi) {
                read_slot<BKM>(rda, rdb, rs, oa, obc, obk, nxt, lo + r);
                __builtin_amdgcn_sched_barrier(0);
              }
            }
            const int qi = s * 8 + mi;
            if (kMore2) {
              __builtin_amdgcn_sched_barrier(0);
              if (qi < 8)
                copy_a(kt + 2, ra2, qi);
              else
                copy_b(kt + 2, qi - 8);
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
      acc_fence<true>(acc[0]);
#pragma unroll
      for (int i = 1; i < 8; ++i) acc_fence<false>(acc[i]);
      __syncthreads();
      float* bias_lds = reinterpret_cast<float*>(lds_raw + kTile * kCPitch);
      if (threadIdx.x < kTile) bias_lds[threadIdx.x] = bias_v;
      __syncthreads();
      typedef __attribute__((address_space(3))) char lds_wchar_t;
      lds_wchar_t* ct = (lds_wchar_t*)lds_raw;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int nl = wn * 128 + q * 16 + (lane >> 4) * 4;
        const f32x4_t bv = *reinterpret_cast<const f32x4_t*>(&bias_lds[nl]);
#pragma unroll
        for (int mi = 0; mi < 8; ++mi) {
          const int ml = wm * 128 + mi * 16 + (lane & 15);
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = acc[mi][q][e] + bv[e];
            if constexpr (RELU) v[e] = __builtin_elementwise_maximum(v[e], 0.0f);
          }
          const bf16x2_t lo = {static_cast<__bf16>(v[0]), static_cast<__bf16>(v[1])};
          const bf16x2_t hi = {static_cast<__bf16>(v[2]), static_cast<__bf16>(v[3])};
          const u32x2 pk = {__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
          *(lds_u32x2_t*)(ct + ml * kCPitch + nl * 2) = pk;
        }
        asm volatile("" ::: "memory");
      }
      __syncthreads();
      constexpr int kLanesPerRow = kTile / 8, kRowsPerStore = 64 / kLanesPerRow;
      const int chunk = lane % kLanesPerRow;
#pragma unroll 4
      for (int i = 0; i < kTile / (4 * kRowsPerStore); ++i) {
        const int row = (i * 4 + wave) * kRowsPerStore + lane / kLanesPerRow;
        const u32x4 v = *(const lds_u32x4_t*)(ct + row * kCPitch + chunk * 16);
        if (!kEdge || (m0 + row < M && n0 + chunk * 8 < N))
          *reinterpret_cast<u32x4*>(C + (m0 + row) * N + n0 + chunk * 8) = v;
      }
    };
    if constexpr (EDGE) {
      if (m0 + kTile > M || n0 + kTile > N)
        tile(std::true_type{});
      else
        tile(std::false_type{});
    } else {
      tile(std::false_type{});
    }
    // every wave has read its rows of the staged tile before the next tile's copies land in LDS
    __syncthreads();
  }
}

// Compute units of the current device, looked up once per device.
int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev < 64) cached[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

}  // namespace m16

// True when this kernel takes the launch: K a multiple of 64, N of 8 (16-byte rows of B and C),
// A given as [M, K], 16-byte aligned tensors, 32-bit copy offsets, and at most 2^30 tiles (the
// persistent loop's tile index plus the grid size stays within int).
bool gemm_m16_fits(int64_t M, int64_t N, int64_t K, bool transpose_a, const void* A, const void* B, const void* C) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B) | reinterpret_cast<uintptr_t>(C);
  const int64_t lim = int64_t(1) << 32;
  const int64_t tm = (M + m16::kTile - 1) / m16::kTile, tn = (N + m16::kTile - 1) / m16::kTile;
  return !transpose_a && M > 0 && N > 0 && K >= m16::kDK && N % 8 == 0 && K % m16::kDK == 0 && (al & 15) == 0 &&
         K * 512 < lim && N * 128 < lim && tm * tn <= (int64_t(1) << 30);
}

hipError_t launch_gemm_m16(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M, int64_t N,
                           int64_t K, bool transpose_b, int relu, hipStream_t s) {
  const int tm = static_cast<int>((M + m16::kTile - 1) / m16::kTile), tn = static_cast<int>((N + m16::kTile - 1) / m16::kTile);
  const bool edge = M % m16::kTile != 0 || N % m16::kTile != 0;
  const int64_t tiles = static_cast<int64_t>(tm) * tn;
  const int cus = m16::device_cus();
  if (cus <= 0) return hipErrorInvalidDevice;
  // one workgroup per CU (the kernel holds all of a CU's LDS and registers)
  const dim3 grid(static_cast<unsigned>(tiles < cus ? tiles : cus)), block(256);
#define IHIP_M16_LAUNCH(BKM, RELU, EDGE) \
  m16::gemm_bf16_m16_kernel<BKM, RELU, EDGE><<<grid, block, 0, s>>>(A, B, bias, C, M, N, K, tm, tn)
  if (transpose_b) {
    if (relu)
      edge ? IHIP_M16_LAUNCH(false, true, true) : IHIP_M16_LAUNCH(false, true, false);
    else
      edge ? IHIP_M16_LAUNCH(false, false, true) : IHIP_M16_LAUNCH(false, false, false);
  } else {
    if (relu)
      edge ? IHIP_M16_LAUNCH(true, true, true) : IHIP_M16_LAUNCH(true, true, false);
    else
      edge ? IHIP_M16_LAUNCH(true, false, true) : IHIP_M16_LAUNCH(true, false, false);
  }
#undef IHIP_M16_LAUNCH
  return hipGetLastError();
}

}  // namespace ihip
