// Packed GEMM path: operands the tiled kernel cannot read in place (rows that do not start
// 16 bytes aligned: K % 8 != 0, N % 8 != 0 with B given as [K, N], M % 8 != 0 with A given as
// [K, M], or 2-byte aligned bases) are first copied into a caller workspace as K-contiguous
// rows of K8 = K rounded up to 8 elements, zero past K, and the tiled kernel then runs on the
// copies (A as [M, K8], B as [N, K8]; C rows that are not 16-byte aligned are written with
// 2-byte stores).  The zeros past K add exact zeros in the k slots the guarded kernel also
// fills with zeros, and both kernels issue the same MFMAs in the same k order, so the result
// is bit-identical to the guarded kernel's.
//
// Packing is one HBM pass per packed operand (read R x K, write R x K8 elements):
//  * a K-contiguous source (A [M, K], B [N, K]) is re-pitched row by row: each thread writes
//    8 consecutive elements (one 16-byte store) from 4-byte loads when every row starts
//    4-byte aligned (K even), else from 2-byte loads;
//  * a K-major source (A [K, M], B [K, N]) is transposed through LDS in 64 x 64 tiles, read
//    along source rows and written in 16-byte stores along destination rows.
//
// Split-K: when the output has too few tiles to occupy the CUs, K is cut into S segments, the
// tiled kernel runs (tile, segment) workgroups that write f32 partial sums into the workspace,
// and a reduce kernel adds the S partials in segment order, then bias and activation.  The
// result is deterministic; it differs from the unsplit kernel's only in the f32 summation
// order.
#include <algorithm>

#include "common.hpp"

namespace ihip {

bool gemm_fast_fits(int64_t M, int64_t N, int64_t K, bool transpose_a, bool transpose_b, const void* A, const void* B,
                    const void* C);
hipError_t launch_gemm_fast(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M, int64_t N,
                            int64_t K, bool transpose_a, bool transpose_b, int relu, int tile, hipStream_t s,
                            bool c_unaligned);
hipError_t launch_gemm_splitk(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                              int64_t N, int64_t K, bool transpose_a, bool transpose_b, int relu, int tile, int S,
                              int64_t kseg, float* P, int64_t ldp, hipStream_t s);
int gemm_fast_tile_extent(int64_t M, int64_t N);

namespace {

constexpr int64_t kWsAlign = 256;

int64_t round8(int64_t k) { return (k + 7) / 8 * 8; }
int64_t align_up(int64_t b) { return (b + kWsAlign - 1) / kWsAlign * kWsAlign; }

// Split rule.  Grids of 256x256 tiles (more than 128 of them) are not split.  For 128x128
// tiles the rule picks the S (segments of at least kSplitMinK k, at most 512 workgroups) of
// least estimated time, in integer nanoseconds:
//   tile-steps (tiles x 32-k steps) / rate(tiles x S)
//   + for S > 1: kSplitFixedNs (reduce launch) + S x M x ldp x 8 bytes (partials written and
//     read back) at kSplitBytesPerNs,
// where rate(G), tile-steps per microsecond with G workgroups, is interpolated from
// kSplitRate (measured on MI355X: the rate per workgroup falls as more CUs draw on the power
// budget and the shared caches) and, past 256 workgroups, scaled by the last wave's fill.
// Ties go to the smaller S.
constexpr int64_t kSplitMinK = 512;
constexpr int64_t kSplitMax = 1024;  // segments at most
constexpr int64_t kSplitMaxGrid = 512;
constexpr int64_t kSplitRate[5] = {0, 305, 533, 680, 800};  // at 0, 64, 128, 192, 256 workgroups
constexpr int64_t kSplitFixedNs = 3500;
constexpr int64_t kSplitBytesPerNs = 6000;

int64_t split_rate(int64_t G) {
  if (G >= 256) {
    const int64_t waves = (G + 255) / 256;
    return kSplitRate[4] * G / (waves * 256);
  }
  const int64_t i = G / 64, f = G % 64;
  return kSplitRate[i] + (kSplitRate[i + 1] - kSplitRate[i]) * f / 64;
}

int64_t split_cost_ns(int64_t tiles, int64_t M, int64_t N, int64_t K, int64_t S) {
  const int64_t rate = std::max<int64_t>(1, split_rate(tiles * S));
  int64_t ns = tiles * ((K + 31) / 32) * 1000 / rate;
  if (S > 1) ns += kSplitFixedNs + S * M * ((N + 3) / 4 * 4) * 8 / kSplitBytesPerNs;
  return ns;
}

struct SplitPlan {
  int S;         // segments (1: no split)
  int64_t kseg;  // k per segment, a multiple of 64 (the last segment may be shorter)
};

// splits: 0 = by the rule above, else the number asked for (at most one per 64 k, and at
// most kSplitMax).  tile: the C tile the launch uses (0: gemm_fast_tile_extent's choice); the
// rule splits grids of 128x128 tiles only.
SplitPlan plan_of(int64_t K, int64_t S) {
  S = std::max<int64_t>(1, std::min<int64_t>({S, (K + 63) / 64, kSplitMax}));
  const int64_t kseg = ((K + S - 1) / S + 63) / 64 * 64;
  return {static_cast<int>((K + kseg - 1) / kseg), kseg};
}

SplitPlan split_plan(int64_t M, int64_t N, int64_t K, int splits, int tile) {
  if (K <= 0) return {1, K};
  if (splits > 0) return plan_of(K, splits);
  if ((tile == 0 ? gemm_fast_tile_extent(M, N) : tile) != 128) return {1, K};
  const int64_t tiles = ((M + 127) / 128) * ((N + 127) / 128);
  const int64_t smax = std::max<int64_t>(1, std::min({K / kSplitMinK, kSplitMax, kSplitMaxGrid / tiles}));
  SplitPlan best = {1, K};
  int64_t best_ns = split_cost_ns(tiles, M, N, K, 1);
  for (int64_t s = 2; s <= smax; ++s) {
    const SplitPlan p = plan_of(K, s);
    const int64_t ns = split_cost_ns(tiles, M, N, K, p.S);
    if (ns < best_ns) best = p, best_ns = ns;
  }
  return best;
}

// f32 partials of a split: S planes of M rows of N rounded up to 4 floats.
int64_t split_ldp(int64_t N) { return (N + 3) / 4 * 4; }
int64_t split_bytes(int64_t M, int64_t N, int S) { return S > 1 ? align_up(S * M * split_ldp(N) * 4) : 0; }

// The tiled kernel on operands it reads in place, split by `plan` when the workspace (ws,
// ws_bytes) holds the partials, else unsplit.
hipError_t launch_tiled(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M, int64_t N,
                        int64_t K, bool ta, bool tb, int relu, int tile, bool c_unaligned, const SplitPlan& plan,
                        void* ws, int64_t ws_bytes, hipStream_t s) {
  if (plan.S > 1 && ws != nullptr && (reinterpret_cast<uintptr_t>(ws) & (kWsAlign - 1)) == 0 &&
      split_bytes(M, N, plan.S) <= ws_bytes)
    return launch_gemm_splitk(A, B, bias, C, M, N, K, ta, tb, relu, tile == 0 ? gemm_fast_tile_extent(M, N) : tile,
                              plan.S, plan.kseg, static_cast<float*>(ws), split_ldp(N), s);
  return launch_gemm_fast(A, B, bias, C, M, N, K, ta, tb, relu, tile, s, c_unaligned);
}

// Which operands the shape alone sends through a packed copy (pointer alignment aside).
bool shape_packs_a(int64_t M, int64_t K, bool ta) { return K % 8 != 0 || (ta && M % 8 != 0); }
bool shape_packs_b(int64_t N, int64_t K, bool tb) { return K % 8 != 0 || (!tb && N % 8 != 0); }

// dst [R, K8] from a K-contiguous src [R, K] (leading dimension K); kPairs: every row starts
// 4-byte aligned (K even, src 4-byte aligned), so pairs of elements load as one dword.
template <bool kPairs>
__global__ __launch_bounds__(256) void pack_rows_kc(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                    int64_t R, int64_t K, int64_t K8) {
  const int64_t chunks = K8 / 8;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= R * chunks) return;
  const int64_t r = t / chunks, k0 = (t % chunks) * 8;
  const uint16_t* s = src + r * K;
  uint32_t w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t k = k0 + 2 * e;
    if (kPairs) {  // K even: a pair is wholly inside the row or wholly past it
      w[e] = k < K ? *reinterpret_cast<const uint32_t*>(s + k) : 0u;
    } else {
      const uint32_t lo = k < K ? s[k] : 0u, hi = k + 1 < K ? s[k + 1] : 0u;
      w[e] = lo | (hi << 16);
    }
  }
  *reinterpret_cast<u32x4*>(dst + r * K8 + k0) = u32x4{w[0], w[1], w[2], w[3]};
}

// dst [R, K8] from a K-major src [K, R] (leading dimension R): 64 x 64 tiles through LDS.
// Reads go along src rows (4-byte loads when every row starts 4-byte aligned, kPairs), writes
// along dst rows in 16-byte stores, 8 lanes per 128-byte row piece.
constexpr int kT = 64;
template <bool kPairs>
__global__ __launch_bounds__(256) void pack_rows_km(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                    int64_t R, int64_t K, int64_t K8) {
  __shared__ uint16_t tile[kT][kT + 2];
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kT, k0 = static_cast<int64_t>(blockIdx.y) * kT;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // read: src row k0 + i holds r0 .. r0+63 contiguously
  if constexpr (kPairs) {
    const int c = 2 * (lane & 31);
    for (int i = 2 * w + (lane >> 5); i < kT; i += 8) {
      const int64_t k = k0 + i, r = r0 + c;
      uint32_t v = 0;
      if (k < K && r + 1 < R) {
        v = *reinterpret_cast<const uint32_t*>(src + k * R + r);
      } else if (k < K && r < R) {
        v = src[k * R + r];
      }
      tile[i][c] = static_cast<uint16_t>(v);
      tile[i][c + 1] = static_cast<uint16_t>(v >> 16);
    }
  } else {
    for (int i = w; i < kT; i += 4) {
      const int64_t k = k0 + i, r = r0 + lane;
      tile[i][lane] = (k < K && r < R) ? src[k * R + r] : 0;
    }
  }
  __syncthreads();
  // write: dst row r0 + i gets k0 .. k0+63 (zeros past K; K8, a multiple of 8, may end inside
  // the tile), 8 columns per lane
  const int c8 = lane & 7;
  for (int i = (lane >> 3) + 8 * w; i < kT; i += 32) {
    const int64_t r = r0 + i, k = k0 + 8 * c8;
    if (r < R && k < K8) {
      uint32_t q[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        q[e] = static_cast<uint32_t>(tile[8 * c8 + 2 * e][i]) | (static_cast<uint32_t>(tile[8 * c8 + 2 * e + 1][i]) << 16);
      *reinterpret_cast<u32x4*>(dst + r * K8 + k) = u32x4{q[0], q[1], q[2], q[3]};
    }
  }
}

hipError_t pack(const uint16_t* src, uint16_t* dst, int64_t R, int64_t K, bool kmajor, hipStream_t s) {
  const int64_t K8 = round8(K);
  if (!kmajor) {
    const int64_t threads = R * (K8 / 8);
    const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
    if (K % 2 == 0 && (reinterpret_cast<uintptr_t>(src) & 3) == 0)
      pack_rows_kc<true><<<grid, dim3(256), 0, s>>>(src, dst, R, K, K8);
    else
      pack_rows_kc<false><<<grid, dim3(256), 0, s>>>(src, dst, R, K, K8);
  } else {
    const dim3 grid(static_cast<unsigned>((R + kT - 1) / kT), static_cast<unsigned>((K8 + kT - 1) / kT));
    if (R % 2 == 0 && (reinterpret_cast<uintptr_t>(src) & 3) == 0)
      pack_rows_km<true><<<grid, dim3(256), 0, s>>>(src, dst, R, K, K8);
    else
      pack_rows_km<false><<<grid, dim3(256), 0, s>>>(src, dst, R, K, K8);
  }
  return hipGetLastError();
}

}  // namespace

// Workspace bytes for this shape: the packed copies it needs, then the split-K partials
// (0: neither; operands whose only problem is a 2-byte aligned base are packed too when the
// workspace passed at launch is large enough for them).
int64_t gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, bool ta, bool tb) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const int64_t K8 = round8(K);
  return (shape_packs_a(M, K, ta) ? align_up(M * K8 * 2) : 0) + (shape_packs_b(N, K, tb) ? align_up(N * K8 * 2) : 0) +
         split_bytes(M, N, split_plan(M, N, K8, 0, 0).S);
}

// Workspace bytes of a split into `splits` segments (0: by the split rule).
int64_t gemm_splitk_workspace_bytes(int64_t M, int64_t N, int64_t K, int splits) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return split_bytes(M, N, split_plan(M, N, K, splits, 0).S);
}

// The tiled kernel split into `splits` segments (1: unsplit; 0: by the split rule) on
// operands it reads in place; hipErrorNotSupported when it cannot read them in place or the
// workspace does not hold the partials.  A split writes C through the reduce kernel, which
// takes any C alignment; unsplit, a C base that is not 16-byte aligned needs B as [N, K].
hipError_t launch_gemm_split(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                             int64_t N, int64_t K, bool ta, bool tb, int relu, int tile, int splits, void* ws,
                             int64_t ws_bytes, hipStream_t s) {
  if (!gemm_fast_fits(M, N, K, ta, tb, A, B, A)) return hipErrorNotSupported;  // C checked below
  const bool c_unaligned = (reinterpret_cast<uintptr_t>(C) & 15) != 0;
  const SplitPlan plan = split_plan(M, N, K, splits, tile);
  if (plan.S > 1 && (ws == nullptr || (reinterpret_cast<uintptr_t>(ws) & (kWsAlign - 1)) != 0 ||
                     split_bytes(M, N, plan.S) > ws_bytes))
    return hipErrorNotSupported;
  if (plan.S == 1 && c_unaligned && !tb) return hipErrorNotSupported;
  return launch_tiled(A, B, bias, C, M, N, K, ta, tb, relu, tile, c_unaligned, plan, ws, ws_bytes, s);
}

// The packed path, or hipErrorNotSupported when it does not apply (then the caller runs the
// guarded kernel): the tiled kernel's size limits on the packed shape, and a workspace that
// holds every operand that must be packed.
hipError_t launch_gemm_packed(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                              int64_t N, int64_t K, bool ta, bool tb, int relu, int tile, void* ws, int64_t ws_bytes,
                              hipStream_t s) {
  if (ws == nullptr || K <= 0 || (reinterpret_cast<uintptr_t>(ws) & (kWsAlign - 1)) != 0) return hipErrorNotSupported;
  const int64_t K8 = round8(K);
  const bool c_unaligned = N % 8 != 0 || (reinterpret_cast<uintptr_t>(C) & 15) != 0;
  const bool pa = shape_packs_a(M, K, ta) || (reinterpret_cast<uintptr_t>(A) & 15) != 0;
  // C written with 2-byte stores needs B as [N, K]: pack B then too
  const bool pb = shape_packs_b(N, K, tb) || (reinterpret_cast<uintptr_t>(B) & 15) != 0 || (c_unaligned && !tb);
  const int64_t a_bytes = pa ? align_up(M * K8 * 2) : 0, b_bytes = pb ? align_up(N * K8 * 2) : 0;
  if (a_bytes + b_bytes > ws_bytes) return hipErrorNotSupported;
  // a transposing copy runs (K8 / 64) x (R / 64) tiles: grid.y holds at most 65535
  const bool km_copy = (pa && ta) || (pb && !tb);
  if (km_copy && (K8 + kT - 1) / kT > 65535) return hipErrorNotSupported;
  uint16_t* a_ws = static_cast<uint16_t*>(ws);
  uint16_t* b_ws = reinterpret_cast<uint16_t*>(static_cast<char*>(ws) + a_bytes);
  const uint16_t* A2 = pa ? a_ws : A;
  const uint16_t* B2 = pb ? b_ws : B;
  const bool ta2 = pa ? false : ta, tb2 = pb ? true : tb;
  // the tiled kernel's conditions on the packed operands (C's alignment is handled by the
  // 2-byte store path; a 16-byte aligned stand-in is passed for it)
  if (!gemm_fast_fits(M, N, K8, ta2, tb2, A2, B2, ws)) return hipErrorNotSupported;
  hipError_t e = hipSuccess;
  if (pa) e = pack(A, a_ws, M, K, ta, s);
  if (e == hipSuccess && pb) e = pack(B, b_ws, N, K, !tb, s);
  if (e != hipSuccess) return e;
  return launch_tiled(A2, B2, bias, C, M, N, K8, ta2, tb2, relu, tile, c_unaligned, split_plan(M, N, K8, 0, tile),
                      static_cast<char*>(ws) + a_bytes + b_bytes, ws_bytes - a_bytes - b_bytes, s);
}

}  // namespace ihip
