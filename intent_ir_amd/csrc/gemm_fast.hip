// Tiled bf16 GEMM for gfx950: C = act(A @ B + bias), A [M,K], B [K,N] row-major bf16,
// f32 accumulation on v_mfma_f32_32x32x16_bf16, C bf16 (RNE).  Any M, N and K as long as
// every row of A and B starts 16-byte aligned (K % 8 == 0, M % 8 == 0 when A is given as
// [K,M], N % 8 == 0 when B is given as [K,N]) and the bases are 16-byte aligned; C rows that
// are not (N % 8 != 0 with B given as [N,K]) are written with 2-byte stores.  Other shapes
// take the guarded kernel in gemm.hip.  Edge tiles (past M or N, or all tiles when K is not a
// multiple of DK) copy through range-checked buffer descriptors: reads past the end of a
// tensor and k-chunks past K load zeros, and what an edge tile reads outside [M) x [N) only
// reaches C rows >= M or columns >= N, which are never stored.
//
// Work decomposition
//  * one 256x256 C tile per workgroup of 256 threads = 4 waves in a 2x2 grid; wave (wm, wn)
//    owns rows wm*128 + [0,128) and the four 32-column blocks wn*32 + 64*ni, ni = 0..3
//    (4x4 MFMA blocks, 256 f32 accumulators per lane, held in AGPRs);
//  * grids of at most 128 such tiles (half the CUs) use 128x128 tiles instead, with the same
//    wave grid over 2x2 MFMA blocks per wave: twice the LDS reads per MFMA, but up to four
//    times the busy CUs; every C element accumulates the same MFMAs in the same k order in
//    either form, so the results are identical;
//  * tiles are remapped so each of the 8 XCDs (private L2) works on one contiguous range,
//    rastered in groups of 8 tile-rows, so concurrently running tiles share A rows and
//    B columns in L2.
//
// Operand staging
//  * a ring of STAGES LDS stages of B (DK x 256 slices); the copy of K-slice kt+STAGES-1 is
//    issued while slice kt is multiplied, so a copy has STAGES-1 slices of MFMA time to land;
//  * A given as [M, K] sits in a ring of three regions, each holding 256 rows of 2*DK k (a
//    pair of slices, 128-byte rows), so every copy reads whole 128-byte cache lines: the two
//    row halves of pair P are copied while slices 2P-4 and 2P-3 are multiplied.  A given as
//    [K, M] uses STAGES stages of DK k-rows like B;
//  * copies use gfx950's direct-to-LDS loads (global_load_lds_dwordx4 in interior tiles,
//    buffer_load_dwordx4 ... lds in edge tiles): lane l of a wave writes 16 bytes at LDS
//    m0 + 16*l; no VGPR holds tile data;
//  * because the LDS position is fixed by the lane, bank conflicts are avoided by choosing
//    which global 16-byte chunk each lane fetches (XOR swizzles, 64-bank LDS):
//      a K-contiguous row r (R bytes: 128 for a paired A, DK*2 for B given as [N, K]) stores
//        logical k-chunk c in slot c ^ ((r / RPW) % CA), where CA = R/16 chunks per row and
//        RPW = 256 / R rows per 256-byte bank window: the 16 rows one ds_read_b128 cycle
//        serves cover all 16 bank positions;
//      B row k (512 bytes) stores logical n-chunk c in slot c ^ 2*(k & 3) ^ 8*((c >> 1) & 1):
//        the 4 rows x 2 column groups one 32-lane ds_read_b64_tr_b16 cycle serves land on
//        8 distinct 32-byte windows;
//  * B fragments come from ds_read_b64_tr_b16: lanes 4t+q of a 16-lane group address
//    row k0+t, columns 4q..4q+3, and lane i receives column i of rows k0..k0+3, i.e. the
//    k-contiguous operand layout, with no VALU transposition.
//  * The MFMA is issued as D = B^T-block x A-block, so each lane's accumulators hold four
//    consecutive n of one m: the epilogue adds bias, applies ReLU, packs 8 bytes of bf16 per
//    lane into the C tile staged in LDS, and writes the tile out in full 512-byte rows.
#include "common.hpp"

#include <type_traits>

namespace ihip {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x8_t __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
typedef __attribute__((address_space(3))) bf16x8_t lds_bf16x8_t;
typedef __attribute__((address_space(3))) char lds_char_t;
typedef __attribute__((address_space(3))) char lds_wchar_t;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2_t;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4_t;
typedef __attribute__((address_space(3))) f32x4_t lds_f32x4_t;

constexpr int kGroupRows = 8;  // tile-rows per raster group

// The K loop of a launch: KL k from the operands' bases (which a split-K launch offsets into
// the tensors), and one past each tensor's last element (edge copies are range-checked
// against the whole tensor).
struct GemmKRange {
  const uint16_t* a_end;
  const uint16_t* b_end;
  int64_t KL;
};

typedef __bf16 bf16x2_pk_t __attribute__((ext_vector_type(2)));

// AKM / BKM select the global layout of each operand: false = K-contiguous rows (A [M,K],
// or B given transposed as [N,K]), true = K-major (A given transposed as [K,M], or B
// [K,N]).  A K-contiguous operand is staged as [256 rows][DK] and read with ds_read_b128; a
// K-major one as [DK][256] and read with the transposing ds_read_b64_tr_b16.  Either way the
// MFMA sees the same fragments, so every layout accumulates in the same order and gives
// identical results.
// EDGE: the tile reaches past M or N; its copies go through range-checked buffer descriptors
// (interior tiles use global_load_lds, which measured ~14% faster on full 8192^3 GEMMs).
// TILE: M and N extent of the workgroup tile (256, or 128 for grids that would leave CUs idle);
// the four waves form a 2x2 grid either way, each owning TILE/64 x TILE/64 MFMA blocks.
template <int DK, int STAGES, bool AKM = false, bool BKM = true, bool EDGE = false, int TILE = 256>
struct FastGemm {
  static_assert(TILE == 256 || TILE == 128, "tile extents");
  static constexpr int kBlk = TILE / 64;           // 32-row A blocks and 32-column B blocks per wave
  static constexpr int kRowA = DK * 2;             // bytes per K-contiguous tile row
  static constexpr int kChunksA = DK / 8;          // 16-byte chunks per row
  static constexpr int kRowsPerWindow = 256 / kRowA;
  static constexpr int kRowKM = TILE * 2;          // bytes per K-major tile row
  static constexpr int kChunksKM = TILE / 8;       // 16-byte chunks per K-major row
  static constexpr int kRowsPerInstrKM = 1024 / kRowKM;
  static constexpr int kStageA = TILE * kRowA;     // bytes per operand tile (either layout)
  static constexpr int kStageB = DK * TILE * 2;
  static constexpr int kInstrA = kStageA / 1024 / 4;  // direct-to-LDS instructions per wave per stage
  static constexpr int kInstrB = kStageB / 1024 / 4;
  static constexpr int kInstr = kInstrA + kInstrB;
  static constexpr int kRowsPerInstrA = 1024 / kRowA;
  static_assert(kInstr * (STAGES - 2) <= 63, "vmcnt field");

  // A given as [M, K] (K-contiguous) is staged in pairs of K slices: a region holds the tile's
  // TILE rows of 2*DK k, 128-byte rows, so that every copy reads whole 128-byte cache lines
  // (64-byte row pieces, one slice each, took ~3% of the GEMM's rate).  Pair P (slices 2P and
  // 2P+1) lives in region P % 3; its upper-row and lower-row halves are copied during slices
  // 2P-4 and 2P-3, when the pair that used the region before (P-3, slices 2P-6 and 2P-5) has
  // been read.  Slice kt reads its pair's k-half kt & 1.  Three regions of 2*DK k and a B ring
  // of STAGES slices fill the 160 KiB LDS.
  static constexpr bool kPairA = !AKM;
  static constexpr int kRowP = 4 * DK;             // bytes per paired A row
  static constexpr int kChunksP = kRowP / 16;
  static constexpr int kRowsPerWindowP = 256 / kRowP;
  static constexpr int kRowsPerInstrP = 1024 / kRowP;
  static constexpr int kRegionA = kPairA ? TILE * kRowP : kStageA;
  static constexpr int kRegionsA = kPairA ? 3 : STAGES;
  static constexpr int kRingA = kRegionsA * kRegionA;
  static constexpr int kLdsRing = kRingA + STAGES * kStageB;
  static_assert(!kPairA || (DK == 32 && STAGES == 4), "paired A: 128-byte rows and a lead of three slices");
  static_assert(kLdsRing <= 160 * 1024, "stages exceed the 160 KiB LDS");

  // LDS byte offsets of slice kt's A stage (unpaired A) and B stage.  A paired A's region is
  // carried through the loops; its k-half is selected by XOR-ing bit 6 into the fragment
  // offsets (the upper half's chunks sit at slots c ^ 4 of the lower half's).
  static __device__ __forceinline__ int a_region(int kt) { return (kt % STAGES) * kStageA; }
  static __device__ __forceinline__ int b_stage(int kt) { return kRingA + (kt % STAGES) * kStageB; }

  static __device__ __forceinline__ int a_slot(int c, int r) { return c ^ ((r / kRowsPerWindow) % kChunksA); }
  static __device__ __forceinline__ int p_slot(int c, int r) { return c ^ ((r / kRowsPerWindowP) % kChunksP); }
  static __device__ __forceinline__ int b_slot(int c, int k) { return c ^ ((k & 3) << 1) ^ (((c >> 1) & 1) << 3); }
  static __device__ __forceinline__ int b_logical(int p, int k) {
    const int x = p ^ ((k & 3) << 1);
    return x ^ (((x >> 1) & 1) << 3);
  }

  // Per-lane offsets: copy offsets (bytes from the copy's scalar base) and fragment LDS
  // offsets.  K-contiguous operand: off[kk], blocks at a fixed stride; K-major: off[block].
  struct Lane {
    uint32_t a, b;
    uint32_t ai[4], bi[4];  // copy offsets per instruction i of a slice (a or b + that instruction's rows)
    int ka, kb;  // first k (within a slice) of the lane's 16-byte chunk; 0 for a K-major operand
    int fa[4], fb[4];
  };

  // Copy offset of a lane: K-contiguous rows (leading dim K) or K-major rows (leading dim ld).
  static __device__ __forceinline__ uint32_t copy_off(bool kmajor, int64_t ld, int64_t K, int wave, int lane) {
    if (!kmajor) {
      // instruction j = 4i + wave holds rows j*RPI + lane / CA, slot lane % CA; the swizzle
      // term (r / RPW) % CA does not depend on i
      const int r0 = wave * kRowsPerInstrA + lane / kChunksA;
      return 2u * static_cast<uint32_t>((lane / kChunksA) * K + a_slot(lane % kChunksA, r0) * 8);
    }
    // instruction j = 4i + wave holds k-rows j*RPK + lane / CK (RPK = 1024 / row bytes, CK
    // chunks per row), chunk lane % CK; k & 3 == (wave*RPK + lane/CK) & 3 for every i
    const int row = lane / kChunksKM;
    const int kb = wave * kRowsPerInstrKM + row;
    return 2u * static_cast<uint32_t>(row * ld + b_logical(lane % kChunksKM, kb) * 8);
  }

  // First k within the slice of the chunk a lane copies (K-contiguous operand; the swizzle
  // term does not depend on the instruction).
  static __device__ __forceinline__ int copy_k(bool kmajor, int wave, int lane) {
    return kmajor ? 0 : a_slot(lane % kChunksA, wave * kRowsPerInstrA + lane / kChunksA) * 8;
  }

  // Fragment offsets of an operand whose wave rows start at `base` with blocks `step` apart.
  static __device__ __forceinline__ void frag_off(bool kmajor, int region, int base, int step, int lane, int (&o)[4]) {
    if (!kmajor) {
      const int r = base + (lane & 31);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) o[kk] = kk < DK / 16 ? region + r * kRowA + a_slot(2 * kk + (lane >> 5), r) * 16 : 0;
    } else {
      const int g = lane >> 4, i = lane & 15;
      const int k = (g >> 1) * 8 + (i >> 2);
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        const int x = base + blk * step + (g & 1) * 16 + 4 * (i & 3);
        o[blk] = region + k * kRowKM + b_slot(x >> 3, k) * 16 + (x & 7) * 2;
      }
    }
  }

  // Paired A.  Copy instruction j = 4i + wave of a half holds region rows
  // h*TILE/2 + j*RPI + lane / CP (RPI = 8 rows of CP = 8 chunks), slot lane % CP; the swizzle
  // term (r / 2) % 8 = (4j + lane / 16) % 8 depends on j only through j & 1 = wave & 1.
  static __device__ __forceinline__ int pair_row(int wave, int lane) {
    return (wave & 1) * kRowsPerInstrP + lane / kChunksP;
  }
  static __device__ __forceinline__ uint32_t pair_copy_off(int64_t K, int wave, int lane) {
    return 2u * static_cast<uint32_t>((lane / kChunksP) * K + p_slot(lane % kChunksP, pair_row(wave, lane)) * 8);
  }
  static __device__ __forceinline__ void pair_frag_off(int base, int lane, int (&o)[4]) {
    const int r = base + (lane & 31);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) o[kk] = kk < DK / 16 ? r * kRowP + p_slot(2 * kk + (lane >> 5), r) * 16 : 0;
  }

  static __device__ __forceinline__ Lane lane_plan(int64_t M, int64_t N, int64_t K, int wave, int wm, int wn,
                                                   int lane) {
    Lane L;
    if constexpr (kPairA) {
      L.a = pair_copy_off(K, wave, lane);
      L.ka = p_slot(lane % kChunksP, pair_row(wave, lane)) * 8;
      pair_frag_off(wm * (TILE / 2), lane, L.fa);
    } else {
      L.a = copy_off(AKM, M, K, wave, lane);
      L.ka = copy_k(AKM, wave, lane);
      frag_off(AKM, 0, wm * (TILE / 2), 32, lane, L.fa);
    }
    L.b = copy_off(BKM, N, K, wave, lane);
    L.kb = copy_k(BKM, wave, lane);
    frag_off(BKM, 0, wn * 32, 64, lane, L.fb);
    // Instruction j = 4i + wave of a slice starts j*RPI rows (or k-rows) past the slice base;
    // with that offset in the lane's VGPR the slice base is the only scalar address per slice.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 4 * i + wave;
      L.ai[i] = i < kInstrA ? L.a + (kPairA ? static_cast<uint32_t>(j * kRowsPerInstrP * K * 2) : instr_off<AKM>(j, M, K))
                            : 0u;
      L.bi[i] = i < kInstrB ? L.b + instr_off<BKM>(j, N, K) : 0u;
    }
    return L;
  }

  // Raw buffer descriptor of the bytes from `base` to `end` (one past a tensor's last
  // element): a lane whose offset reaches past the end reads zeros and touches no memory,
  // which is what makes edge tiles (rows >= M, columns >= N) safe to copy.  The range check
  // covers the VGPR offset (not the SGPR one), so every offset beyond `base` goes there.
  static __device__ __forceinline__ i32x4_t rsrc_of(const uint16_t* base, const uint16_t* end) {
    const int64_t left = (end - base) * 2;
    const uint32_t records = left <= 0 ? 0u : left >= 0xffffffffll ? 0xffffffffu : static_cast<uint32_t>(left);
    const uint64_t addr = reinterpret_cast<uint64_t>(base);
    // word1: base address bits 47:32, stride 0; word3: 32-bit data format, raw (untyped) access
    return i32x4_t{static_cast<int>(addr & 0xffffffffu), static_cast<int>((addr >> 32) & 0xffffu),
                   static_cast<int>(records), 0x00020000};
  }

  // 16 bytes per lane into LDS at m0 + 16 * lane, from sbase + voff (global_load_lds) or
  // from the descriptor's base + voff (buffer_load ... lds).  Inline asm, so the compiler does
  // not treat a copy as an LDS store that every later LDS read must wait for; the kernel waits
  // for the copies itself before reading a stage.
  static __device__ __forceinline__ void dma16(const uint16_t* sbase, uint32_t voff, uint32_t lds_addr) {
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_addr) : "memory");
  }
  static __device__ __forceinline__ void dma16(const i32x4_t& rsrc, uint32_t voff, uint32_t lds_addr) {
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "{m0}"(lds_addr) : "memory");
  }

  // Lane offset that no descriptor covers (operands of a ragged-K launch are < 2 GiB).
  static constexpr uint32_t kNoRecord = 0x80000000u;

  // One copy instruction of an operand slice starting at `base` (`end`: one past the tensor's
  // last element; voff: the lane's offset for this instruction).  In an edge tile, the lanes
  // of a K-contiguous operand whose chunk starts at or past K (k_left = K - k0 elements remain
  // from the slice start, chunk_k = the chunk's first k) take an offset past every record and
  // load zeros; a K-major operand's k-rows past K lie past the tensor's end.
  template <bool kKMajor>
  static __device__ __forceinline__ void copy_one(const uint16_t* base, const uint16_t* end, uint32_t voff,
                                                  int64_t k_left, int chunk_k, uint32_t dst) {
    if constexpr (EDGE)
      dma16(rsrc_of(base, end), kKMajor || chunk_k < k_left ? voff : kNoRecord, dst);
    else
      dma16(base, voff, dst);
  }

  // Byte offset of copy instruction j from its operand's slice base: tile rows j*RPI.. of a
  // K-contiguous operand (leading dim K), k-rows j*RPK.. of a K-major one (leading dim ld).
  template <bool kKMajor>
  static __device__ __forceinline__ uint32_t instr_off(int j, int64_t ld, int64_t K) {
    return static_cast<uint32_t>(kKMajor ? j * kRowsPerInstrKM * ld * 2 : j * kRowsPerInstrA * K * 2);
  }

  // Slice base of an operand: tile rows x0.. at k0 (K-contiguous) or k-row k0 at column x0
  // (K-major).
  template <bool kKMajor>
  static __device__ __forceinline__ const uint16_t* slice_base(const uint16_t* X, int64_t ld, int64_t K, int64_t x0,
                                                               int64_t k0) {
    return kKMajor ? X + k0 * ld + x0 : X + x0 * K + k0;
  }

  // One operand's share of a K slice: tile rows x0.. (K-contiguous) or k-rows k0.. (K-major).
  template <bool kKMajor, int kInstrOp>
  static __device__ __forceinline__ void copy_operand(const uint16_t* __restrict__ X, const uint16_t* end, int64_t ld,
                                                      int64_t K, int64_t KL, int64_t x0, int64_t k0, uint32_t dst,
                                                      int wave, const uint32_t (&voff)[4], int chunk_k) {
    const uint16_t* base = slice_base<kKMajor>(X, ld, K, x0, k0);
#pragma unroll
    for (int i = 0; i < kInstrOp; ++i)
      copy_one<kKMajor>(base, end, voff[i], KL - k0, chunk_k, dst + (4 * i + wave) * 1024);
  }

  // With an odd number of K slices (more than one) the last A pair holds a single slice.
  static __device__ __forceinline__ bool single_last(int KT) { return (KT & 1) && KT > 1; }

  // Where half h of A pair P comes from and goes to.  A single-slice last pair is copied from
  // one slice lower (k0 - DK), so that no lane of an interior tile reads past K, and its slice
  // is read from the upper k-half.  Pairs past the last are placeholders that keep every
  // slice's copy count fixed (the waits count instructions): they re-read the last pair into a
  // region that no slice reads again.
  struct PairSrc {
    const uint16_t* base;  // the half's first row at the pair's first k
    int64_t k_left;        // k from there to K
    uint32_t dst;          // LDS address of the half
  };
  // First k copied for pair P (last: index of the last pair; single: the last pair's index if it
  // holds one slice, else -1).
  static __device__ __forceinline__ int64_t pair_k0(int P, int last, int single) {
    const int pr = P < last ? P : last;
    return static_cast<int64_t>(pr) * 2 * DK - (pr == single ? DK : 0);
  }
  // rows: A + (m0 + h*TILE/2)*K; KL: the k extent of the launch's K loop; k0: pair_k0 of the
  // pair; region: where the pair goes.
  static __device__ __forceinline__ PairSrc pair_src(const uint16_t* rows, int64_t KL, int64_t k0, int region, int h,
                                                     uint32_t lds_addr) {
    return {rows + k0, KL - k0, lds_addr + static_cast<uint32_t>(region * kRegionA + h * (TILE / 2) * kRowP)};
  }

  // Copy instruction i (rows of instruction j = 4i + wave) of a pair half (end: one past A's
  // last element).
  static __device__ __forceinline__ void copy_pair(const PairSrc& ps, const uint16_t* end, int i, int wave,
                                                   const Lane& L) {
    const uint32_t dst = ps.dst + (4 * i + wave) * 1024;
    if constexpr (EDGE)
      dma16(rsrc_of(ps.base, end), L.ka < ps.k_left ? L.ai[i] : kNoRecord, dst);
    else
      dma16(ps.base, L.ai[i], dst);
  }

  // All of this wave's instructions of A pair P (both halves) into region P (prologue: P < 3).
  static __device__ __forceinline__ void copy_pair_all(const uint16_t* rows0, const uint16_t* rows1,
                                                       const uint16_t* end, int64_t KL, int P, int last, int single,
                                                       int wave, const Lane& L, uint32_t lds_addr) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const PairSrc ps = pair_src(h ? rows1 : rows0, KL, pair_k0(P, last, single), P, h, lds_addr);
#pragma unroll
      for (int i = 0; i < kInstrA; ++i) copy_pair(ps, end, i, wave, L);
    }
  }

  // This wave's share of K slice s of B (and of an unpaired A).
  static __device__ __forceinline__ void copy_b(const uint16_t* __restrict__ B, int64_t N, int64_t K, int64_t n0, int s,
                                                int wave, const Lane& L, uint32_t lds_addr, const GemmKRange& R) {
    copy_operand<BKM, kInstrB>(B, R.b_end, N, K, R.KL, n0, static_cast<int64_t>(s) * DK, lds_addr + b_stage(s), wave,
                               L.bi, L.kb);
  }
  static __device__ __forceinline__ void copy_a(const uint16_t* __restrict__ A, int64_t M, int64_t K, int64_t m0, int s,
                                                int wave, const Lane& L, uint32_t lds_addr, const GemmKRange& R) {
    copy_operand<AKM, kInstrA>(A, R.a_end, M, K, R.KL, m0, static_cast<int64_t>(s) * DK, lds_addr + a_region(s), wave,
                               L.ai, L.ka);
  }

  // Wait until at most `pending` slices of this wave's copies are still in flight
  // (copies complete in issue order, kInstr instructions per slice).
  static __device__ __forceinline__ void wait_copies(int pending) {
    static_assert(STAGES <= 5, "wait_copies covers up to 4 pending slices");
    if (pending >= 4) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * kInstr < 63 ? 4 * kInstr : 63) : "memory");
    } else if (pending == 3) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * kInstr < 63 ? 3 * kInstr : 63) : "memory");
    } else if (pending == 2) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kInstr) : "memory");
    } else if (pending == 1) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kInstr) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
  }

  struct Frag {
    bf16x8_t a[kBlk], b[kBlk];
  };

  // Fragment reads of one k16 step from slice bases `st` (hx: the k-half XOR of a paired A).
  template <bool kKMajor>
  static __device__ __forceinline__ void read_operand(const lds_char_t* st, int hx, int kk, const int (&o)[4],
                                                      int blk_stride, bf16x8_t (&f)[kBlk]) {
#pragma unroll
    for (int blk = 0; blk < kBlk; ++blk) {
      if (!kKMajor) {
        f[blk] = *(const lds_bf16x8_t*)(st + (o[kk] ^ hx) + blk * blk_stride);
      } else {
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(st + o[blk] + kk * 16 * kRowKM));
        const i16x4_t hi =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(st + o[blk] + (kk * 16 + 4) * kRowKM));
        const i16x8_t both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        f[blk] = __builtin_bit_cast(bf16x8_t, both);
      }
    }
  }

  // Bytes between the 32-row A blocks of a wave (paired or unpaired rows).
  static constexpr int kBlkStrideA = 32 * (kPairA ? kRowP : kRowA);

  static __device__ __forceinline__ void read(const lds_char_t* sa, int hx, const lds_char_t* sb, int kk,
                                              const Lane& L, Frag& f) {
    read_operand<AKM>(sa, hx, kk, L.fa, kBlkStrideA, f.a);
    read_operand<BKM>(sb, 0, kk, L.fb, 64 * kRowA, f.b);
  }

  // The fragment reads of one k16 step as a flat list of LDS instructions ("slots"): A's
  // first, then B's; a K-contiguous operand takes one ds_read_b128 per block, a K-major one
  // two ds_read_b64_tr_b16 (low and high four k) per block.
  static constexpr int kSlotsA = AKM ? 2 * kBlk : kBlk;
  static constexpr int kSlots = kSlotsA + (BKM ? 2 * kBlk : kBlk);

  template <bool kKMajor>
  static __device__ __forceinline__ void read_operand_slot(const lds_char_t* st, int hx, int kk, const int (&o)[4],
                                                           int blk_stride, bf16x8_t (&f)[kBlk], int slot) {
    if (!kKMajor) {
      f[slot] = *(const lds_bf16x8_t*)(st + (o[kk] ^ hx) + slot * blk_stride);
    } else {
      const int blk = slot >> 1, half = slot & 1;
      const i16x4_t v =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(st + o[blk] + (kk * 16 + half * 4) * kRowKM));
      i16x8_t w = __builtin_bit_cast(i16x8_t, f[blk]);
      if (half == 0) {
        w[0] = v[0], w[1] = v[1], w[2] = v[2], w[3] = v[3];
      } else {
        w[4] = v[0], w[5] = v[1], w[6] = v[2], w[7] = v[3];
      }
      f[blk] = __builtin_bit_cast(bf16x8_t, w);
    }
  }

  static __device__ __forceinline__ void read_slot(const lds_char_t* sa, int hx, const lds_char_t* sb, int kk,
                                                   const Lane& L, Frag& f, int slot) {
    if (slot < kSlotsA)
      read_operand_slot<AKM>(sa, hx, kk, L.fa, kBlkStrideA, f.a, slot);
    else
      read_operand_slot<BKM>(sb, 0, kk, L.fb, 64 * kRowA, f.b, slot - kSlotsA);
  }

  // The MFMAs of B block ni against A blocks lo .. hi-1.
  static __device__ __forceinline__ void mfma_range(const Frag& f, f32x16_t (&acc)[kBlk][kBlk], int ni, int lo,
                                                   int hi) {
#pragma unroll
    for (int mi = 0; mi < kBlk; ++mi)
      if (mi >= lo && mi < hi)
        acc[ni][mi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.b[ni], f.a[mi], acc[ni][mi], 0, 0, 0);
  }

  // Copy instruction i (0 .. kInstr-1) issued during slice kt: A's instructions first (ps: half
  // kt & 1 of pair kt/2 + 2, or slice kt + STAGES - 1 of an unpaired A), then B's (slice
  // kt + STAGES - 1).
  static __device__ __forceinline__ void copy_instr(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                                                    int64_t M, int64_t N, int64_t K, int64_t m0, int64_t n0, int kt,
                                                    const PairSrc& ps, uint32_t lds_addr, int wave, const Lane& L,
                                                    int i, const GemmKRange& R) {
    const int nt = kt + STAGES - 1;
    const int64_t k0 = static_cast<int64_t>(nt) * DK;
    if (i < kInstrA) {
      if constexpr (kPairA)
        copy_pair(ps, R.a_end, i, wave, L);
      else
        copy_one<AKM>(slice_base<AKM>(A, M, K, m0, k0), R.a_end, L.ai[i], R.KL - k0, L.ka,
                      lds_addr + a_region(nt) + (4 * i + wave) * 1024);
    } else {
      const int ib = i - kInstrA;
      copy_one<BKM>(slice_base<BKM>(B, N, K, n0, k0), R.b_end, L.bi[ib], R.KL - k0, L.kb,
                    lds_addr + b_stage(nt) + (4 * ib + wave) * 1024);
    }
  }

  // s_waitcnt vmcnt(n) for a compile-time n.
  template <int n>
  static __device__ __forceinline__ void wait_vm() {
    static_assert(n >= 0 && n <= 63, "vmcnt field");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory");
  }

};

// Bytes per staged C row (16 bytes of padding).
template <int TILE>
constexpr int c_pitch() {
  return TILE * 2 + 16;
}

// LDS bytes of the operand rings, which after the main loop hold the bf16 C tile and the
// tile's bias values.
template <int DK, int STAGES, bool AKM, bool BKM, int TILE>
constexpr int fast_lds_bytes() {
  constexpr int ring = FastGemm<DK, STAGES, AKM, BKM, false, TILE>::kLdsRing;
  constexpr int tail = TILE * c_pitch<TILE>() + TILE * 4;
  return ring > tail ? ring : tail;
}

// One TILE x TILE C tile at (m0, n0); lds_raw is the kernel's LDS.  CU: C rows are not 16-byte
// aligned (N % 8 != 0, only with B given as [N, K]); C is then written with 2-byte stores.
// kPartial (split-K): the tile's f32 sums over R's K segment go to P (row-major, ldp floats
// per row) instead of bias + activation into C.
template <int DK, int STAGES, bool AKM, bool BKM, bool EDGE, int TILE, bool CU, bool kPartial = false>
__device__ __forceinline__ void gemm_fast_tile(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                                               const float* __restrict__ bias, uint16_t* __restrict__ C, int64_t M,
                                               int64_t N, int64_t K, int relu, int64_t m0, int64_t n0,
                                               char* lds_raw, const GemmKRange& R, float* __restrict__ P = nullptr,
                                               int64_t ldp = 0) {
  using G = FastGemm<DK, STAGES, AKM, BKM, EDGE, TILE>;
  constexpr int kBlk = G::kBlk;
  constexpr int kCPitch = c_pitch<TILE>();
  static_assert(STAGES >= 3, "the pipeline keeps two slices ahead");
  const lds_char_t* lds = (const lds_char_t*)lds_raw;
  const uint32_t lds_addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave & 1, wn = wave >> 1;

  f32x16_t acc[kBlk][kBlk];
#pragma unroll
  for (int i = 0; i < kBlk; ++i)
#pragma unroll
    for (int j = 0; j < kBlk; ++j) acc[i][j] = f32x16_t{};

  // The tile's TILE bias values are loaded now, one per thread, so the epilogue does not wait
  // on global loads; they are staged in LDS after the main loop, whose rings fill the LDS.
  const float bias_v =
      threadIdx.x < TILE && bias != nullptr && (!EDGE || n0 + threadIdx.x < N) ? bias[n0 + threadIdx.x] : 0.0f;

  const typename G::Lane L = G::lane_plan(M, N, K, wave, wm, wn, lane);
  const int KT = static_cast<int>((R.KL + DK - 1) / DK);  // a ragged last slice only in edge instances
  // Slice kt's copies fill the stage slice kt-1 used, so a copy is issued kLead slices ahead.
  constexpr int kLead = STAGES - 1;
  // Paired A: row bases of the two halves of the tile, the last pair, and the last pair (or
  // slice) again when it holds a single slice (else -1).
  const uint16_t* const a_rows0 = A + m0 * K;
  const uint16_t* const a_rows1 = A + (m0 + TILE / 2) * K;
  const int last_pair = (KT - 1) >> 1;
  const int single_pair = G::single_last(KT) ? last_pair : -1;
  const int single_slice = G::single_last(KT) ? KT - 1 : -1;
  if constexpr (G::kPairA) {
    // Prologue: A pairs 0 and 1 (slices 0-3) and B slices 0-2 in flight, in the order
    // [pair 0, B 0] [B 1] [pair 1, B 2], then the first group must land.  With the steady
    // loop's kInstr copies per slice, the waits below stay exact: when slice kt+1 must land,
    // every copy issued up to slice kt-2 (B slice kt+1, pair (kt+1)/2) is complete.
    G::copy_pair_all(a_rows0, a_rows1, R.a_end, R.KL, 0, last_pair, single_pair, wave, L, lds_addr);
    G::copy_b(B, N, K, n0, 0, wave, L, lds_addr, R);
    if (KT > 1) G::copy_b(B, N, K, n0, 1, wave, L, lds_addr, R);
    if (KT > 2) {
      G::copy_pair_all(a_rows0, a_rows1, R.a_end, R.KL, 1, last_pair, single_pair, wave, L, lds_addr);
      G::copy_b(B, N, K, n0, 2, wave, L, lds_addr, R);
      G::template wait_vm<2 * G::kInstr>();
    } else if (KT > 1) {
      G::template wait_vm<G::kInstrB>();
    } else {
      G::template wait_vm<0>();
    }
  } else {
    // Prologue: slices 0 .. kLead-1 in flight, then slice 0 must land.
#pragma unroll
    for (int s = 0; s < kLead; ++s)
      if (s < KT) {
        G::copy_a(A, M, K, m0, s, wave, L, lds_addr, R);
        G::copy_b(B, N, K, n0, s, wave, L, lds_addr, R);
      }
    G::wait_copies((KT < kLead ? KT : kLead) - 1);
  }
  __syncthreads();

  // Main loop, software-pipelined per k16 step.  A step is kBlk quarters of kBlk MFMAs (one
  // B block against the wave's A blocks); the next step's fragment reads are slotted between a
  // quarter's MFMAs (sched_group_barrier), so no MFMA waits on LDS, and one copy instruction of
  // slice kt+kLead follows each of the first kPerStep quarters, so a wave never issues its
  // copies in a burst (a burst of copies stalls the issuing wave and skews the waves against
  // the slice barrier).  At the last step of slice kt the wave issues kPre MFMAs, waits for
  // its copies of slice kt+1, passes the barrier and reads slice kt+1's first fragments under
  // the remaining MFMAs.  The barrier is fenced: every wave's LDS reads of slice kt-1 are
  // complete once it passes the barrier ending slice kt-1, so slice kt may refill that stage.
  // The steady loop and the tail are separate straight-line loops: with merged control flow
  // the compiler's LDS wait counts become conservative and stall the MFMAs on reads of the
  // next slice.
  constexpr int NK = DK / 16;
  constexpr int kPerStep = G::kInstr / NK;
  static_assert(G::kInstr % NK == 0 && kPerStep <= kBlk, "at most one copy per quarter");
  constexpr int kPerQ = G::kSlots / kBlk;
  static_assert(G::kSlots % kBlk == 0 && kPerQ <= 4, "reads split evenly over quarters");
  static_assert(NK % 2 == 0, "fragment double buffer alternates within a slice");
  constexpr int kPre = 1;
  // copies in flight when slice kt+1 must have landed: slices kt+2 .. kt+kLead-1 and the part
  // of slice kt+kLead issued before the last step
  constexpr int kSteadyPending = (kLead - 2) * G::kInstr + (NK - 1) * kPerStep;
  typename G::Frag f[2];
  G::read(lds + (G::kPairA ? 0 : G::a_region(0)), 0, lds + G::b_stage(0), 0, L, f[0]);
  // Slice kt.  pa: region of its A pair (paired A); a_k0: pair_k0 of the pair it copies
  // (kt/2 + 2); par_tag: kt & 1 when known at compile time (-1: read kt).  Steady slices
  // (copy_tag true) never hold the single-slice last pair, so their k-halves follow kt & 1.
  auto slice = [&](int kt, int pa, int64_t a_k0, auto copy_tag, auto par_tag, int pending) {
    constexpr bool kCopy = decltype(copy_tag)::value;
    constexpr int kPar = decltype(par_tag)::value;
    const int odd = kPar >= 0 ? kPar : (kt & 1);
    const int pa1 = odd ? (pa == 2 ? 0 : pa + 1) : pa;
    const lds_char_t* sa = lds + (G::kPairA ? pa * G::kRegionA : G::a_region(kt));
    const lds_char_t* sa1 = lds + (G::kPairA ? pa1 * G::kRegionA : G::a_region(kt + 1));
    int hx = odd << 6, hx1 = (odd ^ 1) << 6;
    if (!kCopy) {
      hx = kt == single_slice ? 64 : hx;
      hx1 = kt + 1 == single_slice ? 64 : hx1;
    }
    if (!G::kPairA) hx = hx1 = 0;
    const lds_char_t* sb = lds + G::b_stage(kt);
    // A copies of this slice: half kt & 1 of pair kt/2 + 2, into the region pair kt/2 - 1 used
    typename G::PairSrc ps{};
    if constexpr (kCopy && G::kPairA)
      ps = G::pair_src(odd ? a_rows1 : a_rows0, R.KL, a_k0, pa == 0 ? 2 : pa - 1, odd, lds_addr);
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      typename G::Frag& cur = f[kk & 1];
      typename G::Frag& nxt = f[(kk & 1) ^ 1];
      const bool boundary = kk + 1 == NK;
      const bool more = !boundary || pending >= 0;  // a next step exists
      const lds_char_t* ra = boundary ? sa1 : sa;
      const lds_char_t* rb = boundary ? lds + G::b_stage(kt + 1) : sb;
      const int rhx = boundary ? hx1 : hx;
      const int rk = boundary ? 0 : kk + 1;
#pragma unroll
      for (int q = 0; q < kBlk; ++q) {
        // every quarter starts after all instructions of the previous one
        __builtin_amdgcn_sched_barrier(0);
        const bool pre = boundary && q == 0 && more;
        if (pre) {
          G::mfma_range(cur, acc, 0, 0, kPre);
          if constexpr (kCopy)
            G::template wait_vm<kSteadyPending>();
          else
            G::wait_copies(pending);
          __syncthreads();
          __builtin_amdgcn_sched_barrier(0);
        }
        const int from = pre ? kPre : 0;
        if (more) {
#pragma unroll
          for (int r = 0; r < kPerQ; ++r) G::read_slot(ra, rhx, rb, rk, L, nxt, q * kPerQ + r);
        }
        G::mfma_range(cur, acc, q, from, kBlk);
        if (more) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (j < kBlk - from) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            if (j < kPerQ) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     // one LDS read
          }
        }
        if constexpr (kCopy) {
          if (q < kPerStep) {
            __builtin_amdgcn_sched_barrier(0);
            G::copy_instr(A, B, M, N, K, m0, n0, kt, ps, lds_addr, wave, L, kk * kPerStep + q, R);
          }
        }
      }
    }
  };
  using Even = std::integral_constant<int, 0>;
  using Odd = std::integral_constant<int, 1>;
  using AnyPar = std::integral_constant<int, -1>;
  int kt = 0, pa = 0;
  // steady state: every slice copies, and waits for a fixed number of copies; two slices (one
  // A pair) per iteration, then at most one more
  for (; kt + 1 + kLead < KT; kt += 2) {
    const int64_t a_k0 = G::pair_k0((kt >> 1) + 2, last_pair, single_pair);
    slice(kt, pa, a_k0, std::true_type{}, Even{}, 0);
    slice(kt + 1, pa, a_k0, std::true_type{}, Odd{}, 0);
    pa = pa == 2 ? 0 : pa + 1;
  }
  if (kt + kLead < KT) {
    slice(kt, pa, G::pair_k0((kt >> 1) + 2, last_pair, single_pair), std::true_type{}, Even{}, 0);
    ++kt;
  }
  // tail: everything is issued; slice kt+1 must land, later ones may stay in flight
  for (; kt < KT; ++kt) {
    slice(kt, pa, 0, std::false_type{}, AnyPar{}, kt + 1 < KT ? KT - 2 - kt : -1);
    if (kt & 1) pa = pa == 2 ? 0 : pa + 1;
  }

  if constexpr (kPartial) {
    // Split-K partial sums in f32, staged through LDS TILE / 2 rows at a time (pass h: the
    // rows of the two waves with wm == h) and stored as whole rows of TILE floats, TILE / 4
    // lanes of 16 bytes per row; stored straight
    // from the MFMA layout, each instruction would write 32 bytes into each of 32 rows.  Rows
    // past M and 4-column groups at or past N are skipped (ldp, a multiple of 4, covers the
    // last group).  LDS rows are padded by 16 bytes against bank conflicts.
    constexpr int kPitchF = TILE + 4;
    constexpr int kChunkRows = TILE / 2;
    static_assert(kChunkRows * kPitchF * 4 <= fast_lds_bytes<DK, STAGES, AKM, BKM, TILE>(), "LDS");
    constexpr int kLanesPerRow = TILE / 4;
    constexpr int kRowsPerInstr = 64 / kLanesPerRow;
    lds_f32x4_t* const pt = (lds_f32x4_t*)lds_raw;  // viewed in 16-byte units: kPitchF / 4 per row
    const int c4 = lane % kLanesPerRow;
    __syncthreads();  // every wave's last fragment reads are done before the rings are overwritten
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (wm == h) {
#pragma unroll
        for (int ni = 0; ni < kBlk; ++ni)
#pragma unroll
          for (int mi = 0; mi < kBlk; ++mi) {
            const int ml = mi * 32 + (lane & 31);
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              const int nl = wn * 32 + ni * 64 + g4 * 8 + (lane >> 5) * 4;
              pt[(ml * kPitchF + nl) / 4] = f32x4_t{acc[ni][mi][g4 * 4], acc[ni][mi][g4 * 4 + 1],
                                                   acc[ni][mi][g4 * 4 + 2], acc[ni][mi][g4 * 4 + 3]};
            }
          }
      }
      __syncthreads();
#pragma unroll 4
      for (int i = 0; i < kChunkRows / (4 * kRowsPerInstr); ++i) {
        const int row = (i * 4 + wave) * kRowsPerInstr + lane / kLanesPerRow;
        const int64_t m = m0 + h * kChunkRows + row, n = n0 + c4 * 4;
        const f32x4_t v = pt[(row * kPitchF) / 4 + c4];
        if (!EDGE || (m < M && n < N)) *reinterpret_cast<f32x4_t*>(P + m * ldp + n) = v;
      }
      if (h == 0) __syncthreads();
    }
    return;
  }

  // Epilogue.  The tile is staged in LDS as bf16 rows and then written out in full 512-byte
  // rows: stored straight from the MFMA layout, every store instruction would write 16 bytes
  // into each of 32 rows (partial cache lines), which took ~19k cycles per tile against ~5k.
  // Bias add and activation are branch-free: no bias adds +0, ReLU is maximum(t, 0) (NaN
  // stays NaN) and no ReLU is maximum(t, -inf); v_cvt_pk_bf16_f32 rounds two values to
  // nearest even in one instruction.  One 32x32 block at a time (the empty asm keeps the
  // compiler from pulling all 256 accumulators into VGPRs at once).
  __syncthreads();  // every wave's last fragment reads are done before the rings are overwritten
  float* bias_lds = reinterpret_cast<float*>(lds_raw + TILE * kCPitch);
  if (threadIdx.x < TILE) bias_lds[threadIdx.x] = bias_v;
  __syncthreads();
  lds_wchar_t* ct = (lds_wchar_t*)lds_raw;
  const float floor_v = relu ? 0.0f : -__builtin_inff();
#pragma unroll
  for (int ni = 0; ni < kBlk; ++ni) {
    f32x4_t bv[4];
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4)
      bv[g4] = *reinterpret_cast<const f32x4_t*>(&bias_lds[wn * 32 + ni * 64 + g4 * 8 + (lane >> 5) * 4]);
#pragma unroll
    for (int mi = 0; mi < kBlk; ++mi) {
      const int ml = wm * (TILE / 2) + mi * 32 + (lane & 31);
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int nl = wn * 32 + ni * 64 + g4 * 8 + (lane >> 5) * 4;
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = __builtin_elementwise_maximum(acc[ni][mi][g4 * 4 + q] + bv[g4][q], floor_v);
        const bf16x2_pk_t lo = {static_cast<__bf16>(v[0]), static_cast<__bf16>(v[1])};
        const bf16x2_pk_t hi = {static_cast<__bf16>(v[2]), static_cast<__bf16>(v[3])};
        const u32x2 pk = {__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
        *(lds_u32x2_t*)(ct + ml * kCPitch + nl * 2) = pk;
      }
      asm volatile("" ::: "memory");
    }
  }
  __syncthreads();
  // TILE rows of TILE*2 bytes; one store instruction covers 64 / (TILE/8) rows (TILE/8 lanes of
  // 16 bytes per row).  An edge tile stores only rows < M and columns < N (whole 16-byte
  // chunks when N % 8 == 0, single elements otherwise).
  constexpr int kLanesPerRow = TILE / 8;
  constexpr int kRowsPerStore = 64 / kLanesPerRow;
  const int chunk = lane % kLanesPerRow;
  const bool col_ok = n0 + chunk * 8 < N;
  const int64_t col_left = N - (n0 + chunk * 8);  // columns of this chunk inside C (CU)
#pragma unroll 4
  for (int i = 0; i < TILE / (4 * kRowsPerStore); ++i) {
    const int row = (i * 4 + wave) * kRowsPerStore + lane / kLanesPerRow;
    const u32x4 v = *(const lds_u32x4_t*)(ct + row * kCPitch + chunk * 16);
    if constexpr (CU) {
      if (!EDGE || (col_ok && m0 + row < M)) {
        uint16_t* dst = C + (m0 + row) * N + n0 + chunk * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (!EDGE || e < col_left) dst[e] = static_cast<uint16_t>(v[e >> 1] >> (16 * (e & 1)));
      }
    } else {
      if (!EDGE || (col_ok && m0 + row < M)) *reinterpret_cast<u32x4*>(C + (m0 + row) * N + n0 + chunk * 8) = v;
    }
  }
}

template <int DK, int STAGES, bool AKM, bool BKM, int TILE, bool CU>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_bf16_fast_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, const float* __restrict__ bias,
                           uint16_t* __restrict__ C, int64_t M, int64_t N, int64_t K, int relu, int tiles_m,
                           int tiles_n) {
  constexpr int kLdsBytes = fast_lds_bytes<DK, STAGES, AKM, BKM, TILE>();
  static_assert(kLdsBytes <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) char lds_raw[kLdsBytes];

  const int bid = xcd_contiguous(blockIdx.x, gridDim.x);
  const int per_group = kGroupRows * tiles_n;
  const int grp = bid / per_group, first_m = grp * kGroupRows;
  const int gsz = (tiles_m - first_m) < kGroupRows ? (tiles_m - first_m) : kGroupRows;
  const int tm = first_m + (bid % per_group) % gsz, tn = (bid % per_group) / gsz;
  const int64_t m0 = static_cast<int64_t>(tm) * TILE, n0 = static_cast<int64_t>(tn) * TILE;

  // Uniform per workgroup: edge tiles (and every tile when K is not a whole number of K steps,
  // or, with a paired A, a single K step, whose pair would reach past K) run the range-checked
  // instance of the tile code.
  const GemmKRange R{A + M * K, B + K * N, K};
  if (m0 + TILE <= M && n0 + TILE <= N && K % DK == 0 && (AKM || K > DK))
    gemm_fast_tile<DK, STAGES, AKM, BKM, false, TILE, CU>(A, B, bias, C, M, N, K, relu, m0, n0, lds_raw, R);
  else
    gemm_fast_tile<DK, STAGES, AKM, BKM, true, TILE, CU>(A, B, bias, C, M, N, K, relu, m0, n0, lds_raw, R);
}

// Split-K: workgroup (tile, s) multiplies K segment s, k in [s * kseg, min((s + 1) * kseg, K)),
// into the f32 partials P + s * M * ldp.  kseg is a multiple of 64, so every segment but the
// last is a whole number of A pairs and reads nothing past its end.  One-dimensional grid of
// tiles x segments: workgroups are dispatched to the XCDs round robin (bid % 8), and each
// XCD (whose L2 is its own) is given a contiguous run of the segment-major order, tiles in
// groups of kGroupRows tile-rows walked column by column, so that it reads a compact slab of
// A and B rather than all of them.
template <int DK, int STAGES, bool AKM, bool BKM, int TILE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_bf16_splitk_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, float* __restrict__ P,
                             int64_t M, int64_t N, int64_t K, int64_t kseg, int64_t ldp, int tiles_m, int tiles_n) {
  constexpr int kLdsBytes = fast_lds_bytes<DK, STAGES, AKM, BKM, TILE>();
  static_assert(kLdsBytes <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) char lds_raw[kLdsBytes];

  const int bid = xcd_contiguous(blockIdx.x, gridDim.x);
  const int T = tiles_m * tiles_n;
  const int seg = bid / T, t = bid % T;
  const int per_group = kGroupRows * tiles_n;
  const int first_m = (t / per_group) * kGroupRows;
  const int gsz = (tiles_m - first_m) < kGroupRows ? (tiles_m - first_m) : kGroupRows;
  const int tm = first_m + (t % per_group) % gsz, tn = (t % per_group) / gsz;
  const int64_t m0 = static_cast<int64_t>(tm) * TILE, n0 = static_cast<int64_t>(tn) * TILE;
  const int64_t kb = static_cast<int64_t>(seg) * kseg;
  const int64_t KL = K - kb < kseg ? K - kb : kseg;
  const uint16_t* As = AKM ? A + kb * M : A + kb;
  const uint16_t* Bs = BKM ? B + kb * N : B + kb;
  float* Ps = P + static_cast<int64_t>(seg) * M * ldp;
  const GemmKRange R{A + M * K, B + K * N, KL};
  if (m0 + TILE <= M && n0 + TILE <= N && KL % DK == 0 && (AKM || KL > DK))
    gemm_fast_tile<DK, STAGES, AKM, BKM, false, TILE, false, true>(As, Bs, nullptr, nullptr, M, N, K, 0, m0, n0,
                                                                    lds_raw, R, Ps, ldp);
  else
    gemm_fast_tile<DK, STAGES, AKM, BKM, true, TILE, false, true>(As, Bs, nullptr, nullptr, M, N, K, 0, m0, n0,
                                                                   lds_raw, R, Ps, ldp);
}

// C = act(sum over the S segments of P + bias) in bf16 (round to nearest even), segments added
// in order 0 .. S-1; one thread per 4 consecutive columns of a row.  C rows are written with
// one 8-byte store where 8-byte aligned, else with 2-byte stores.
__global__ __launch_bounds__(256) void gemm_splitk_reduce(const float* __restrict__ P, int S, int64_t M, int64_t N,
                                                          int64_t ldp, const float* __restrict__ bias, int relu,
                                                          uint16_t* __restrict__ C) {
  const int64_t groups = ldp / 4;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= M * groups) return;
  const int64_t m = t / groups, n = (t % groups) * 4;
  if (n >= N) return;
  const int64_t plane = M * ldp;
  const f32x4_t* const src = reinterpret_cast<const f32x4_t*>(P + m * ldp + n);
  const auto part = [&](int s) { return src[s * (plane / 4)]; };
  // loads four segments ahead of the additions, which stay in segment order
  f32x4_t sum = part(0);
  int s = 1;
  for (; s + 3 < S; s += 4) {
    const f32x4_t p1 = part(s), p2 = part(s + 1), p3 = part(s + 2), p4 = part(s + 3);
    sum += p1;
    sum += p2;
    sum += p3;
    sum += p4;
  }
  for (; s < S; ++s) sum += part(s);
  const float floor_v = relu ? 0.0f : -__builtin_inff();
  float v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    v[q] = __builtin_elementwise_maximum(sum[q] + (bias != nullptr && n + q < N ? bias[n + q] : 0.0f), floor_v);
  uint16_t* dst = C + m * N + n;
  const u32x2 pk = {pack_bf16x2_rne(v[0], v[1]), pack_bf16x2_rne(v[2], v[3])};
  if (n + 4 <= N && (reinterpret_cast<uintptr_t>(dst) & 7) == 0) {
    *reinterpret_cast<u32x2*>(dst) = pk;
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (n + q < N) dst[q] = static_cast<uint16_t>(pk[q >> 1] >> (16 * (q & 1)));
  }
}

// K step and ring depth of the fast path.
constexpr int kFastDK = 32;
constexpr int kFastStages = 4;
// At most this many 256x256 tiles (half of the 256 CUs busy) the launch uses 128x128 tiles:
// measured 0.74-0.99 PF/s on such grids against 0.4-0.8 with 256x256 tiles; from 144 tiles up
// the 256x256 kernel is faster (fewer busy CUs also run at a higher clock on this power-limited
// chip).  Skinny products (M <= 128, the rows of a decode step) with more than one round of
// 256x256 tiles also take 128x128 tiles: a 256-row tile computes at least twice the rows it
// stores, and halving that waste was 10-18% faster at M = 32-128 with N = 128256, K = 4096
// (with a single round, 16 x 50257 x 4096, the 256x256 tiles stayed 15% faster).
constexpr int64_t kSmallGridTiles = 128;
constexpr int64_t kSkinnyRows = 128;

// Any M, N and K (edge tiles are copied through the descriptor's range check and stored under
// masks) as long as every row of A and B starts 16 bytes aligned: K % 8 == 0, M % 8 == 0 when
// A is given as [K, M], and N % 8 == 0 when B is given as [K, N].  With B given as [N, K]
// (the layout of a linear layer's weight) N may be anything: C rows that are not 16-byte
// aligned are written with 2-byte stores.  When K is not a whole number of K steps, A and B
// must be below 2 GiB each (the ragged k-chunks are pointed past every record).
bool gemm_fast_fits(int64_t M, int64_t N, int64_t K, bool transpose_a, bool transpose_b, const void* A, const void* B,
                    const void* C) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B) | reinterpret_cast<uintptr_t>(C);
  // per-lane copy offsets from a slice base are 32-bit: up to 256 rows of K elements, or
  // 64 k-rows of M or N elements
  const int64_t lim = int64_t(1) << 32;
  const bool sizes = K * 512 < lim && N * 128 < lim && M * 128 < lim;
  const bool ragged_k_ok = K % kFastDK == 0 || (M * K * 2 < (int64_t(1) << 31) && K * N * 2 < (int64_t(1) << 31));
  return M > 0 && N > 0 && K > 0 && (N % 8 == 0 || transpose_b) && K % 8 == 0 && (!transpose_a || M % 8 == 0) &&
         (al & 15) == 0 && sizes && ragged_k_ok;
}

int gemm_fast_tile_extent(int64_t M, int64_t N) {
  const int64_t tiles256 = ((M + 255) / 256) * ((N + 255) / 256);
  const int64_t tiles128 = ((M + 127) / 128) * ((N + 127) / 128);
  // one row of 256x256 tiles holding 129-256 rows: 128x128 tiles would take two rounds for a
  // second tile-row of at most half the rows (256 x 32000 x 4096: 7-17% slower than 256x256)
  const bool one_full_row = M > kSkinnyRows && M <= 256 && tiles128 > 256;
  return (tiles256 <= kSmallGridTiles && !one_full_row) || (M <= kSkinnyRows && tiles256 > 256) ? 128 : 256;
}

bool gemm_m16_fits(int64_t M, int64_t N, int64_t K, bool transpose_a, const void* A, const void* B, const void* C);
hipError_t launch_gemm_m16(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M, int64_t N,
                           int64_t K, bool transpose_b, int relu, hipStream_t s);

template <int TILE, bool CU>
static void launch_tiles(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M, int64_t N,
                         int64_t K, bool transpose_a, bool transpose_b, int relu, hipStream_t s) {
  const int64_t tm = (M + TILE - 1) / TILE, tn = (N + TILE - 1) / TILE;
  const dim3 grid(static_cast<unsigned>(tm * tn)), block(256);
  const int itm = static_cast<int>(tm), itn = static_cast<int>(tn);
  constexpr int DK = kFastDK, ST = kFastStages;
  if constexpr (CU) {  // only B given as [N, K] reaches here
    if (!transpose_a)
      gemm_bf16_fast_kernel<DK, ST, false, false, TILE, true><<<grid, block, 0, s>>>(A, B, bias, C, M, N, K, relu, itm, itn);
    else
      gemm_bf16_fast_kernel<DK, ST, true, false, TILE, true><<<grid, block, 0, s>>>(A, B, bias, C, M, N, K, relu, itm, itn);
  } else {
    if (!transpose_a && !transpose_b)
      gemm_bf16_fast_kernel<DK, ST, false, true, TILE, false><<<grid, block, 0, s>>>(A, B, bias, C, M, N, K, relu, itm, itn);
    else if (!transpose_a)
      gemm_bf16_fast_kernel<DK, ST, false, false, TILE, false><<<grid, block, 0, s>>>(A, B, bias, C, M, N, K, relu, itm, itn);
    else if (!transpose_b)
      gemm_bf16_fast_kernel<DK, ST, true, true, TILE, false><<<grid, block, 0, s>>>(A, B, bias, C, M, N, K, relu, itm, itn);
    else
      gemm_bf16_fast_kernel<DK, ST, true, false, TILE, false><<<grid, block, 0, s>>>(A, B, bias, C, M, N, K, relu, itm, itn);
  }
}

// transpose_a: A is given as [K, M]; transpose_b: B is given as [N, K].  tile: 0 = by grid
// size (gemm_fast_tile_extent), else 128 or 256.  c_unaligned: C's base is not 16-byte aligned
// (only with transpose_b): C is written with 2-byte stores, as for N % 8 != 0.
hipError_t launch_gemm_fast(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M, int64_t N,
                            int64_t K, bool transpose_a, bool transpose_b, int relu, int tile, hipStream_t s,
                            bool c_unaligned) {
  const bool small = (tile == 0 ? gemm_fast_tile_extent(M, N) : tile) == 128, cu = N % 8 != 0 || c_unaligned;
  // 256x256 tiles and K in 64-k slices: the 16x16x32 kernel (gemm_m16.hip), whose sums are
  // bit-identical to this file's
  if (!small && !cu && gemm_m16_fits(M, N, K, transpose_a, A, B, C))
    return launch_gemm_m16(A, B, bias, C, M, N, K, transpose_b, relu, s);
  if (small && cu)
    launch_tiles<128, true>(A, B, bias, C, M, N, K, transpose_a, transpose_b, relu, s);
  else if (small)
    launch_tiles<128, false>(A, B, bias, C, M, N, K, transpose_a, transpose_b, relu, s);
  else if (cu)
    launch_tiles<256, true>(A, B, bias, C, M, N, K, transpose_a, transpose_b, relu, s);
  else
    launch_tiles<256, false>(A, B, bias, C, M, N, K, transpose_a, transpose_b, relu, s);
  return hipGetLastError();
}

// Split-K with S segments of kseg k (gemm_split_k): the tiled kernel writes f32 partials to P
// (S x M x ldp floats) and gemm_splitk_reduce adds them in order with bias and activation.
// Same operand conditions as launch_gemm_fast; C may have any alignment.
template <int TILE>
static void launch_splitk_tiles(const uint16_t* A, const uint16_t* B, float* P, int64_t M, int64_t N, int64_t K,
                                int64_t kseg, int S, int64_t ldp, bool ta, bool tb, hipStream_t s) {
  const int64_t tm = (M + TILE - 1) / TILE, tn = (N + TILE - 1) / TILE;
  const dim3 grid(static_cast<unsigned>(tm * tn * S)), block(256);
  const int itm = static_cast<int>(tm), itn = static_cast<int>(tn);
  constexpr int DK = kFastDK, ST = kFastStages;
  if (!ta && !tb)
    gemm_bf16_splitk_kernel<DK, ST, false, true, TILE><<<grid, block, 0, s>>>(A, B, P, M, N, K, kseg, ldp, itm, itn);
  else if (!ta)
    gemm_bf16_splitk_kernel<DK, ST, false, false, TILE><<<grid, block, 0, s>>>(A, B, P, M, N, K, kseg, ldp, itm, itn);
  else if (!tb)
    gemm_bf16_splitk_kernel<DK, ST, true, true, TILE><<<grid, block, 0, s>>>(A, B, P, M, N, K, kseg, ldp, itm, itn);
  else
    gemm_bf16_splitk_kernel<DK, ST, true, false, TILE><<<grid, block, 0, s>>>(A, B, P, M, N, K, kseg, ldp, itm, itn);
}

hipError_t launch_gemm_splitk(const uint16_t* A, const uint16_t* B, const float* bias, uint16_t* C, int64_t M,
                              int64_t N, int64_t K, bool transpose_a, bool transpose_b, int relu, int tile, int S,
                              int64_t kseg, float* P, int64_t ldp, hipStream_t s) {
  if (tile == 256)
    launch_splitk_tiles<256>(A, B, P, M, N, K, kseg, S, ldp, transpose_a, transpose_b, s);
  else
    launch_splitk_tiles<128>(A, B, P, M, N, K, kseg, S, ldp, transpose_a, transpose_b, s);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t threads = M * (ldp / 4);
  gemm_splitk_reduce<<<dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0, s>>>(P, S, M, N, ldp, bias,
                                                                                             relu, C);
  return hipGetLastError();
}

}  // namespace ihip
