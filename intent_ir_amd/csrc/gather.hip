// gather over a 2-D f32 tensor: out[i] = inp[row[i], col[i]] for i < L, or other_value where
// the index pair lies outside [0, M) x [0, N) (negative indices included).  That is the CUDA
// backend's gather2d (backends/cuda/codegen/intentir_to_cuda.py:1779-1832, pinned by
// tests/backends/cuda/test_cuda_backend_smoke.py:292-336); in range it is the interpreter's
// numpy fancy indexing (verify/interpreter.py:284-291).
//
// Streaming of the index arrays and the output (12 bytes per element) plus one 4-byte read of
// inp per element at a data-dependent address, which costs a whole cache line when the
// addresses are scattered: random gathers are bound by the rate of distinct lines, not by
// bytes (measured 41-50 G elements/s from a 256 MB-4 GB inp, 150-175 G/s from an L2-resident
// one, where the L1 tag lookups of 64 scattered lanes per instruction set the pace; 2 to 8
// vectors per thread instead of 1 changed that by at most 4%).  A thread owns 4 consecutive
// elements: with 16-byte aligned index and output arrays it reads both index quadruples with
// one 16-byte load each, issues its four inp loads before it needs any of them, and writes the
// four results with one 16-byte store (index and output streams non-temporal; inp is read
// through the caches, which catch repeated and neighbouring indices).  Otherwise each thread
// takes single elements.
#include "common.hpp"

namespace ihip {

typedef int32_t i32x4_g __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float gather_one(const float* __restrict__ inp, int32_t r, int32_t c, int64_t M, int64_t N,
                                            float other) {
  // one unsigned comparison per index: a negative index is far above any extent
  const bool ok = static_cast<uint64_t>(static_cast<int64_t>(r)) < static_cast<uint64_t>(M) &&
                  static_cast<uint64_t>(static_cast<int64_t>(c)) < static_cast<uint64_t>(N);
  return ok ? inp[static_cast<int64_t>(r) * N + c] : other;
}

__global__ __launch_bounds__(256) void gather2d_f32_vec(const float* __restrict__ inp, const i32x4_g* __restrict__ row,
                                                        const i32x4_g* __restrict__ col, f32x4* __restrict__ out,
                                                        int64_t M, int64_t N, int64_t L4, float other) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q >= L4) return;
  const i32x4_g r = __builtin_nontemporal_load(row + q);
  const i32x4_g c = __builtin_nontemporal_load(col + q);
  const f32x4 v = {gather_one(inp, r.x, c.x, M, N, other), gather_one(inp, r.y, c.y, M, N, other),
                   gather_one(inp, r.z, c.z, M, N, other), gather_one(inp, r.w, c.w, M, N, other)};
  __builtin_nontemporal_store(v, out + q);
}

// Elements first .. L-1, one per thread (the tail of the vector form, or every element when the
// arrays are not 16-byte aligned).
__global__ __launch_bounds__(256) void gather2d_f32_any(const float* __restrict__ inp, const int32_t* __restrict__ row,
                                                        const int32_t* __restrict__ col, float* __restrict__ out,
                                                        int64_t M, int64_t N, int64_t first, int64_t L, float other) {
  const int64_t i = first + static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= L) return;
  out[i] = gather_one(inp, row[i], col[i], M, N, other);
}

hipError_t launch_gather2d_f32(const float* inp, const int32_t* row, const int32_t* col, float* out, int64_t M,
                               int64_t N, int64_t L, float other, hipStream_t s) {
  if (L == 0) return hipSuccess;
  const bool vec = ((reinterpret_cast<uintptr_t>(row) | reinterpret_cast<uintptr_t>(col) |
                     reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  const int64_t L4 = vec ? L / 4 : 0;
  if (L4 > 0) {
    const int64_t blocks = (L4 + 255) / 256;
    if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
    gather2d_f32_vec<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s>>>(
        inp, reinterpret_cast<const i32x4_g*>(row), reinterpret_cast<const i32x4_g*>(col), reinterpret_cast<f32x4*>(out),
        M, N, L4, other);
  }
  const int64_t rest = L - 4 * L4;
  if (rest > 0) {
    const int64_t blocks = (rest + 255) / 256;
    if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
    gather2d_f32_any<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s>>>(inp, row, col, out, M, N, 4 * L4, L,
                                                                               other);
  }
  return hipGetLastError();
}

}  // namespace ihip
