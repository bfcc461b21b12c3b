// CSR SpMM out = A * dense, f32 values and features, i32 indices, for gfx950.
//
// Semantics: csr_spmm (python/intent/examples/kernels/sparse/csr_spmm.py:11-33). For every row r
// and feature f: acc = 0; for nz in [row_offsets[r], row_offsets[r+1]) in order,
// acc = acc + values[nz] * dense[column_indices[nz], f] with the product rounded before the add
// (no fused multiply-add); out[r, f] = acc. The fold order is the definition's, so results are
// bit-identical to it. Columns outside [0, cols) read row cols - 1 and offsets are clamped to
// [0, nnz] (the definition assumes both in bounds), so bad indices cannot fault.
//
// Design: the dense operand ([cols, features] f32, 4 MB at the reference shape) is re-read once
// per nonzero, so the kernel is bound by L2/MALL gather bandwidth; the HBM algorithmic bytes are
// the CSR arrays, dense once and the output. One wave per row (the row index is wave-uniform,
// so its offsets come through scalar loads); lanes own features, 2 per lane (8-byte loads, each
// gather a contiguous 512 B) when the layout allows, 1 otherwise. The row's (column, value) pairs
// arrive 64 at a time in one coalesced load and are broadcast by v_readlane; 16 gathers are
// issued together, then folded in order.
#include "common.hpp"

namespace intent_hip {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 64;
constexpr int kBatch = 16;

// acc + v * d with the product rounded before the add: contraction into an FMA is switched off
// here, whatever the file-wide floating-point options say.
__device__ __forceinline__ float fold(float acc, float v, float d) {
#pragma clang fp contract(off)
  const float product = v * d;
  return acc + product;
}

template <int kVec>   // features per lane: 2 (float2 loads) or 1
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(8))) void csr_spmm_rows(const int32_t *__restrict__ off,
                                                          const int32_t *__restrict__ col,
                                                          const float *__restrict__ val,
                                                          const float *__restrict__ dense, float *__restrict__ out,
                                                          int rows, int cols, int nnz, int features, int64_t ldd,
                                                          int64_t ldo) {
  typedef float vec_t __attribute__((ext_vector_type(kVec)));
  const int lane = threadIdx.x & 63;
  const int row = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x) * kRowsPerBlock +
                                                 static_cast<int>(threadIdx.x >> 6));
  if (row >= rows) return;
  int start = off[row], stop = off[row + 1];
  start = start < 0 ? 0 : (start > nnz ? nnz : start);
  stop = stop < start ? start : (stop > nnz ? nnz : stop);
  for (int f0 = 0; f0 < features; f0 += 64 * kVec) {
    const int f = f0 + lane * kVec;
    const bool in = f < features;                 // features % kVec == 0 on the vector path
    vec_t acc = {};
    for (int base = start; base < stop; base += 64) {
      // Up to 64 (column, value) pairs in one coalesced load; lane j holds pair base + j.
      const int n = stop - base < 64 ? stop - base : 64;
      int column = 0;
      float value = 0.0f;
      if (lane < n) {
        const int c = col[base + lane];
        column = static_cast<uint32_t>(c) < static_cast<uint32_t>(cols) ? c : cols - 1;
        value = val[base + lane];
      }
      for (int j0 = 0; j0 < n; j0 += kBatch) {
        vec_t d[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          d[j] = vec_t{};
          const int64_t r = __builtin_amdgcn_readlane(column, j0 + j);
          if (j0 + j < n && in) d[j] = *reinterpret_cast<const vec_t *>(dense + r * ldd + f);
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          if (j0 + j < n) {
            const float v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, value), j0 + j));
#pragma unroll
            for (int e = 0; e < kVec; ++e) acc[e] = fold(acc[e], v, d[j][e]);
          }
        }
      }
    }
    if (in) *reinterpret_cast<vec_t *>(out + row * ldo + f) = acc;
  }
}

}  // namespace

int spmm_resources(int64_t features, IntentHipKernelResources *out) {
  if (features % 2 == 0)
    return describe_kernel(reinterpret_cast<const void *>(&csr_spmm_rows<2>), "csr_spmm_rows<2>", kThreads, out);
  return describe_kernel(reinterpret_cast<const void *>(&csr_spmm_rows<1>), "csr_spmm_rows<1>", kThreads, out);
}

}  // namespace intent_hip

using namespace intent_hip;

extern "C" int intent_hip_csr_spmm_f32(const int32_t *row_offsets, const int32_t *column_indices,
                                       const float *values, const float *dense, float *out, int64_t rows,
                                       int64_t cols, int64_t nnz, int64_t features, int64_t ldd, int64_t ldo,
                                       void *stream) {
  if (rows < 0 || cols < 0 || nnz < 0 || features < 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (rows >= INT32_MAX || nnz > INT32_MAX || cols > INT32_MAX || features > INT32_MAX)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "extents must stay below 2^31 (32-bit CSR indices)");
  if (rows == 0 || features == 0) return INTENT_HIP_OK;
  if (nnz > 0 && cols == 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "nonzeros in a matrix with no columns");
  if (ldd < features || ldo < features) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "row stride below the row width");
  if (row_offsets == nullptr || out == nullptr ||
      (nnz > 0 && (column_indices == nullptr || values == nullptr || dense == nullptr)))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null tensor pointer");
  const bool vector = features % 2 == 0 && ldd % 2 == 0 && ldo % 2 == 0 && aligned(dense, 8) && aligned(out, 8);
  const dim3 grid(static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock));
  const hipStream_t s = as_stream(stream);
  const int r32 = static_cast<int>(rows), c32 = cols > 0 ? static_cast<int>(cols) : 1;
  if (vector)
    csr_spmm_rows<2><<<grid, dim3(kThreads), 0, s>>>(row_offsets, column_indices, values, dense, out, r32, c32,
                                                    static_cast<int>(nnz), static_cast<int>(features), ldd, ldo);
  else
    csr_spmm_rows<1><<<grid, dim3(kThreads), 0, s>>>(row_offsets, column_indices, values, dense, out, r32, c32,
                                                    static_cast<int>(nnz), static_cast<int>(features), ldd, ldo);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("csr_spmm_rows");
  return INTENT_HIP_OK;
}
