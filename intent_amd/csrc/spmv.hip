// CSR SpMV y = A x (f32 values, i32 indices) for gfx950.
//
// Semantics (python/intent/examples/kernels/sparse/csr_spmv.py:11-29): for every row,
// acc = 0.0f; for nz in [off[r], off[r+1]) in order: acc = acc + values[nz] * x[col[nz]];
// y[r] = acc. Index traversal is exact; the product is rounded to f32 before the add
// (no fused multiply-add), so any row that one thread folds alone reproduces the
// ordered loop bit for bit. Longer rows are split and their partial sums combined in a
// fixed, data-independent order (left part + right part), which reassociates the fold.
//
// Design: merge-path partition (Merrill & Garland, "Merge-based parallel sparse
// matrix-vector multiplication", SC'16). The work items are the R row ends merged with
// the NNZ nonzeros; every workgroup takes exactly kBlockItems of them and every thread
// kItems, whatever the row-length distribution (4M rows of length 1 next to rows of
// 65536). Launches:
//   1. partition: one thread per row writes the row that contains each workgroup's
//      starting diagonal (no searches in global memory);
//   2. placement (place, place_fill): logical workgroups inside one long row are
//      mapped to the XCD whose L2 serves their column window; the rest fill free slots;
//   3. merge: a workgroup stages its row ends and its products values*x[col] in LDS
//      (coalesced non-temporal col/value loads that do not evict x from L2, gathers of
//      x), each thread searches its diagonal in LDS and folds kItems items in order;
//      partial rows are combined by a segmented scan across the workgroup; the partial
//      row left open at the workgroup's end goes to the workspace;
//   4. fixup: the first workgroup of each run of equal open rows adds the run's
//      partials (in workgroup order) to y.
// Placement changes only which hardware workgroup runs a logical block, never what the
// block computes, so results do not depend on it.
#include "common.hpp"

namespace intent_hip {
namespace {

constexpr int kThreads = 256;
constexpr int kItems = 8;
constexpr int kBlockItems = kThreads * kItems;

inline size_t align256(size_t bytes) { return (bytes + 255) & ~static_cast<size_t>(255); }

struct Workspace {
  int32_t *splits;      // [blocks + 1]: row of each workgroup's starting diagonal
  int32_t *carry_rows;  // [blocks]: row left open at the workgroup's end, -1 if none
  float *carry_values;  // [blocks]: its partial sum
  int32_t *perm;        // [blocks]: logical block run by hardware workgroup h
  int32_t *overflow;    // [blocks]: logical blocks not placed on their XCD
  int32_t *counters;    // [64]: per-XCD fill counts, overflow count
};

size_t workspace_bytes(int64_t blocks) {
  return align256(4 * static_cast<size_t>(blocks + 1)) + 4 * align256(4 * static_cast<size_t>(blocks)) + 256;
}

Workspace carve(void *base, int64_t blocks) {
  char *p = static_cast<char *>(base);
  Workspace w;
  w.splits = reinterpret_cast<int32_t *>(p);
  p += align256(4 * static_cast<size_t>(blocks + 1));
  w.carry_rows = reinterpret_cast<int32_t *>(p);
  p += align256(4 * static_cast<size_t>(blocks));
  w.carry_values = reinterpret_cast<float *>(p);
  p += align256(4 * static_cast<size_t>(blocks));
  w.perm = reinterpret_cast<int32_t *>(p);
  p += align256(4 * static_cast<size_t>(blocks));
  w.overflow = reinterpret_cast<int32_t *>(p);
  p += align256(4 * static_cast<size_t>(blocks));
  w.counters = reinterpret_cast<int32_t *>(p);
  return w;
}

constexpr int kXcds = 8;

// Hardware workgroup h runs on XCD h % 8. A logical block whose items all lie inside one row
// gathers x from a narrow column window (columns are sorted within a row); it is placed on the
// XCD that owns that eighth of the columns, so its gathers come from that XCD's L2. Other blocks
// fill the remaining slots. Each logical block computes the same result wherever it runs.
__global__ __launch_bounds__(kThreads) void spmv_place(const int32_t *__restrict__ col, int32_t cols,
                                                       int32_t blocks, int64_t total, int64_t nnz,
                                                       Workspace ws) {
  // Slots are reserved per workgroup: LDS atomics rank the threads, then one global atomic
  // per XCD (and one for the overflow list) reserves the workgroup's range.
  __shared__ int32_t s_count[kXcds + 1];
  __shared__ int32_t s_base[kXcds + 1];
  const int t = threadIdx.x;
  const int64_t g = static_cast<int64_t>(blockIdx.x) * kThreads + t;
  if (t <= kXcds) s_count[t] = 0;
  __syncthreads();
  int xcd = -1;
  if (g < blocks) {
    const int32_t x0 = ws.splits[g], x1 = ws.splits[g + 1];
    const int64_t y0 = g * kBlockItems - x0;
    const int64_t d1 = (g + 1) * kBlockItems < total ? (g + 1) * kBlockItems : total;
    const int64_t y1 = d1 - x1;
    if (x1 - x0 <= 1 && y1 - y0 >= kBlockItems / 2 && y0 >= 0 && y1 <= nnz) {
      const int64_t mid = (y0 + y1) / 2;
      xcd = static_cast<int>((static_cast<int64_t>(col[mid]) * kXcds) / cols);
      xcd = xcd < 0 ? 0 : (xcd >= kXcds ? kXcds - 1 : xcd);
    }
  }
  const int32_t local = xcd >= 0 ? atomicAdd(&s_count[xcd], 1) : 0;
  __syncthreads();
  if (t < kXcds) s_base[t] = s_count[t] > 0 ? atomicAdd(&ws.counters[t], s_count[t]) : 0;
  __syncthreads();
  bool spill = g < blocks;
  if (xcd >= 0) {
    const int32_t capacity = (blocks - xcd + kXcds - 1) / kXcds;   // slots h = xcd + 8 i < blocks
    const int32_t slot = s_base[xcd] + local;
    if (slot < capacity) {
      ws.perm[xcd + kXcds * slot] = static_cast<int32_t>(g);
      spill = false;
    }
  }
  const int32_t rank = spill ? atomicAdd(&s_count[kXcds], 1) : 0;
  __syncthreads();
  if (t == 0) s_base[kXcds] = s_count[kXcds] > 0 ? atomicAdd(&ws.counters[kXcds], s_count[kXcds]) : 0;
  __syncthreads();
  if (spill) ws.overflow[s_base[kXcds] + rank] = static_cast<int32_t>(g);
}

__global__ __launch_bounds__(kThreads) void spmv_place_fill(int32_t blocks, Workspace ws) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (j >= ws.counters[kXcds]) return;
  // Free slots of XCD e are i in [filled_e, capacity_e); enumerate them XCD by XCD.
  int64_t rank = j;
  for (int e = 0; e < kXcds; ++e) {
    const int32_t capacity = (blocks - e + kXcds - 1) / kXcds;
    const int32_t filled = min(ws.counters[e], capacity);
    const int32_t free_slots = capacity - filled;
    if (rank < free_slots) {
      ws.perm[e + kXcds * (filled + rank)] = ws.overflow[j];
      return;
    }
    rank -= free_slots;
  }
}

// Row r owns the diagonals [off[r] + r, off[r+1] + r + 1): its nonzeros, then its end.
// It records itself as the split of every workgroup boundary g * kBlockItems inside that range.
// Workgroup 0 also clears the placement counters (a store, not a memset node, so the launch
// sequence can be captured in a graph).
__global__ __launch_bounds__(kThreads) void spmv_partition(const int32_t *__restrict__ off, int32_t rows,
                                                           int32_t blocks, int32_t *__restrict__ splits,
                                                           int32_t *__restrict__ counters) {
  if (blockIdx.x == 0 && threadIdx.x < 64) counters[threadIdx.x] = 0;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (r > rows) return;
  if (r == rows) {
    splits[blocks] = rows;
    return;
  }
  const int64_t begin = static_cast<int64_t>(off[r]) + r;
  const int64_t end = static_cast<int64_t>(off[r + 1]) + r + 1;
  int64_t g = (begin + kBlockItems - 1) / kBlockItems;
  int64_t last = (end - 1) / kBlockItems;
  if (g < 0) g = 0;
  if (last > blocks - 1) last = blocks - 1;
  for (; g <= last; ++g) splits[g] = static_cast<int32_t>(r);
}

__global__ __launch_bounds__(kThreads) void spmv_merge(const int32_t *__restrict__ off,
                                                       const int32_t *__restrict__ col,
                                                       const float *__restrict__ val,
                                                       const float *__restrict__ x, float *__restrict__ y,
                                                       int32_t rows, int32_t cols, int64_t total,
                                                       Workspace ws) {
  __shared__ int32_t s_end[kBlockItems + 1];  // row ends of this workgroup, relative to y0
  __shared__ float s_prod[kBlockItems];       // values * x[col] of this workgroup's nonzeros
  __shared__ int32_t s_key[kThreads];
  __shared__ float s_val[kThreads];

  const int t = threadIdx.x;
  const int32_t placed = ws.perm[blockIdx.x];  // a permutation of [0, gridDim.x) by construction
  const int64_t g = placed < 0 ? 0 : (placed >= static_cast<int32_t>(gridDim.x) ? gridDim.x - 1 : placed);
  const int64_t d0 = g * kBlockItems;
  const int64_t d1 = d0 + kBlockItems < total ? d0 + kBlockItems : total;
  const int32_t x0 = ws.splits[g];
  const int32_t x1 = ws.splits[g + 1];
  const int64_t y0 = d0 - x0;
  // Row ends completed inside this workgroup (local rows 0..n_ends-1) and nonzeros.
  int32_t n_ends = x1 - x0;
  int32_t n_nz = static_cast<int32_t>((d1 - x1) - y0);
  // Defensive clamps: valid CSR input always satisfies them.
  n_ends = n_ends < 0 ? 0 : (n_ends > kBlockItems ? kBlockItems : n_ends);
  n_nz = n_nz < 0 ? 0 : (n_nz > kBlockItems ? kBlockItems : n_nz);

  for (int i = t; i < n_ends; i += kThreads) s_end[i] = static_cast<int32_t>(off[x0 + i + 1] - y0);
  {
    int32_t c[kItems];
    float v[kItems];
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
      const int i = t + k * kThreads;
      const bool live = i < n_nz;
      c[k] = live ? __builtin_nontemporal_load(col + y0 + i) : 0;
      v[k] = live ? __builtin_nontemporal_load(val + y0 + i) : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
      const int i = t + k * kThreads;
      if (i < n_nz) {
        const uint32_t column = static_cast<uint32_t>(c[k]) < static_cast<uint32_t>(cols) ? c[k] : cols - 1;
        s_prod[i] = __fmul_rn(v[k], x[column]);
      }
    }
  }
  __syncthreads();

  // This thread's local diagonal range and its starting merge coordinate.
  const int32_t items = n_ends + n_nz;
  const int32_t dt = t * kItems < items ? t * kItems : items;
  const int32_t dt_end = dt + kItems < items ? dt + kItems : items;
  int32_t lo = dt - n_nz > 0 ? dt - n_nz : 0;
  int32_t hi = dt < n_ends ? dt : n_ends;
  while (lo < hi) {
    const int32_t mid = (lo + hi) >> 1;
    if (s_end[mid] <= dt - mid - 1) lo = mid + 1;
    else hi = mid;
  }
  int32_t xt = lo;
  int32_t yt = dt - lo;

  float acc = 0.0f;
  float head = 0.0f;
  int32_t head_row = -1;
  for (int32_t d = dt; d < dt_end; ++d) {
    if (xt < n_ends && s_end[xt] <= yt) {
      if (head_row < 0) {
        head_row = xt;
        head = acc;
      } else {
        y[x0 + xt] = acc;
      }
      acc = 0.0f;
      ++xt;
    } else if (yt < n_nz) {
      acc = __fadd_rn(acc, s_prod[yt]);
      ++yt;
    }
  }

  // Segmented inclusive scan of the open-row partials (keys are non-decreasing).
  s_key[t] = xt;
  s_val[t] = acc;
  float scanned = acc;
  for (int offset = 1; offset < kThreads; offset <<= 1) {
    __syncthreads();
    const float add = (t >= offset && s_key[t - offset] == xt) ? s_val[t - offset] : 0.0f;
    __syncthreads();
    scanned = __fadd_rn(scanned, add);
    s_val[t] = scanned;
  }
  __syncthreads();
  if (head_row >= 0) {
    const float carry = t > 0 ? s_val[t - 1] : 0.0f;
    y[x0 + head_row] = __fadd_rn(carry, head);
  }
  if (t == kThreads - 1) {
    const int64_t open_row = static_cast<int64_t>(x0) + xt;
    ws.carry_rows[g] = open_row < rows ? static_cast<int32_t>(open_row) : -1;
    ws.carry_values[g] = scanned;
  }
}

__global__ __launch_bounds__(kThreads) void spmv_fixup(float *__restrict__ y, int32_t blocks, Workspace ws) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (g >= blocks) return;
  const int32_t r = ws.carry_rows[g];
  if (r < 0 || (g > 0 && ws.carry_rows[g - 1] == r)) return;
  float sum = ws.carry_values[g];
  for (int64_t h = g + 1; h < blocks && ws.carry_rows[h] == r; ++h) sum = __fadd_rn(sum, ws.carry_values[h]);
  y[r] = __fadd_rn(sum, y[r]);
}

int64_t block_count(int64_t rows, int64_t nnz) { return (rows + nnz + kBlockItems - 1) / kBlockItems; }

}  // namespace

int spmv_resources(int64_t rows, int64_t nnz, IntentHipKernelResources *out) {
  (void)rows;
  (void)nnz;
  return describe_kernel(reinterpret_cast<const void *>(&spmv_merge), "spmv_merge", kThreads, out);
}

}  // namespace intent_hip

using namespace intent_hip;

extern "C" int intent_hip_csr_spmv_workspace_bytes(int64_t rows, int64_t nnz, size_t *bytes) {
  if (bytes == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null output");
  if (rows < 0 || nnz < 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  *bytes = workspace_bytes(block_count(rows, nnz));
  return INTENT_HIP_OK;
}

extern "C" int intent_hip_csr_spmv_f32(const int32_t *row_offsets, const int32_t *column_indices,
                                       const float *values, const float *x, float *y, int64_t rows,
                                       int64_t cols, int64_t nnz, void *workspace, size_t workspace_size,
                                       void *stream) {
  if (rows < 0 || cols < 0 || nnz < 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (rows + nnz > INT32_MAX)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "rows + nnz must stay below 2^31 (32-bit CSR indices)");
  if (rows == 0) return INTENT_HIP_OK;
  if (nnz > 0 && cols == 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "nonzeros in a matrix with no columns");
  if (row_offsets == nullptr || y == nullptr || (nnz > 0 && (column_indices == nullptr || values == nullptr || x == nullptr)))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null tensor pointer");
  const int64_t blocks = block_count(rows, nnz);
  if (workspace == nullptr || workspace_size < workspace_bytes(blocks))
    return fail(INTENT_HIP_ERR_WORKSPACE, "SpMV needs %zu workspace bytes, got %zu", workspace_bytes(blocks),
                workspace_size);
  const Workspace ws = carve(workspace, blocks);
  const hipStream_t s = as_stream(stream);
  const int32_t r32 = static_cast<int32_t>(rows), b32 = static_cast<int32_t>(blocks);
  const int32_t c32 = cols > INT32_MAX ? INT32_MAX : static_cast<int32_t>(cols);
  const int64_t total = rows + nnz;
  spmv_partition<<<dim3(static_cast<unsigned>((rows + 1 + kThreads - 1) / kThreads)), dim3(kThreads), 0, s>>>(
      row_offsets, r32, b32, ws.splits, ws.counters);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("spmv_partition");
  spmv_place<<<dim3(static_cast<unsigned>((blocks + kThreads - 1) / kThreads)), dim3(kThreads), 0, s>>>(
      column_indices, c32 > 0 ? c32 : 1, b32, total, nnz, ws);
  spmv_place_fill<<<dim3(static_cast<unsigned>((blocks + kThreads - 1) / kThreads)), dim3(kThreads), 0, s>>>(b32, ws);
  spmv_merge<<<dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s>>>(row_offsets, column_indices, values, x,
                                                                             y, r32, c32, total, ws);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("spmv_merge");
  spmv_fixup<<<dim3(static_cast<unsigned>((blocks + kThreads - 1) / kThreads)), dim3(kThreads), 0, s>>>(y, b32, ws);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("spmv_fixup");
  return INTENT_HIP_OK;
}
