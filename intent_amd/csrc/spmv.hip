// CSR SpMV y = A x (f32 values, i32 indices) for gfx950.
//
// Semantics (python/intent/examples/kernels/sparse/csr_spmv.py:11-29): for every row,
// acc = 0.0f; for nz in [off[r], off[r+1]) in order: acc = acc + values[nz] * x[col[nz]];
// y[r] = acc. Positions are absolute, so off[0] may be above 0 and off[R] below nnz (a row slice
// of a larger CSR). Index traversal is exact. Rows of up to 4 nonzeros are folded by one lane in
// order, with each product rounded before the add (no fused multiply-add): that reproduces the
// ordered loop bit for bit. Longer rows are split into pieces whose partial sums are combined in a
// fixed, data-independent order, a reassociation of the fold.
//
// Design. The cost of this operator is the gather of x, one per nonzero. A gather that hits L2 is
// still one L2 request: at config 5 (67M nonzeros), gathers confined to an L2-resident window of
// x took 300 us of a 450 us merge-path kernel, and the real gathers (61% L2 hits) 470 us of 615.
// Rows are therefore classed by length:
//   * up to 4 nonzeros: one lane per row, ordered fold (spmv_rows, four rows per thread with
//     their loads issued together);
//   * 5 to 127: 16 lanes per row (spmv_rows);
//   * medium (128 to big - 1): the row is cut at the boundaries of 8 column windows of C / 8
//     columns, the share of x one XCD's 4 MB L2 holds, and the piece in window w runs on XCD w
//     (hardware workgroup h runs on XCD h % 8), so its gathers hit that L2 (spmv_windows);
//   * large (big = max(128, 32 S) or more): the row is cut at the boundaries of S slices of 32768
//     columns; a workgroup stages one slice of x (128 KB) in LDS and runs that slice's piece of
//     many large rows, gathering from LDS (spmv_slices).
// Each piece runs on one wave: coalesced loads of its columns and values, one reduction per piece.
// The medium and large row lists are built without atomics: spmv_count counts each 1024-row
// block's rows of each class, and the totals of each group of 4 blocks; spmv_rows sums the
// totals and counts before a block into its list offset and writes the block's rows there in row
// order. (Wave-level atomics on two list counters cost 115 us at config 5; a one-workgroup scan
// launch between the two kernels cost 9 us.) The cut workgroups of spmv_rows estimate each cut by
// interpolation search and make the cuts of a row non-decreasing with a prefix maximum, so the
// pieces partition the row for any estimate and any column order; an entry outside its window or
// slice only reads x from another place. spmv_combine adds the pieces of each medium or large row
// in window or slice order.
#include <algorithm>
#include <mutex>

#include "common.hpp"

namespace intent_hip {
namespace {

constexpr int kLaneRow = 4;         // rows of up to 4 nonzeros: one lane, exact ordered fold
constexpr int kGroupRow = 128;      // rows below 128 nonzeros: 16 lanes
constexpr int kGroup = 16;
constexpr int kRowsPerThread = 4;   // spmv_rows: 1024 rows per 256-thread workgroup
constexpr int kBlockRows = 256 * kRowsPerThread;
constexpr int kSuperBlocks = 4;     // spmv_count: four blocks per 1024-thread workgroup
constexpr int kWindows = 8;         // one column window per XCD
constexpr int kSliceCols = 32768;   // 128 KB of x in LDS per workgroup
constexpr int kSliceTiles = 256;    // slice workgroups per launch: one per CU, all resident at once
constexpr int kWindowTiles = 64;    // medium-row workgroups per window (two per CU of the XCD)
constexpr int kSearchSteps = 8;     // interpolation steps per cut

inline size_t align256(size_t bytes) { return (bytes + 255) & ~static_cast<size_t>(255); }

// Row classes and the workspace carved for them.
struct Plan {
  int32_t *counters;      // [64]: [0] medium rows, [1] large rows
  int32_t *block_counts;  // [blocks][2]: medium and large rows of each 1024-row block
  int32_t *super_counts;  // [supers][2]: the same of each group of kSuperBlocks blocks
  int32_t *mid_rows;      // [cap_mid] row ids of medium rows, in row order
  int32_t *big_rows;      // [cap_big]
  int32_t *mid_cuts;      // [cap_mid][9]: piece w is [cut w, cut w + 1)
  float *mid_parts;       // [cap_mid][8]
  int32_t *big_cuts;      // [cap_big][slices + 1]
  float *big_parts;       // [cap_big][slices]
  int32_t cap_mid, cap_big, slices, big, blocks, supers;
};

int64_t slice_count(int64_t cols) { return cols > 0 ? (cols + kSliceCols - 1) / kSliceCols : 1; }
// Rows of at least big = max(128, 32 S) nonzeros (32 per slice on average) are large.
int64_t big_length(int64_t slices) { const int64_t l = slices * (kSliceCols / 1024); return l > kGroupRow ? l : kGroupRow; }
int64_t mid_capacity(int64_t rows, int64_t nnz) { return nnz / kGroupRow < rows ? nnz / kGroupRow : rows; }
int64_t big_capacity(int64_t rows, int64_t nnz, int64_t slices) {
  const int64_t by_nnz = nnz / big_length(slices);
  return by_nnz < rows ? by_nnz : rows;
}
int64_t block_count(int64_t rows) { return (rows + kBlockRows - 1) / kBlockRows; }
int64_t super_count(int64_t rows) { return (block_count(rows) + kSuperBlocks - 1) / kSuperBlocks; }
// Entries (cuts plus parts plus row ids) of the large-row region: cap_big * (2 S + 2) <= 18 nnz / 128
// for every slice count S, so the bound below holds whatever the column count.
int64_t big_entries_bound(int64_t nnz) { return (18 * nnz + 127) / 128 + 64; }

size_t workspace_bytes(int64_t rows, int64_t nnz) {
  const int64_t cap_mid = mid_capacity(rows, nnz);
  return 256 + align256(8 * static_cast<size_t>(block_count(rows))) + align256(8 * static_cast<size_t>(super_count(rows))) +
         align256(4 * static_cast<size_t>(cap_mid)) +
         align256(36 * static_cast<size_t>(cap_mid)) + align256(32 * static_cast<size_t>(cap_mid)) +
         align256(4 * static_cast<size_t>(big_entries_bound(nnz))) + 1024;
}

Plan carve(void *base, int64_t rows, int64_t cols, int64_t nnz) {
  Plan p;
  p.slices = static_cast<int32_t>(slice_count(cols));
  p.big = static_cast<int32_t>(big_length(p.slices));
  p.cap_mid = static_cast<int32_t>(mid_capacity(rows, nnz));
  p.cap_big = static_cast<int32_t>(big_capacity(rows, nnz, p.slices));
  p.blocks = static_cast<int32_t>(block_count(rows));
  p.supers = static_cast<int32_t>(super_count(rows));
  char *c = static_cast<char *>(base);
  p.counters = reinterpret_cast<int32_t *>(c);
  c += 256;
  p.block_counts = reinterpret_cast<int32_t *>(c);
  c += align256(8 * static_cast<size_t>(p.blocks));
  p.super_counts = reinterpret_cast<int32_t *>(c);
  c += align256(8 * static_cast<size_t>(p.supers));
  p.mid_rows = reinterpret_cast<int32_t *>(c);
  c += align256(4 * static_cast<size_t>(p.cap_mid));
  p.mid_cuts = reinterpret_cast<int32_t *>(c);
  c += align256(36 * static_cast<size_t>(p.cap_mid));
  p.mid_parts = reinterpret_cast<float *>(c);
  c += align256(32 * static_cast<size_t>(p.cap_mid));
  p.big_rows = reinterpret_cast<int32_t *>(c);
  c += align256(4 * static_cast<size_t>(p.cap_big));
  p.big_cuts = reinterpret_cast<int32_t *>(c);
  c += align256(4 * static_cast<size_t>(p.cap_big) * (p.slices + 1));
  p.big_parts = reinterpret_cast<float *>(c);
  return p;
}

__device__ __forceinline__ int32_t clamp_col(int32_t c, int32_t cols) {
  return static_cast<uint32_t>(c) < static_cast<uint32_t>(cols) ? c : cols - 1;
}

// Row r's nonzeros [begin, end), clamped into [0, nnz] (valid CSR never needs the clamp).
__device__ __forceinline__ void row_span(const int32_t *off, int64_t r, int64_t nnz, int32_t &begin, int32_t &end) {
  const int64_t b = off[r], e = off[r + 1];
  const int64_t cb = b < 0 ? 0 : (b > nnz ? nnz : b);
  const int64_t ce = e < cb ? cb : (e > nnz ? nnz : e);
  begin = static_cast<int32_t>(cb);
  end = static_cast<int32_t>(ce);
}

__device__ __forceinline__ float group16_sum(float v) {
  v += __shfl_xor(v, 8);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 1);
  return v;
}

__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
  return v;
}

// Medium and large rows of every 1024-row block, and of every group of kSuperBlocks blocks (a
// superblock): threads 256 p .. 256 p + 255 of workgroup g count block kSuperBlocks g + p, four rows
// each (rows base + t + 256 k, their offset loads issued together).
__global__ __launch_bounds__(256 * kSuperBlocks) void spmv_count(const int32_t *__restrict__ off, int32_t rows,
                                                               int64_t nnz, Plan plan) {
  __shared__ int s_part[2][4 * kSuperBlocks];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int part = threadIdx.x >> 8, t = threadIdx.x & 255;
  const int block = static_cast<int>(blockIdx.x) * kSuperBlocks + part;
  const int64_t base = static_cast<int64_t>(block) * kBlockRows;
  int mid = 0, big = 0;
  int32_t b[kRowsPerThread], e[kRowsPerThread];
#pragma unroll
  for (int k = 0; k < kRowsPerThread; ++k) {
    const int64_t r = base + t + 256 * k;
    b[k] = e[k] = 0;
    if (block < plan.blocks && r < rows) row_span(off, r, nnz, b[k], e[k]);
  }
#pragma unroll
  for (int k = 0; k < kRowsPerThread; ++k) {
    mid += (e[k] - b[k] >= kGroupRow && e[k] - b[k] < plan.big) ? 1 : 0;
    big += (e[k] - b[k] >= plan.big) ? 1 : 0;
  }
  mid = wave_sum_int(mid);
  big = wave_sum_int(big);
  if (lane == 0) {
    s_part[0][wave] = mid;
    s_part[1][wave] = big;
  }
  __syncthreads();
  if (threadIdx.x < 2 * kSuperBlocks) {   // block counts: thread 2 p + c
    const int p = threadIdx.x >> 1, c = threadIdx.x & 1;
    const int blk = static_cast<int>(blockIdx.x) * kSuperBlocks + p;
    if (blk < plan.blocks)
      plan.block_counts[2 * blk + c] = s_part[c][4 * p] + s_part[c][4 * p + 1] + s_part[c][4 * p + 2] + s_part[c][4 * p + 3];
  } else if (threadIdx.x < 2 * kSuperBlocks + 2) {   // superblock totals
    const int c = threadIdx.x - 2 * kSuperBlocks;
    int total = 0;
#pragma unroll
    for (int w = 0; w < 4 * kSuperBlocks; ++w) total += s_part[c][w];
    plan.super_counts[2 * blockIdx.x + c] = total;
  }
}

// Medium and large rows in the superblocks before `super`, summed by every thread of a 256-thread
// workgroup (all of them call it); `s_pre` is the workgroup's LDS scratch. Every thread gets both.
__device__ __forceinline__ void superblock_prefix(const Plan &plan, int super, int &mid_before, int &big_before,
                                                  int (*s_pre)[4]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int mid = 0, big = 0;
  for (int s = threadIdx.x; s < super; s += 256) {
    mid += plan.super_counts[2 * s];
    big += plan.super_counts[2 * s + 1];
  }
  mid = wave_sum_int(mid);
  big = wave_sum_int(big);
  if (lane == 0) {
    s_pre[0][wave] = mid;
    s_pre[1][wave] = big;
  }
  __syncthreads();
  mid_before = s_pre[0][0] + s_pre[0][1] + s_pre[0][2] + s_pre[0][3];
  big_before = s_pre[1][0] + s_pre[1][1] + s_pre[1][2] + s_pre[1][3];
  __syncthreads();   // s_pre may be written again
}

// The list offsets of `block`: the superblocks before its own, then its own superblock's blocks
// before it (at most kSuperBlocks - 1 counts, read by every lane).
__device__ __forceinline__ void block_prefix(const Plan &plan, int block, int mid_super, int big_super, int &first_mid,
                                             int &first_big) {
  first_mid = mid_super;
  first_big = big_super;
  for (int j = block / kSuperBlocks * kSuperBlocks; j < block; ++j) {
    first_mid += plan.block_counts[2 * j];
    first_big += plan.block_counts[2 * j + 1];
  }
}

// Short rows and the row lists. Rows base + tid + 256 k of the block: rows of up to 4 nonzeros are
// folded by their lane (the loads of the thread's four rows issued together); rows of 5..127 by a
// 16-lane group (four rows per wave at a time); medium and large rows are written to their lists
// at the block's list offset (block_prefix), in row order.
__device__ __forceinline__ void rows_block(const int32_t *__restrict__ off, const int32_t *__restrict__ col,
                                           const float *__restrict__ val, const float *__restrict__ x,
                                           float *__restrict__ y, int32_t rows, int32_t cols, int64_t nnz, Plan plan,
                                           int block) {
  __shared__ int s_wave[2][4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t base = static_cast<int64_t>(block) * kBlockRows;
  int32_t begin[kRowsPerThread], length[kRowsPerThread];
#pragma unroll
  for (int k = 0; k < kRowsPerThread; ++k) {
    const int64_t r = base + threadIdx.x + 256 * k;
    int32_t b = 0, e = 0;
    if (r < rows) row_span(off, r, nnz, b, e);
    begin[k] = b;
    length[k] = r < rows ? e - b : -1;
  }
  // Lane rows: all column and value loads, then all gathers, then the ordered folds.
  {
    int32_t c[kRowsPerThread][kLaneRow];
    float v[kRowsPerThread][kLaneRow], xs[kRowsPerThread][kLaneRow];
#pragma unroll
    for (int k = 0; k < kRowsPerThread; ++k)
#pragma unroll
      for (int j = 0; j < kLaneRow; ++j) {
        const bool ok = length[k] <= kLaneRow && j < length[k];
        c[k][j] = ok ? col[begin[k] + j] : 0;
        v[k][j] = ok ? val[begin[k] + j] : 0.0f;
      }
#pragma unroll
    for (int k = 0; k < kRowsPerThread; ++k)
#pragma unroll
      for (int j = 0; j < kLaneRow; ++j)
        xs[k][j] = (length[k] <= kLaneRow && j < length[k]) ? x[clamp_col(c[k][j], cols)] : 0.0f;
#pragma unroll
    for (int k = 0; k < kRowsPerThread; ++k) {
      // hipcc would otherwise fuse each product and add into one FMA, which rounds once.
#pragma clang fp contract(off)
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < kLaneRow; ++j)
        if (j < length[k]) acc = acc + v[k][j] * xs[k][j];
      if (length[k] >= 0 && length[k] <= kLaneRow) y[base + threadIdx.x + 256 * k] = acc;
    }
  }
  // Lists: rank of each medium / large row within the block, in row order (k, then thread).
  int first[2];
  {
    __shared__ int s_pre[2][4];
    int mid_super, big_super;
    superblock_prefix(plan, block / kSuperBlocks, mid_super, big_super, s_pre);
    block_prefix(plan, block, mid_super, big_super, first[0], first[1]);
  }
  // The last block's workgroup writes the list lengths that the piece kernels read.
  if (block == plan.blocks - 1 && threadIdx.x < 2)
    plan.counters[threadIdx.x] = first[threadIdx.x] + plan.block_counts[2 * block + threadIdx.x];
#pragma unroll
  for (int k = 0; k < kRowsPerThread; ++k) {
    const bool is_mid = length[k] >= kGroupRow && length[k] < plan.big;
    const bool is_big = length[k] >= plan.big;
    const uint64_t m_mid = __ballot(is_mid), m_big = __ballot(is_big);
    if (lane == 0) {
      s_wave[0][wave] = __builtin_popcountll(m_mid);
      s_wave[1][wave] = __builtin_popcountll(m_big);
    }
    __syncthreads();
    int before[2] = {first[0], first[1]};
    for (int w = 0; w < wave; ++w) {
      before[0] += s_wave[0][w];
      before[1] += s_wave[1][w];
    }
    const uint64_t below = (1ull << lane) - 1;
    const int32_t r = static_cast<int32_t>(base + threadIdx.x + 256 * k);
    if (is_mid) {
      const int at = before[0] + __builtin_popcountll(m_mid & below);
      if (at < plan.cap_mid) plan.mid_rows[at] = r;
    }
    if (is_big) {
      const int at = before[1] + __builtin_popcountll(m_big & below);
      if (at < plan.cap_big) plan.big_rows[at] = r;
    }
    first[0] += s_wave[0][0] + s_wave[0][1] + s_wave[0][2] + s_wave[0][3];
    first[1] += s_wave[1][0] + s_wave[1][1] + s_wave[1][2] + s_wave[1][3];
    __syncthreads();
  }
  // Rows of 5..127 nonzeros: group g (16 lanes) takes the g-th pending row of the wave.
  const int g = lane >> 4, l16 = lane & 15;
#pragma unroll
  for (int k = 0; k < kRowsPerThread; ++k) {
    uint64_t pending = __ballot(length[k] > kLaneRow && length[k] < kGroupRow);
    while (pending != 0) {   // wave-uniform
      uint64_t m = pending;
      for (int q = 0; q < g; ++q) m &= m - 1;   // drop the g lowest pending rows
      const bool has = m != 0;
      const int from = has ? __builtin_ctzll(m) : lane;
      const int32_t gb = __shfl(begin[k], from), ge = gb + __shfl(length[k], from);
      float acc = 0.0f;
      if (has) {   // at most 8 nonzeros per lane, all loads issued together
        constexpr int kPer = kGroupRow / kGroup;
        int32_t c[kPer];
        float v[kPer];
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
          const int32_t p = gb + l16 + kGroup * q;
          c[q] = p < ge ? col[p] : 0;
          v[q] = p < ge ? val[p] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < kPer; ++q)
          if (gb + l16 + kGroup * q < ge) acc = fmaf(v[q], x[clamp_col(c[q], cols)], acc);
      }
      acc = group16_sum(acc);
      if (has && l16 == 0) y[base + from + (threadIdx.x & ~63) + 256 * k] = acc;
      for (int q = 0; q < 4 && pending != 0; ++q) pending &= pending - 1;   // four rows consumed
    }
  }
}

// Cuts of one row by a group of G lanes (gl: lane in the group, gbase: its first lane). Cut k
// estimates the lower bound of column k * spacing among the row's columns (cut 0 is the row start;
// a threshold at or past `cols` gives the row end) by interpolation search: at most kSearchSteps
// probes, each placed where a uniform spread of the columns between the known bracket values
// would put the threshold. That converges in a few steps on sorted columns. A prefix maximum over
// the group then makes the cuts non-decreasing, so the pieces partition the row for any estimate
// and any column order (an entry outside its window or slice only reads x from another place).
// `rounds` (cuts per lane, rounded up) must be the same for every lane of the wave.
template <int G>
__device__ __forceinline__ void cut_row(const int32_t *__restrict__ col, int32_t begin, int32_t end, int n_cuts,
                                        int rounds, int64_t spacing, int32_t cols, int gl, int gbase,
                                        int32_t *__restrict__ out) {
  int32_t carry = begin;   // running maximum of the cuts of earlier rounds
  for (int u0 = 0; u0 < rounds; u0 += 4) {
    // Thresholds at or past `cols` give the row end, so they are kept clamped to cols (32 bits);
    // the interpolation product needs 64.
    int32_t lo[4], hi[4], thr[4], vlo[4], vhi[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k = gl + G * (u0 + u);
      const int64_t t = static_cast<int64_t>(k) * spacing;
      thr[u] = static_cast<int32_t>(t < cols ? t : cols);
      lo[u] = begin;
      hi[u] = end;
      vlo[u] = -1;
      vhi[u] = cols;
      if (k == 0 || t >= cols) lo[u] = hi[u] = k == 0 ? begin : end;
    }
    for (int step = 0; step < kSearchSteps; ++step) {
      int32_t at[4], cv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t span = hi[u] - lo[u] + 1, rise = static_cast<int64_t>(vhi[u]) - vlo[u];
        int64_t guess = lo[u] - 1 + ((static_cast<int64_t>(thr[u]) - vlo[u]) * span + rise / 2) / (rise > 0 ? rise : 1);
        guess = guess < lo[u] ? lo[u] : (guess > hi[u] - 1 ? hi[u] - 1 : guess);
        at[u] = static_cast<int32_t>(guess);
        cv[u] = lo[u] < hi[u] ? col[at[u]] : 0;
      }
      bool open = false;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (lo[u] < hi[u]) {
          if (cv[u] < thr[u]) {
            lo[u] = at[u] + 1;
            vlo[u] = cv[u];
          } else {
            hi[u] = at[u];
            vhi[u] = cv[u];
          }
        }
        open |= lo[u] < hi[u];
      }
      if (!open) break;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      // Prefix maximum in cut order: lanes gl within this round, after the earlier rounds.
      int32_t cut = lo[u] > carry ? lo[u] : carry;
#pragma unroll
      for (int d = 1; d < G; d <<= 1) {
        const int32_t up = __shfl(cut, gbase + (gl >= d ? gl - d : gl), 64);
        cut = up > cut ? up : cut;
      }
      const int k = gl + G * (u0 + u);
      if (k < n_cuts) out[k] = cut;
      carry = __shfl(cut, gbase + G - 1, 64);
    }
  }
}

// Cuts of the medium and large rows of one 1024-row block, by one wave: the block's rows are
// classified again (as spmv_count did) and ranked in row order, which gives each its list position
// from the block's list offset (block_prefix), the position spmv_rows writes the row id at. Medium
// rows go eight at a time, one 8-lane group per row (9 cuts: the starts of windows 0..8); large
// rows one at a time, the whole wave (slices + 1 cuts). `list` is the wave's LDS scratch for the block's rows.
constexpr int kMidGroup = 8;
__device__ __forceinline__ void cut_block(const int32_t *__restrict__ off, const int32_t *__restrict__ col,
                                          int32_t rows, int32_t cols, int64_t nnz, const Plan &plan, int block,
                                          int lane, int32_t *list, int first_mid, int first_big) {
  const int64_t base = static_cast<int64_t>(block) * kBlockRows;
  // Medium rows at list[0 ..), large rows at list[kBlockRows - 1] downwards, in row order. The
  // offsets are read 256 rows (4 per lane) at a time, all loads of a batch issued together (rows
  // past the end read the last row's).
  constexpr int kBatch = 4;
  int n_mid = 0, n_big = 0;
  for (int k0 = 0; k0 < kBlockRows / 64; k0 += kBatch) {
    int32_t ob[kBatch], oe[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int64_t r = min(base + 64 * (k0 + k) + lane, static_cast<int64_t>(rows) - 1);
      ob[k] = off[r];
      oe[k] = off[r + 1];
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int64_t cb = ob[k] < 0 ? 0 : (ob[k] > nnz ? nnz : static_cast<int64_t>(ob[k]));   // row_span's clamps
      const int64_t ce = oe[k] < cb ? cb : (oe[k] > nnz ? nnz : static_cast<int64_t>(oe[k]));
      const int64_t len = base + 64 * (k0 + k) + lane < rows ? ce - cb : 0;
      const bool is_mid = len >= kGroupRow && len < plan.big, is_big = len >= plan.big;
      const uint64_t m_mid = __ballot(is_mid), m_big = __ballot(is_big);
      const uint64_t below = (1ull << lane) - 1;
      if (is_mid) list[n_mid + __builtin_popcountll(m_mid & below)] = 64 * (k0 + k) + lane;
      if (is_big) list[kBlockRows - 1 - n_big - __builtin_popcountll(m_big & below)] = 64 * (k0 + k) + lane;
      n_mid += __builtin_popcountll(m_mid);
      n_big += __builtin_popcountll(m_big);
    }
  }
  __builtin_amdgcn_wave_barrier();

  const int64_t window = (static_cast<int64_t>(cols) + kWindows - 1) / kWindows;
  const int g = lane / kMidGroup;
  for (int q = 0; q < n_mid; q += 64 / kMidGroup) {   // wave-uniform
    const int i = q + g;
    const int at = first_mid + i;
    const bool ok = i < n_mid && at < plan.cap_mid;
    int32_t b = 0, e = 0;
    if (ok) row_span(off, base + list[i], nnz, b, e);
    cut_row<kMidGroup>(col, b, e, ok ? kWindows + 1 : 0, (kWindows + 1 + kMidGroup - 1) / kMidGroup, window, cols,
                       lane % kMidGroup, g * kMidGroup, plan.mid_cuts + static_cast<int64_t>(ok ? at : 0) * (kWindows + 1));
  }
  const int big_cuts = plan.slices + 1;
  for (int i = 0; i < n_big; ++i) {   // wave-uniform
    const int at = first_big + i;
    if (at >= plan.cap_big) break;
    int32_t b, e;
    row_span(off, base + list[kBlockRows - 1 - i], nnz, b, e);
    cut_row<64>(col, b, e, big_cuts, (big_cuts + 63) / 64, kSliceCols, cols, lane, 0,
                plan.big_cuts + static_cast<int64_t>(at) * big_cuts);
  }
}

// Short rows, row lists and cuts in one launch. The first cut_groups workgroups compute the cuts
// (one wave per 1024-row block), the rest fold the short rows and write the lists (one workgroup
// per block). The cuts are chains of dependent probes, the short rows are bound by the fabric's
// random line fetches; in one grid the cut chains run beside the short rows instead of after them
// (config 5: 165 us for both, against 140 + 52 us as two launches).
__global__ __launch_bounds__(256) void spmv_rows(const int32_t *__restrict__ off, const int32_t *__restrict__ col,
                                                    const float *__restrict__ val, const float *__restrict__ x,
                                                    float *__restrict__ y, int32_t rows, int32_t cols, int64_t nnz,
                                                    Plan plan, int cut_groups) {
  __shared__ int32_t s_list[4][kBlockRows];
  if (static_cast<int>(blockIdx.x) < cut_groups) {   // workgroup-uniform
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int block = static_cast<int>(blockIdx.x) * 4 + wave;   // the four blocks of one superblock
    __shared__ int s_pre[2][4];
    int mid_super, big_super, first_mid, first_big;
    superblock_prefix(plan, static_cast<int>(blockIdx.x), mid_super, big_super, s_pre);
    if (block < plan.blocks) {   // wave-uniform; the last group may hold fewer than four blocks
      block_prefix(plan, block, mid_super, big_super, first_mid, first_big);
      cut_block(off, col, rows, cols, nnz, plan, block, lane, s_list[wave], first_mid, first_big);
    }
    return;
  }
  rows_block(off, col, val, x, y, rows, cols, nnz, plan, static_cast<int>(blockIdx.x) - cut_groups);
}

// Pieces of listed rows. Wave w of a workgroup takes the pieces of list rows i = k + K t for
// t = w, w + 16, ..., one piece at a time: lanes stride the piece 64 nonzeros at a time, a block of
// strides loaded together (coalesced), and the piece's sum is one wave reduction in a fixed order.
constexpr int kSliceThreads = 1024;
constexpr int kSliceWaves = kSliceThreads / 64;

// Medium rows, one column window per part: workgroup h takes window h % 8 and runs on XCD h % 8,
// whose L2 holds that window of x. While a piece is summed, the next piece's cuts (scalar loads)
// and first block are in flight. The pieces are short (77 nonzeros on average at config 5), so
// lanes past a piece's end load nothing: issuing their loads anyway, so that the wait counters
// could overlap two pieces ahead, measured slower (101.6 / 98.7 against 94.9 us with blocks of 4 /
// 2 strides); the window gathers are bound by the loads issued, not by their latency.
constexpr int kWindowUnroll = 4;
__global__ __launch_bounds__(kSliceThreads) void spmv_windows(const int32_t *__restrict__ col,
                                                             const float *__restrict__ val,
                                                             const float *__restrict__ x, int32_t cols,
                                                             const int32_t *__restrict__ cuts, int cut_stride,
                                                             float *__restrict__ parts, int part_stride,
                                                             const int32_t *__restrict__ count, int capacity) {
  constexpr int kU = kWindowUnroll;
  const int tid = threadIdx.x, lane = tid & 63;
  // Wave-uniform in a scalar register, so the cuts below are scalar loads (counted by lgkmcnt).
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int K = static_cast<int>(gridDim.x) / part_stride;
  const int part = static_cast<int>(blockIdx.x % part_stride);
  const int k = static_cast<int>(blockIdx.x / part_stride);
  const int n_rows = min(*count, capacity);
  if (n_rows <= k) return;   // workgroup-uniform
  const int n_tile = (n_rows - k + K - 1) / K;
  auto cut_at = [&](int t, int side) {
    return __builtin_amdgcn_readfirstlane(cuts[(k + static_cast<int64_t>(K) * t) * cut_stride + part + side]);
  };
  auto load_block = [&](int32_t p0, int32_t e, int32_t (&cu)[kU], float (&vu)[kU]) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int32_t p = p0 + 64 * u + lane;
      cu[u] = p < e ? __builtin_nontemporal_load(col + p) : 0;
      vu[u] = p < e ? __builtin_nontemporal_load(val + p) : 0.0f;
    }
  };
  // Masked lanes leave the sum as it was (a select after the FMA): multiplying their stand-in x by
  // zero would turn an inf or NaN elsewhere in x into a NaN here.
  auto add_block = [&](int32_t p0, int32_t e, const int32_t (&cu)[kU], const float (&vu)[kU], float &acc) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const bool ok = p0 + 64 * u + lane < e;
      const float sum = fmaf(vu[u], x[clamp_col(ok ? cu[u] : 0, cols)], acc);
      acc = ok ? sum : acc;
    }
  };
  // Two register sets alternate: while piece t is summed from one, the next piece's first block
  // loads into the other, and the cuts of the piece after next load (scalar). Unrolled by two so
  // that no set is copied into the other, which would wait for the loads in flight.
  int t = wave;
  if (t >= n_tile) return;
  int32_t b0 = cut_at(t, 0), e0 = cut_at(t, 1);
  int32_t b1 = 0, e1 = 0;
  if (t + kSliceWaves < n_tile) {
    b1 = cut_at(t + kSliceWaves, 0);
    e1 = cut_at(t + kSliceWaves, 1);
  }
  int32_t cu0[kU], cu1[kU];
  float vu0[kU], vu1[kU];
  load_block(b0, e0, cu0, vu0);
  auto piece = [&](int32_t b, int32_t e, const int32_t (&cu)[kU], const float (&vu)[kU], int32_t nb, int32_t ne,
                   int32_t (&ncu)[kU], float (&nvu)[kU], int32_t &fb, int32_t &fe) {
    const bool more = t + kSliceWaves < n_tile;   // wave-uniform
    if (more) load_block(nb, ne, ncu, nvu);
    if (t + 2 * kSliceWaves < n_tile) {
      fb = cut_at(t + 2 * kSliceWaves, 0);
      fe = cut_at(t + 2 * kSliceWaves, 1);
    }
    float acc = 0.0f;
    add_block(b, e, cu, vu, acc);
    for (int32_t p0 = b + 64 * kU; p0 < e; p0 += 64 * kU) {   // wave-uniform: rest of the piece
      int32_t cr[kU];
      float vr[kU];
      load_block(p0, e, cr, vr);
      add_block(p0, e, cr, vr, acc);
    }
    const float sum = wave_sum(acc);
    if (lane == 0) parts[(k + static_cast<int64_t>(K) * t) * part_stride + part] = sum;
    return more;
  };
  while (true) {   // wave-uniform
    if (!piece(b0, e0, cu0, vu0, b1, e1, cu1, vu1, b0, e0)) break;
    t += kSliceWaves;
    if (!piece(b1, e1, cu1, vu1, b0, e0, cu0, vu0, b1, e1)) break;
    t += kSliceWaves;
  }
}

// Large rows, one slice of kSliceCols columns per part (workgroups part * K + k): the slice of x is
// staged in LDS and the pieces gather from it. An entry outside the slice (possible with an inexact
// cut) reads x from global memory.
//
// Three pieces are in flight per wave: while piece t is summed, the first blocks of pieces t + 16
// and t + 32 are loading. Vector loads and stores complete out of order with each other, so a
// store among the loads would make the compiler wait for all of them; the piece sums therefore
// collect in a register (lane j: piece 64 g + j) and are stored 64 at a time. Every load of a block
// is unconditional (lanes past a piece's end re-read its last entry, one address for all of them),
// so the wait for a block counts exactly the loads issued after it. The cuts come 64 pieces at a
// time, one vector load per side, read with readlane: no scalar loads in the loop, whose
// out-of-order returns would make every wait for the LDS gathers a full lgkmcnt(0).
// Against the two-deep loop with per-piece stores: 100.2 against 110.2 us at config 5, bit-identical.
constexpr int kSliceUnroll = 4;   // strides per block
__global__ __launch_bounds__(kSliceThreads) void spmv_slices(const int32_t *__restrict__ col,
                                                            const float *__restrict__ val,
                                                            const float *__restrict__ x, int32_t cols,
                                                            const int32_t *__restrict__ cuts, int cut_stride,
                                                            float *__restrict__ parts, int part_stride,
                                                            const int32_t *__restrict__ count, int capacity) {
  constexpr int kU = kSliceUnroll;
  __shared__ float sx[kSliceCols];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int K = static_cast<int>(gridDim.x) / part_stride;
  const int part = static_cast<int>(blockIdx.x) / K;
  const int k = static_cast<int>(blockIdx.x) % K;
  const int n_rows = min(*count, capacity);
  if (n_rows <= k) return;   // workgroup-uniform
  const int64_t c0 = static_cast<int64_t>(part) * kSliceCols;
  const int width = static_cast<int>(min(static_cast<int64_t>(kSliceCols), cols - c0));
  {
    constexpr int kPer = kSliceCols / kSliceThreads;
    float staged[kPer];
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int c = tid + kSliceThreads * q;
      staged[q] = c < width ? x[c0 + c] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < kPer; ++q) sx[tid + kSliceThreads * q] = staged[q];
  }
  __syncthreads();
  const int n_tile = (n_rows - k + K - 1) / K;
  if (wave >= n_tile) return;   // wave-uniform

  // This wave's pieces i = 0 .. n_pieces - 1 are t = wave + 16 i. Their cuts come 64 at a time
  // (lane j holds those of piece 64 g + j); a piece past the wave's last is empty, at the last
  // piece's end (a valid position, so its loads stay in bounds).
  const int n_pieces = (n_tile - wave + kSliceWaves - 1) / kSliceWaves;
  int32_t lane_b = 0, lane_e = 0, group = -1;
  auto cuts_of = [&](int i, int32_t &b, int32_t &e) {
    if ((i >> 6) != group) {   // wave-uniform; once per 64 pieces
      group = i >> 6;
      const int t = wave + kSliceWaves * (64 * group + lane);
      const int64_t at = (k + static_cast<int64_t>(K) * min(t, n_tile - 1)) * cut_stride + part;
      const int32_t lb = cuts[at], le = cuts[at + 1];
      lane_b = t < n_tile ? lb : le;
      lane_e = le;
    }
    b = __builtin_amdgcn_readlane(lane_b, i & 63);
    e = __builtin_amdgcn_readlane(lane_e, i & 63);
  };
  float sums = 0.0f;
  auto store_sums = [&](int g) {   // the pieces 64 g + lane that exist
    const int t = wave + kSliceWaves * (64 * g + lane);
    if (t < n_tile) parts[(k + static_cast<int64_t>(K) * t) * part_stride + part] = sums;
  };
  // The block of [p0, e): every lane loads; lanes past the end re-read entry e - 1 (entry 0 of an
  // empty piece at 0). add_block masks them where it uses them.
  auto load_block = [&](int32_t p0, int32_t e, int32_t (&cu)[kU], float (&vu)[kU]) {
    const int32_t last = e > 0 ? e - 1 : 0;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int32_t p = p0 + 64 * u + lane;
      const int32_t at = p < e ? p : last;
      cu[u] = __builtin_nontemporal_load(col + at);
      vu[u] = __builtin_nontemporal_load(val + at);
    }
  };
  // Products of the block of [p0, e) into acc; those of entries outside the slice go to `stray`,
  // read from global x. Masked lanes leave the sums as they were (a select after the FMA):
  // multiplying their stand-in x by zero would turn an inf or NaN elsewhere in x into a NaN here.
  // The LDS and global reads stay separate: written as one select of an LDS and a global load,
  // hipcc merged them into a generic flat load, which sent every gather through the vector memory
  // path.
  auto add_block = [&](int32_t p0, int32_t e, const int32_t (&cu)[kU], const float (&vu)[kU], float &acc,
                       float &stray) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const bool ok = p0 + 64 * u + lane < e;
      const int32_t local = cu[u] - static_cast<int32_t>(c0);
      const bool in = !ok || static_cast<uint32_t>(local) < static_cast<uint32_t>(width);
      const float xl = sx[ok && in ? local : 0];
      const float sum = fmaf(vu[u], xl, acc);
      acc = ok && in ? sum : acc;   // an entry outside the slice adds into stray only
      if (__builtin_expect(__any(!in), 0)) {   // wave-uniform
        if (!in) stray = fmaf(vu[u], __builtin_nontemporal_load(x + clamp_col(cu[u], cols)), stray);
      }
    }
  };
  // Piece i from set (b, e, cu, vu); the block of piece i + 2 loads into set (fb, fe, fcu, fvu).
  auto piece = [&](int i, int32_t b, int32_t e, const int32_t (&cu)[kU], const float (&vu)[kU], int32_t &fb,
                   int32_t &fe, int32_t (&fcu)[kU], float (&fvu)[kU]) {
    if ((i & 63) == 0 && i > 0) {   // wave-uniform; once per 64 pieces
      store_sums((i >> 6) - 1);
      sums = 0.0f;
      __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8));   // vmcnt(0): the store out of the way
    }
    cuts_of(i + 2, fb, fe);
    load_block(fb, fe, fcu, fvu);
    // Nothing that waits for this piece's data moves above the loads of piece i + 2.
    __builtin_amdgcn_sched_barrier(0);
    float acc = 0.0f, stray = 0.0f;
    add_block(b, e, cu, vu, acc, stray);
    for (int32_t p0 = b + 64 * kU; p0 < e; p0 += 64 * kU) {   // wave-uniform: rest of the piece
      int32_t cr[kU];
      float vr[kU];
      load_block(p0, e, cr, vr);
      add_block(p0, e, cr, vr, acc, stray);
    }
    const float sum = wave_sum(acc + stray);
    sums = lane == (i & 63) ? sum : sums;
  };
  int32_t b0, e0, b1, e1, b2 = 0, e2 = 0;
  int32_t cu0[kU], cu1[kU], cu2[kU];
  float vu0[kU], vu1[kU], vu2[kU];
  // Issued in this order (the scheduler may not interleave them), so that the loop's first wait
  // for piece 0's block leaves piece 1's in flight, as every later wait does.
  cuts_of(0, b0, e0);
  load_block(b0, e0, cu0, vu0);
  __builtin_amdgcn_sched_barrier(0);
  cuts_of(1, b1, e1);
  load_block(b1, e1, cu1, vu1);
  __builtin_amdgcn_sched_barrier(0);
  // Three pieces per iteration (the last ones empty past the wave's end), so that the sets rotate
  // without being copied (a copy waits for its loads) and no exit sits between them.
  int i = 0;
  for (; i < n_pieces; i += 3) {   // wave-uniform
    piece(i, b0, e0, cu0, vu0, b2, e2, cu2, vu2);
    piece(i + 1, b1, e1, cu1, vu1, b0, e0, cu0, vu0);
    piece(i + 2, b2, e2, cu2, vu2, b1, e1, cu1, vu1);
  }
  store_sums((i - 1) >> 6);
}

// y of every medium row (thread per row: windows 0..7 in order) and large row (wave per row: lane
// l sums slices l, l + 64, ... in order, then a fixed reduction tree). The first mid_groups
// workgroups take the medium rows, the rest the large rows, as many as the list capacity needs up
// to 128 and 512 (beyond that they loop), so that a wave sums about one large row at config 5: with
// 64 workgroups for the large rows each wave summed eight (9.8 us).
__global__ __launch_bounds__(256) void spmv_combine(float *__restrict__ y, Plan plan, int mid_groups) {
  const int64_t n_mid = min(plan.counters[0], plan.cap_mid), n_big = min(plan.counters[1], plan.cap_big);
  const int half = mid_groups;
  if (static_cast<int>(blockIdx.x) < half) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n_mid;
         i += static_cast<int64_t>(half) * 256) {
      const float4 a = *reinterpret_cast<const float4 *>(plan.mid_parts + i * kWindows);
      const float4 b = *reinterpret_cast<const float4 *>(plan.mid_parts + i * kWindows + 4);
      y[plan.mid_rows[i]] = ((((((a.x + a.y) + a.z) + a.w) + b.x) + b.y) + b.z) + b.w;
    }
    return;
  }
  const int lane = threadIdx.x & 63;
  const int S = plan.slices;
  const int64_t big_groups = static_cast<int64_t>(gridDim.x) - half;
  for (int64_t i = static_cast<int64_t>(blockIdx.x - half) * 4 + (threadIdx.x >> 6); i < n_big;
       i += big_groups * 4) {   // uniform within a wave
    float acc = 0.0f;
    for (int s = lane; s < S; s += 64) acc += plan.big_parts[i * S + s];
    const float sum = wave_sum(acc);
    if (lane == 0) y[plan.big_rows[i]] = sum;
  }
}

}  // namespace

int spmv_resources(int64_t rows, int64_t nnz, IntentHipKernelResources *out) {
  (void)rows;
  (void)nnz;
  return describe_kernel(reinterpret_cast<const void *>(&spmv_slices), "spmv_slices", kSliceThreads, out);
}

}  // namespace intent_hip

using namespace intent_hip;

extern "C" int intent_hip_csr_spmv_workspace_bytes(int64_t rows, int64_t nnz, size_t *bytes) {
  if (bytes == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null output");
  if (rows < 0 || nnz < 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  *bytes = workspace_bytes(rows, nnz);
  return INTENT_HIP_OK;
}

extern "C" int intent_hip_csr_spmv_f32(const int32_t *row_offsets, const int32_t *column_indices,
                                       const float *values, const float *x, float *y, int64_t rows,
                                       int64_t cols, int64_t nnz, void *workspace, size_t workspace_size,
                                       void *stream) {
  if (rows < 0 || cols < 0 || nnz < 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (rows + nnz > INT32_MAX || cols > INT32_MAX)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "rows + nnz and cols must stay below 2^31 (32-bit CSR indices)");
  if (rows == 0) return INTENT_HIP_OK;
  if (nnz > 0 && cols == 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "nonzeros in a matrix with no columns");
  if (row_offsets == nullptr || y == nullptr || (nnz > 0 && (column_indices == nullptr || values == nullptr || x == nullptr)))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null tensor pointer");
  if (workspace == nullptr || workspace_size < workspace_bytes(rows, nnz) || !aligned(workspace, 256))
    return fail(INTENT_HIP_ERR_WORKSPACE, "SpMV needs %zu workspace bytes (256-byte aligned), got %zu",
                workspace_bytes(rows, nnz), workspace_size);
  const Plan plan = carve(workspace, rows, cols, nnz);
  const hipStream_t s = as_stream(stream);
  const int32_t r32 = static_cast<int32_t>(rows), c32 = static_cast<int32_t>(cols > 0 ? cols : 1);
  spmv_count<<<dim3(static_cast<unsigned>(plan.supers)), dim3(256 * kSuperBlocks), 0, s>>>(row_offsets, r32, nnz,
                                                                                          plan);
  // No row can be medium or large: no cut workgroups.
  const int cut_groups = plan.cap_mid == 0 && plan.cap_big == 0 ? 0 : (plan.blocks + 3) / 4;
  spmv_rows<<<dim3(static_cast<unsigned>(plan.blocks + cut_groups)), dim3(256), 0, s>>>(
      row_offsets, column_indices, values, x, y, r32, c32, nnz, plan, cut_groups);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("spmv_rows");
  if (plan.cap_mid == 0 && plan.cap_big == 0) return INTENT_HIP_OK;   // no row can be medium or large
  if (plan.cap_mid > 0)
    spmv_windows<<<dim3(kWindows * kWindowTiles), dim3(kSliceThreads), 0, s>>>(
        column_indices, values, x, c32, plan.mid_cuts, kWindows + 1, plan.mid_parts, kWindows, plan.counters + 0,
        plan.cap_mid);
  if (plan.cap_big > 0) {
    const int K = static_cast<int>((kSliceTiles + plan.slices - 1) / plan.slices);
    spmv_slices<<<dim3(static_cast<unsigned>(plan.slices) * static_cast<unsigned>(K)), dim3(kSliceThreads), 0,
                  s>>>(column_indices, values, x, c32, plan.big_cuts, plan.slices + 1, plan.big_parts,
                       plan.slices, plan.counters + 1, plan.cap_big);
  }
  const int mid_groups = static_cast<int>(std::min<int64_t>((plan.cap_mid + 255) / 256, 128)) + 1;
  const int big_groups = static_cast<int>(std::min<int64_t>((plan.cap_big + 3) / 4, 512)) + 1;
  spmv_combine<<<dim3(static_cast<unsigned>(mid_groups + big_groups)), dim3(256), 0, s>>>(y, plan, mid_groups);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("spmv_combine");
  return INTENT_HIP_OK;
}

// ---------------------------------------------------------------- no-allocation entry point
// For callers that cannot allocate (code under graph capture, serving loops, harnesses that forbid
// hipMalloc): the workspace is a static device array, `scratch`, of INTENT_HIP_STATIC_SCRATCH_BYTES.
// Each GPU the library runs on holds its own copy until the process ends; its address on the
// current device is looked up once (hipGetSymbolAddress) and kept per device. Every call on a GPU
// shares that GPU's array, so calls that overlap on one GPU race. Nothing in it has to start at
// zero: every kernel writes what a later kernel of the same call reads.
namespace intent_hip {

static __device__ __align__(256) char scratch[INTENT_HIP_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void *g_scratch_address[kMaxDevices] = {};

// The current device's address of `scratch` (the host-side name of the array is not a device
// address and is never passed to a kernel).
int scratch_address(void **out) {
  int device = -1;
  hipError_t status = hipGetDevice(&device);
  if (status != hipSuccess) return fail(INTENT_HIP_ERR_DEVICE, "hipGetDevice: %s", hipGetErrorString(status));
  if (device < 0 || device >= kMaxDevices)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "device %d is beyond the %d devices the static scratch tracks", device,
                kMaxDevices);
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (g_scratch_address[device] == nullptr) {
    void *address = nullptr;
    status = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (status != hipSuccess || address == nullptr)
      return fail(INTENT_HIP_ERR_DEVICE, "hipGetSymbolAddress(scratch) on device %d: %s", device,
                  hipGetErrorString(status));
    g_scratch_address[device] = address;
  }
  *out = g_scratch_address[device];
  return INTENT_HIP_OK;
}

}  // namespace
}  // namespace intent_hip

extern "C" int intent_hip_csr_spmv_f32_static(const int32_t *row_offsets, const int32_t *column_indices,
                                              const float *values, const float *x, float *y, int64_t rows,
                                              int64_t cols, int64_t nnz, void *stream) {
  if (rows < 0 || cols < 0 || nnz < 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (rows + nnz > INT32_MAX) return fail(INTENT_HIP_ERR_UNSUPPORTED, "rows + nnz must stay below 2^31");
  const size_t need = workspace_bytes(rows, nnz);
  if (need > INTENT_HIP_STATIC_SCRATCH_BYTES)
    return fail(INTENT_HIP_ERR_WORKSPACE,
                "SpMV of %lld rows and %lld nonzeros needs %zu workspace bytes, beyond the %zu-byte static scratch; "
                "use intent_hip_csr_spmv_f32 with a caller-owned workspace",
                static_cast<long long>(rows), static_cast<long long>(nnz), need,
                static_cast<size_t>(INTENT_HIP_STATIC_SCRATCH_BYTES));
  if (rows == 0) return INTENT_HIP_OK;
  void *address = nullptr;
  if (const int rc = scratch_address(&address)) return rc;
  return intent_hip_csr_spmv_f32(row_offsets, column_indices, values, x, y, rows, cols, nnz, address,
                                 INTENT_HIP_STATIC_SCRATCH_BYTES, stream);
}
