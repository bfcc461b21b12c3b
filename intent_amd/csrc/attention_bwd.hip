// Attention backward (f16 storage, f32 arithmetic) for gfx950: delta, dQ and dK/dV.
//
// Semantics (python/intent/examples/kernels/backward/attention.py):
//   attention_backward_delta (:17-34): delta[b,h,q] = sum_d o * do (f32);
//   attention_backward_dq (:171-211) with summarize_query_gradients (:140-163);
//   attention_backward_dkdv (:87-137) with summarize_key_value_gradients (:47-79):
//     s = q . k (f32); p = exp2(s * scale * log2 e - lse * log2 e) (v_exp_f32, approximate);
//     causal validity q >= k; excluded pairs have p = 0 and dS = 0;
//     dp = do . v; dS = p * (dp - delta);
//     dV = sum_q f16(p) do; dK = scale * sum_q f16(dS) q; dQ = scale * sum_k f16(dS) k.
//   Query head h uses key/value head h / head_group; dK/dV of a key head sum over the
//   head_group query heads that share it. The summed axes are reassociated (region folds
//   combined by addition).
//
// Design (head dimension D = 64 or 128, v_mfma_f32_32x32x16_f16 throughout):
//   * dQ: a workgroup owns 32 queries per wave of one (batch, query head); 64-key tiles of K and
//     V stream through LDS (global_load_lds_dwordx4, kStages stages). Per 32-key half:
//     S^T = K Q^T and dP^T = V dO^T with the wave's Q and dO fragments in registers (lane l
//     holds the scores of query l % 32), dS^T rounded to f16 in registers, then
//     dQ^T += K^T dS^T over that half's keys, with K^T read by ds_read_b64_tr_b16 from K's
//     natural [key][d] layout.
//   * dK/dV: a workgroup owns 32 keys per wave of one (batch, key head); 64-query tiles of Q and
//     dO (of every query head in the group) stream through LDS, with their lse and delta. Per
//     32-query half: S = Q K^T and dP = dO V^T with the wave's K and V fragments in registers
//     (lane l holds key l % 32), P and dS rounded to f16 in registers, then dV^T += dO^T P and
//     dK^T += Q^T dS over that half's queries, with transposing LDS reads of Q and dO.
//   * Wide grids (at least kWideRows rows) run 8 waves per workgroup, two per SIMD: while one
//     wave issues MFMAs (at raised priority, s_setprio 1) the other's exp and LDS work fills the
//     gaps, and each streamed tile serves 256 rows. dK/dV then runs as two kernels, dK (S, dP,
//     dK) and dV (S, dV), each within the 256 registers a lane has at two waves per SIMD; the
//     combined kernel needs about 400. Narrow grids run 4 waves per workgroup (more workgroups),
//     dK and dV together.
//   * Rows past the end of a tensor read its last row (finite data that the mask excludes).
//     Causal work is skipped per wave where no pair of a tile is valid.
#include "common.hpp"

namespace intent_hip {
namespace {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int kThreads = 256;   // delta, the split reduction, and the 4-wave dQ / dK-dV kernels
constexpr int kRows = 128;      // queries (dQ) or keys (dK/dV) per 4-wave workgroup
constexpr int kTile = 64;       // keys (dQ) or queries (dK/dV) per streamed tile
// Calls with at least this many rows (batch x heads x sequence, query heads for dQ, key heads for
// dK/dV) use the 8-wave, 256-row workgroups: enough rows for 256 of them.
constexpr int64_t kWideRows = 256 * 256;

// The part of dK/dV a kernel computes.
enum DkdvPart { kBoth = 0, kOnlyDk = 1, kOnlyDv = 2 };
constexpr float kLog2e = 1.4426950408889634f;

#define INTENT_WAIT_VMCNT0() __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8))

// Streamed tiles go through kStages LDS stages, two tiles per barrier: at each barrier the waves
// hold the current two tiles and the next two are fetched into the stages of the two before, so
// the waves synchronise once per two tiles. Against one barrier per tile with three tiles in
// flight (interleaved, bit-identical): B4 HQ32 HK8 S4096 D128 2.830 -> 2.740 ms, the reference
// example 58.0 -> 57.2 us, B1 HQ16 HK4 S2048 D128 180.5 -> 178.2 us.
constexpr int kStages = 4;

__device__ __forceinline__ f32x16_t mma(f16x8_t a, f16x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint4 select(bool keep, uint4 v) {
  return make_uint4(keep ? v.x : 0u, keep ? v.y : 0u, keep ? v.z : 0u, keep ? v.w : 0u);
}

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, round_to<_Float16>(lo))) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, round_to<_Float16>(hi))) << 16);
}

// Element strides of the backward operands (batch, head, row, col for 4-D; batch, head, row for
// lse and delta).
struct BwdGeometry {
  int64_t q[4], k[4], v[4], dout[4], lse[3], delta[3], out0[4], out1[4];
};

// LDS tile of kTile rows of D f16 (rows of D / 8 16-byte chunks). Chunk c of row r is stored at
// c ^ swz(r); both row reads and transposing reads go through this map, so any swizzle is
// correct. This one is conflict-free for both (64 banks, 256 bytes per bank row):
//   * 16-byte row reads of 16 consecutive rows land on 16 distinct 16-byte slots of a bank row
//     (D = 128: one row per bank row, swz a bijection of r % 16; D = 64: two rows per bank row,
//     swz a bijection of (r / 2) % 8);
//   * transposing reads of 4 consecutive rows (starting at a multiple of 4) over an aligned group
//     of 4 chunks land on 4 disjoint chunk groups.
template <int D>
__device__ __forceinline__ int swz(int row) {
  if constexpr (D == 128) return ((row & 3) << 2) | ((row >> 2) & 3);
  return (((row >> 1) & 1) << 2) | ((row >> 2) & 3);
}

// Row fragment of an MFMA A operand: rows `row` (lane & 31 within a 32-row block), 8
// consecutive columns starting at 16 ks + 8 half.
template <int D>
__device__ __forceinline__ f16x8_t row_frag(const uint4 *tile, int row, int ks, int half) {
  return __builtin_bit_cast(f16x8_t, tile[row * (D / 8) + ((ks * 2 + half) ^ swz<D>(row))]);
}

// Transposed fragment (A operand rows = columns of the tile): this lane receives rows
// 16 sl + 8 r + 4 half + 0..3 of column 32 mt + (its column), for r = 0, 1.
template <int D>
__device__ __forceinline__ f16x8_t tr_frag(const uint16_t *tile, int sl, int mt, int t_row, int t_col) {
  i16x4_t parts[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int row = sl * 16 + 8 * r + t_row;
    const int col = mt * 32 + t_col;
    const int chunk = (col >> 3) ^ swz<D>(row);
    parts[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(tile + row * D + chunk * 8 + (col & 7)));
  }
  return __builtin_bit_cast(f16x8_t, parts);
}

// ---------------------------------------------------------------- excluded pairs
// The reference leaves causally excluded pairs (and rows past the end) out of the gradient
// products even when their operands are non-finite (masked_gradient_product,
// backward/attention.py:37-44). The MFMA path gives an excluded pair a zero weight, which is
// exact for finite operand rows, but 0 * inf or 0 * NaN would reach the gradient. So a tile that
// holds excluded pairs and whose operand rows (K for dQ; Q for dK; dO for dV) hold an inf or NaN
// is left out of the MFMA loop, and after that loop the wave folds it again one pair at a time,
// from global memory, skipping the excluded pairs. The check costs a few LDS reads per edge tile;
// the scalar fold runs only for such inputs. It sits after the loop, not in it: inside the tile
// loop, its code raised the 8-wave D = 128 kernels to 256 VGPRs with spills in the hot path.

// Nonzero when either f16 half of w has an all-ones exponent (inf or NaN): 0x7C00 + 0x0400 sets
// bit 15 of that half, smaller exponents do not, and no carry crosses into the upper half.
__device__ __forceinline__ uint32_t nonfinite_halves(uint32_t w) {
  return ((w & 0x7C007C00u) + 0x04000400u) & 0x80008000u;
}

__device__ __forceinline__ uint32_t nonfinite_chunk(uint4 w) {
  return nonfinite_halves(w.x) | nonfinite_halves(w.y) | nonfinite_halves(w.z) | nonfinite_halves(w.w);
}

// True (for the whole wave) when an element of the 64 rows of an LDS tile is inf or NaN. Lane l
// reads half of rows l % 32 and 32 + l % 32; the lane pair (l, l ^ 32) covers both rows.
template <int D>
__device__ __forceinline__ bool tile_nonfinite(const uint4 *tile, int lane) {
  const int half = lane >> 5;
  uint32_t bad = 0;
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    const int row = st * 32 + (lane & 31);
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) bad |= nonfinite_chunk(tile[row * (D / 8) + ((ks * 2 + half) ^ swz<D>(row))]);
  }
  return __any(bad != 0);
}

// The same test on rows [first, first + 64) of a tensor in global memory (row r at base + r * ld,
// rows past `last` read row `last`, as the tile DMA does).
template <int D>
__device__ __forceinline__ bool rows_nonfinite(const uint16_t *base, int64_t ld, int first, int last, int lane) {
  const int half = lane >> 5;
  uint32_t bad = 0;
#pragma unroll 1
  for (int st = 0; st < 2; ++st) {
    const uint16_t *row = base + static_cast<int64_t>(min(first + st * 32 + (lane & 31), last)) * ld;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) bad |= nonfinite_chunk(*reinterpret_cast<const uint4 *>(row + ks * 16 + half * 8));
  }
  return __any(bad != 0);
}

// Dot product of this lane's half of a row held in registers (D / 16 fragments of 8 f16, columns
// 16 ks + 8 half + 0..7) with the same columns of a row in global memory, completed across the lane
// pair. Packed f16 dot products (v_dot2_f32_f16) take the fragments as they are.
template <int D>
__device__ __forceinline__ float pair_dot(const f16x8_t (&frag)[D / 16], const uint16_t *row, int half) {
  typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
  float sum = 0.0f;
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) {
    const uint4 x = *reinterpret_cast<const uint4 *>(row + ks * 16 + half * 8);
    const uint4 f = __builtin_bit_cast(uint4, frag[ks]);
    sum = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, f.x), __builtin_bit_cast(f16x2_t, x.x), sum, false);
    sum = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, f.y), __builtin_bit_cast(f16x2_t, x.y), sum, false);
    sum = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, f.z), __builtin_bit_cast(f16x2_t, x.z), sum, false);
    sum = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, f.w), __builtin_bit_cast(f16x2_t, x.w), sum, false);
  }
  return sum + __shfl_xor(sum, 32);
}

__device__ __forceinline__ float f16_bits_to_float(uint32_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits & 0xFFFFu)));
}

// acc (MFMA accumulator order: slot 4 gq + j of tile mt is column 32 mt + 8 gq + 4 half + j) +=
// w * the lane's columns of a row in global memory; each product is rounded once into the sum
// (fmaf), as in the MFMA.
template <int D>
__device__ __forceinline__ void add_row(f32x16_t (&acc)[D / 32], float w, const uint16_t *row, int half) {
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const uint2 x = *reinterpret_cast<const uint2 *>(row + mt * 32 + gq * 8 + half * 4);
      acc[mt][4 * gq + 0] = fmaf(w, f16_bits_to_float(x.x), acc[mt][4 * gq + 0]);
      acc[mt][4 * gq + 1] = fmaf(w, f16_bits_to_float(x.x >> 16), acc[mt][4 * gq + 1]);
      acc[mt][4 * gq + 2] = fmaf(w, f16_bits_to_float(x.y), acc[mt][4 * gq + 2]);
      acc[mt][4 * gq + 3] = fmaf(w, f16_bits_to_float(x.y >> 16), acc[mt][4 * gq + 3]);
    }
}

// ---------------------------------------------------------------- delta
// D / 8 lanes per row, 8 elements (one 16-byte load of o and of do) per lane.
template <int D>
__global__ __launch_bounds__(kThreads) void attention_bwd_delta(const uint16_t *__restrict__ O,
                                                                const uint16_t *__restrict__ G,
                                                                float *__restrict__ delta, int heads, int sq,
                                                                int64_t rows, BwdGeometry g) {
  constexpr int kLanes = D / 8;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t row = t / kLanes;
  const int part = static_cast<int>(t % kLanes);
  const bool live = row < rows;
  const int64_t r = live ? row : 0;
  const int64_t b = r / (static_cast<int64_t>(heads) * sq), h = (r / sq) % heads, q = r % sq;
  const uint4 ov = *reinterpret_cast<const uint4 *>(O + b * g.q[0] + h * g.q[1] + q * g.q[2] + part * 8);
  const uint4 gv = *reinterpret_cast<const uint4 *>(G + b * g.dout[0] + h * g.dout[1] + q * g.dout[2] + part * 8);
  const f16x8_t of = __builtin_bit_cast(f16x8_t, ov), gf = __builtin_bit_cast(f16x8_t, gv);
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) sum = fmaf(static_cast<float>(of[i]), static_cast<float>(gf[i]), sum);
#pragma unroll
  for (int off = kLanes / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  if (live && part == 0) delta[b * g.delta[0] + h * g.delta[1] + q * g.delta[2]] = sum;
}

// ---------------------------------------------------------------- dQ
// kW waves of 32 queries per workgroup (4 or 8). With splits > 1 the key tiles of each query
// block are divided into `splits` consecutive ranges, one workgroup each, which write unscaled
// f32 partial sums to `partial` (split after split, each [D / 8][batch * heads * sq][8]: column
// c of row r at (c / 8, r, c % 8), so the 32 rows of a wave store 1 KB contiguously per
// instruction); attention_bwd_dq_reduce folds them in split order. Used when too few workgroups
// would run.
template <int D, int kW>
__device__ __forceinline__ void attention_bwd_dq_body(
    const uint16_t *__restrict__ Q, const uint16_t *__restrict__ K, const uint16_t *__restrict__ V,
    const uint16_t *__restrict__ G, const float *__restrict__ LSE, const float *__restrict__ DELTA,
    uint16_t *__restrict__ DQ, float *__restrict__ partial, int heads, int head_group, int sq, int sk,
    BwdGeometry g, float scale, int causal, int q_blocks, int splits, uint4 *lds) {
  constexpr int kChunks = kTile * D / 8;          // 16-byte chunks of one K (or V) tile
  constexpr int kDma = kChunks / (kW * 64);        // per thread per operand
  constexpr int kQRows = kW * 32;
  static_assert(kDma * kW * 64 == kChunks, "DMA split");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int split = static_cast<int>(blockIdx.x) % splits;
  const int item = static_cast<int>(blockIdx.x) / splits;
  const int bh_count = gridDim.x / (q_blocks * splits);
  const int qb = q_blocks - 1 - item / bh_count;   // heaviest blocks first
  const int bh = item % bh_count;
  const int b = bh / heads, h = bh % heads, kh = h / head_group;
  const uint16_t *kbase = K + b * g.k[0] + kh * g.k[1];
  const uint16_t *vbase = V + b * g.v[0] + kh * g.v[1];

  const int wq0 = qb * kQRows + wave * 32;
  const int lane_q = wq0 + (lane & 31);
  const int half = lane >> 5;
  const bool q_ok = lane_q < sq;
  const int qr = q_ok ? lane_q : 0;

  f16x8_t qf[D / 16], of[D / 16];
  {
    const uint16_t *qrow = Q + b * g.q[0] + h * g.q[1] + static_cast<int64_t>(qr) * g.q[2];
    const uint16_t *grow = G + b * g.dout[0] + h * g.dout[1] + static_cast<int64_t>(qr) * g.dout[2];
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      qf[ks] = __builtin_bit_cast(f16x8_t, select(q_ok, *reinterpret_cast<const uint4 *>(qrow + ks * 16 + half * 8)));
      of[ks] = __builtin_bit_cast(f16x8_t, select(q_ok, *reinterpret_cast<const uint4 *>(grow + ks * 16 + half * 8)));
    }
  }
  const float lse2 = q_ok ? LSE[b * g.lse[0] + h * g.lse[1] + static_cast<int64_t>(qr) * g.lse[2]] * kLog2e : 0.0f;
  const float dlt = q_ok ? DELTA[b * g.delta[0] + h * g.delta[1] + static_cast<int64_t>(qr) * g.delta[2]] : 0.0f;
  INTENT_WAIT_VMCNT0();

  const int q_last_block = min(qb * kQRows + kQRows, sq) - 1;
  const int k_end = causal ? min(sk, q_last_block + 1) : sk;
  const int all_tiles = (k_end + kTile - 1) / kTile;
  const int t_begin = split * all_tiles / splits, t_end = (split + 1) * all_tiles / splits;
  const int wave_q_last = min(wq0 + 31, sq - 1);

  // Key tile kt goes to stage (kt - t_begin) % kStages.
  auto issue = [&](int kt) {
    uint4 *stage = lds + ((kt - t_begin) % kStages) * 2 * kChunks;
    const int key0 = kt * kTile;
#pragma unroll
    for (int i = 0; i < kDma; ++i) {
      const int p = (wave * kDma + i) * 64 + lane;
      const int row = p / (D / 8), pc = p % (D / 8);
      const int key = min(key0 + row, sk - 1);
      const int src = (pc ^ swz<D>(row)) * 8;
      __builtin_amdgcn_global_load_lds(kbase + static_cast<int64_t>(key) * g.k[2] + src,
                                       (lds_void_t *)(stage + (wave * kDma + i) * 64), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(vbase + static_cast<int64_t>(key) * g.v[2] + src,
                                       (lds_void_t *)(stage + kChunks + (wave * kDma + i) * 64), 16, 0, 0);
    }
  };

  f32x16_t acc[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[mt][e] = 0.0f;
  const float c1 = scale * kLog2e;
  const int frag_row = lane & 31;
  const int g16 = lane >> 4, i16 = lane & 15;
  const int t_row = 4 * (g16 >> 1) + (i16 >> 2);
  const int t_col = 16 * (g16 & 1) + 4 * (i16 & 3);

  // Tiles holding excluded pairs: keys past this wave's first query (causal) or past the end.
  auto edge_tile = [&](int key0) { return (causal && key0 + kTile - 1 > wq0) || key0 + kTile > sk; };
  bool skipped = false;   // wave-uniform: some edge tile was left for the masked fold

  for (int kt = t_begin; kt < t_begin + 2 && kt < t_end; ++kt) issue(kt);
  for (int kt = t_begin; kt < t_end; ++kt) {
    if (((kt - t_begin) & 1) == 0) {   // one barrier per two tiles
      INTENT_WAIT_VMCNT0();
      __syncthreads();          // tiles kt, kt + 1 are in LDS; every wave is done with kt - 2, kt - 1
      if (kt + 2 < t_end) issue(kt + 2);
      if (kt + 3 < t_end) issue(kt + 3);
    }
    const int key0 = kt * kTile;
    if ((causal && key0 > wave_q_last) || wq0 >= sq) continue;   // wave-uniform
    const uint4 *ktile = lds + ((kt - t_begin) % kStages) * 2 * kChunks;
    const uint4 *vtile = ktile + kChunks;
    const uint16_t *kt16 = reinterpret_cast<const uint16_t *>(ktile);
    if (edge_tile(key0) && tile_nonfinite<D>(ktile, lane)) {   // folded after the loop
      skipped = true;
      continue;
    }
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      f16x8_t dsf[2];
      f32x16_t s, dp;
#pragma unroll
      for (int e = 0; e < 16; ++e) s[e] = dp[e] = 0.0f;
      __builtin_amdgcn_iglp_opt(0);   // hipcc's DS/MFMA interleave for the loop below
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
        s = mma(row_frag<D>(ktile, st * 32 + frag_row, ks, half), qf[ks], s);
        dp = mma(row_frag<D>(vtile, st * 32 + frag_row, ks, half), of[ks], dp);
      }
      __builtin_amdgcn_s_setprio(0);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = key0 + st * 32 + 8 * (e >> 2) + 4 * half + (e & 3);
        const bool valid = key < sk && (!causal || key <= lane_q);
        const float p = valid ? __builtin_amdgcn_exp2f(fmaf(s[e], c1, -lse2)) : 0.0f;
        dsf[e >> 3][e & 7] = round_to<_Float16>(valid ? p * (dp[e] - dlt) : 0.0f);
      }
      // This half's 32 keys are 16-key slices 2 st and 2 st + 1 of the tile.
      __builtin_amdgcn_iglp_opt(0);   // hipcc's DS/MFMA interleave for the loop below
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
        for (int mt = 0; mt < D / 32; ++mt) acc[mt] = mma(tr_frag<D>(kt16, st * 2 + h2, mt, t_row, t_col), dsf[h2], acc[mt]);
      __builtin_amdgcn_s_setprio(0);
    }
  }

  // Edge tiles left out above (K rows with an inf or NaN): fold their valid keys one by one.
  if (skipped) {
#pragma unroll 1
    for (int kt = t_begin; kt < t_end; ++kt) {
      const int key0 = kt * kTile;
      if ((causal && key0 > wave_q_last) || !edge_tile(key0) || !rows_nonfinite<D>(kbase, g.k[2], key0, sk - 1, lane))
        continue;
      const int last = (causal ? min(sk - 1, lane_q) : sk - 1) - key0;   // last valid tile row of this query
#pragma unroll 1
      for (int j = 0; j < kTile; ++j) {
        const int key = min(key0 + j, sk - 1);
        const uint16_t *krow = kbase + static_cast<int64_t>(key) * g.k[2];
        const float s = pair_dot<D>(qf, krow, half);
        const float dp = pair_dot<D>(of, vbase + static_cast<int64_t>(key) * g.v[2], half);
        if (j > last) continue;
        const float p = __builtin_amdgcn_exp2f(fmaf(s, c1, -lse2));
        add_row<D>(acc, static_cast<float>(round_to<_Float16>(p * (dp - dlt))), krow, half);
      }
    }
  }

  if (!q_ok) return;
  if (partial != nullptr) {
    const int64_t rows = static_cast<int64_t>(bh_count) * sq;
    float *pslot = partial + split * rows * D + (static_cast<int64_t>(bh) * sq + lane_q) * 8 + 4 * half;
#pragma unroll
    for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq)
        *reinterpret_cast<float4 *>(pslot + (mt * 4 + gq) * rows * 8) =
            make_float4(acc[mt][4 * gq], acc[mt][4 * gq + 1], acc[mt][4 * gq + 2], acc[mt][4 * gq + 3]);
    return;
  }
  uint16_t *orow = DQ + b * g.out0[0] + h * g.out0[1] + static_cast<int64_t>(lane_q) * g.out0[2];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq)
      *reinterpret_cast<uint2 *>(orow + mt * 32 + 8 * gq + 4 * half) =
          make_uint2(pack_f16x2(acc[mt][4 * gq] * scale, acc[mt][4 * gq + 1] * scale),
                     pack_f16x2(acc[mt][4 * gq + 2] * scale, acc[mt][4 * gq + 3] * scale));
}

template <int D, int kW>
__global__ __launch_bounds__(kW * 64, 1) void attention_bwd_dq(
    const uint16_t *__restrict__ Q, const uint16_t *__restrict__ K, const uint16_t *__restrict__ V,
    const uint16_t *__restrict__ G, const float *__restrict__ LSE, const float *__restrict__ DELTA,
    uint16_t *__restrict__ DQ, float *__restrict__ partial, int heads, int head_group, int sq, int sk,
    BwdGeometry g, float scale, int causal, int q_blocks, int splits) {
  constexpr int kChunks = kTile * D / 8;
  __shared__ uint4 lds[kStages * 2 * kChunks];
  attention_bwd_dq_body<D, kW>(Q, K, V, G, LSE, DELTA, DQ, partial, heads, head_group, sq, sk, g, scale, causal,
                               q_blocks, splits, lds);
}

// dQ = f16(scale * sum over the splits of the partial dQ), in split order; four columns per thread.
template <int D>
__global__ __launch_bounds__(kThreads) void attention_bwd_dq_reduce(const float *__restrict__ partial,
                                                                    uint16_t *__restrict__ DQ, int heads, int sq,
                                                                    int splits, int64_t rows, BwdGeometry g,
                                                                    float scale) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (t >= rows * (D / 4)) return;
  const int64_t e = 4 * t, row = e % (rows * 8) / 8;   // partial layout: [column / 8][row][column % 8]
  const int col = static_cast<int>(e / (rows * 8)) * 8 + static_cast<int>(e % 8);
  const int64_t q = row % sq, bh = row / sq;
  const int64_t b = bh / heads, h = bh % heads;
  float4 s4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int i = 0; i < splits; ++i) {
    const float4 a = *reinterpret_cast<const float4 *>(partial + i * rows * D + e);
    s4 = make_float4(s4.x + a.x, s4.y + a.y, s4.z + a.z, s4.w + a.w);
  }
  uint16_t *qrow = DQ + b * g.out0[0] + h * g.out0[1] + q * g.out0[2];
  *reinterpret_cast<uint2 *>(qrow + col) =
      make_uint2(pack_f16x2(s4.x * scale, s4.y * scale), pack_f16x2(s4.z * scale, s4.w * scale));
}

// ---------------------------------------------------------------- dK / dV
// kSplit: the workgroup takes one query head of the group and one of `qsplits` consecutive
// ranges of its query tiles (grid x head_group x qsplits) and writes its unscaled f32 dK and dV
// sums to `partial` (head_group * qsplits parts of dK, then as many of dV, each
// [D / 8][batch * kv_heads * sk][8] as in dQ), which attention_bwd_dkdv_reduce folds. Used when too
// few workgroups would run.
// kPart: dK and dV together, or one of them (DkdvPart); kW: waves of 32 keys per workgroup.
template <int D, bool kSplit, int kPart, int kW>
__device__ __forceinline__ void attention_bwd_dkdv_body(
    const uint16_t *__restrict__ Q, const uint16_t *__restrict__ K, const uint16_t *__restrict__ V,
    const uint16_t *__restrict__ G, const float *__restrict__ LSE, const float *__restrict__ DELTA,
    uint16_t *__restrict__ DK, uint16_t *__restrict__ DV, float *__restrict__ partial, int kv_heads,
    int head_group, int sq, int sk, BwdGeometry g, float scale, int causal, int k_blocks, int qsplits, uint4 *lds) {
  constexpr int kChunks = kTile * D / 8;          // 16-byte chunks of one Q (or dO) tile
  constexpr int kDma = kChunks / (kW * 64);
  constexpr int kKRows = kW * 32;
  constexpr bool kDoK = kPart != kOnlyDv, kDoV = kPart != kOnlyDk;
  static_assert(kDma * kW * 64 == kChunks, "DMA split");
  constexpr int kStage = 2 * kChunks + 2 * (kTile / 4);   // Q, dO, then lse and delta (64 floats each)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bh_count = gridDim.x / k_blocks;
  const int kb = static_cast<int>(blockIdx.x) / bh_count;   // causal: first key blocks see the most queries
  const int bhs = static_cast<int>(blockIdx.x) % bh_count;
  const int qs = kSplit ? bhs % qsplits : 0;                 // the query-tile range (split mode)
  const int rest = kSplit ? bhs / qsplits : bhs;
  const int split = kSplit ? rest % head_group : 0;          // the query head of the group (split mode)
  const int bh = kSplit ? rest / head_group : rest;
  const int b = bh / kv_heads, kh = bh % kv_heads;

  const int wk0 = kb * kKRows + wave * 32;
  const int lane_k = wk0 + (lane & 31);
  const int half = lane >> 5;
  const bool k_ok = lane_k < sk;
  const int kr = k_ok ? lane_k : 0;

  f16x8_t kf[D / 16], vf[D / 16];
  {
    const uint16_t *krow = K + b * g.k[0] + kh * g.k[1] + static_cast<int64_t>(kr) * g.k[2];
    const uint16_t *vrow = V + b * g.v[0] + kh * g.v[1] + static_cast<int64_t>(kr) * g.v[2];
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      kf[ks] = __builtin_bit_cast(f16x8_t, select(k_ok, *reinterpret_cast<const uint4 *>(krow + ks * 16 + half * 8)));
      if constexpr (kDoK)
        vf[ks] = __builtin_bit_cast(f16x8_t, select(k_ok, *reinterpret_cast<const uint4 *>(vrow + ks * 16 + half * 8)));
    }
    INTENT_WAIT_VMCNT0();
  }

  // Query tiles: for each of the head_group query heads, the 64-query tiles that can hold a valid
  // pair for this workgroup's keys (causal: queries >= its first key).
  const int q_tiles = (sq + kTile - 1) / kTile;
  const int first_all = causal ? min(kb * kKRows / kTile, q_tiles) : 0;
  const int span = q_tiles - first_all;
  const int first = first_all + (kSplit ? qs * span / qsplits : 0);
  const int per_head = kSplit ? first_all + (qs + 1) * span / qsplits - first : span;
  const int tiles = (kSplit ? 1 : head_group) * per_head;

  auto tile_head = [&](int t) { return kh * head_group + (kSplit ? split : t / per_head); };
  auto tile_q0 = [&](int t) { return (first + t % per_head) * kTile; };
  auto issue = [&](int t) {
    uint4 *stage = lds + (t % kStages) * kStage;
    const int hq = tile_head(t), q0 = tile_q0(t);
    const uint16_t *qbase = Q + b * g.q[0] + hq * g.q[1];
    const uint16_t *gbase = G + b * g.dout[0] + hq * g.dout[1];
#pragma unroll
    for (int i = 0; i < kDma; ++i) {
      const int p = (wave * kDma + i) * 64 + lane;
      const int row = p / (D / 8), pc = p % (D / 8);
      const int q = min(q0 + row, sq - 1);
      const int src = (pc ^ swz<D>(row)) * 8;
      __builtin_amdgcn_global_load_lds(qbase + static_cast<int64_t>(q) * g.q[2] + src,
                                       (lds_void_t *)(stage + (wave * kDma + i) * 64), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(gbase + static_cast<int64_t>(q) * g.dout[2] + src,
                                       (lds_void_t *)(stage + kChunks + (wave * kDma + i) * 64), 16, 0, 0);
    }
    if (wave < (kDoK ? 2 : 1)) {   // lse (wave 0) and delta (wave 1): one float of row q0 + lane per lane
      const int q = min(q0 + lane, sq - 1);
      const float *src = wave == 0 ? LSE + b * g.lse[0] + hq * g.lse[1] + static_cast<int64_t>(q) * g.lse[2]
                                   : DELTA + b * g.delta[0] + hq * g.delta[1] + static_cast<int64_t>(q) * g.delta[2];
      __builtin_amdgcn_global_load_lds(src, (lds_void_t *)(stage + 2 * kChunks + wave * (kTile / 4)), 4, 0, 0);
    }
  };

  f32x16_t acc_k[D / 32], acc_v[D / 32];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc_k[mt][e] = acc_v[mt][e] = 0.0f;
  const float c1 = scale * kLog2e;
  const int frag_row = lane & 31;
  const int g16 = lane >> 4, i16 = lane & 15;
  const int t_row = 4 * (g16 >> 1) + (i16 >> 2);
  const int t_col = 16 * (g16 & 1) + 4 * (i16 & 3);

  // Tiles holding excluded pairs: queries before this wave's last key (causal) or past the end.
  auto edge_tile = [&](int q0) { return (causal && q0 < wk0 + 31) || q0 + kTile > sq; };
  bool skipped = false;   // wave-uniform: some edge tile was left for the masked fold

  for (int t = 0; t < 2 && t < tiles; ++t) issue(t);
  for (int t = 0; t < tiles; ++t) {
    if ((t & 1) == 0) {   // one barrier per two tiles
      INTENT_WAIT_VMCNT0();
      __syncthreads();          // tiles t, t + 1 are in LDS; every wave is done with t - 2, t - 1
      if (t + 2 < tiles) issue(t + 2);
      if (t + 3 < tiles) issue(t + 3);
    }
    const int q0 = tile_q0(t);
    if (wk0 >= sk || (causal && q0 + kTile - 1 < wk0)) continue;   // wave-uniform: no valid pair
    const uint4 *qtile = lds + (t % kStages) * kStage;
    const uint4 *gtile = qtile + kChunks;
    const float *lse_s = reinterpret_cast<const float *>(qtile + 2 * kChunks);
    const float *dlt_s = lse_s + kTile;
    // lse_s[i] / dlt_s[i] hold row q0 + i (the last row for i past the end, excluded by the mask).
    const uint16_t *q16 = reinterpret_cast<const uint16_t *>(qtile);
    const uint16_t *g16p = reinterpret_cast<const uint16_t *>(gtile);
    if (edge_tile(q0) && ((kDoK && tile_nonfinite<D>(qtile, lane)) || (kDoV && tile_nonfinite<D>(gtile, lane)))) {
      skipped = true;   // folded after the loop
      continue;
    }
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      f16x8_t pf[2], dsf[2];
      f32x16_t s, dp;
#pragma unroll
      for (int e = 0; e < 16; ++e) s[e] = dp[e] = 0.0f;
      __builtin_amdgcn_iglp_opt(0);   // hipcc's DS/MFMA interleave for the loop below
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
        s = mma(row_frag<D>(qtile, st * 32 + frag_row, ks, half), kf[ks], s);
        if constexpr (kDoK) dp = mma(row_frag<D>(gtile, st * 32 + frag_row, ks, half), vf[ks], dp);
      }
      __builtin_amdgcn_s_setprio(0);
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int local = st * 32 + 8 * e4 + 4 * half;        // rows local .. local + 3 of the tile
        const float4 l4 = *reinterpret_cast<const float4 *>(lse_s + local);
        const float4 d4 = kDoK ? *reinterpret_cast<const float4 *>(dlt_s + local) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const float lv[4] = {l4.x, l4.y, l4.z, l4.w}, dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int e = 4 * e4 + j;
          const int q = q0 + local + j;
          const bool valid = q < sq && (!causal || lane_k <= q);
          const float p = valid ? __builtin_amdgcn_exp2f(fmaf(s[e], c1, -lv[j] * kLog2e)) : 0.0f;
          if constexpr (kDoV) pf[e >> 3][e & 7] = static_cast<_Float16>(p);
          if constexpr (kDoK) dsf[e >> 3][e & 7] = round_to<_Float16>(valid ? p * (dp[e] - dv[j]) : 0.0f);
        }
      }
      // This half's 32 queries are 16-query slices 2 st and 2 st + 1 of the tile.
      __builtin_amdgcn_iglp_opt(0);   // hipcc's DS/MFMA interleave for the loop below
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
        for (int mt = 0; mt < D / 32; ++mt) {
          if constexpr (kDoV) acc_v[mt] = mma(tr_frag<D>(g16p, st * 2 + h2, mt, t_row, t_col), pf[h2], acc_v[mt]);
          if constexpr (kDoK) acc_k[mt] = mma(tr_frag<D>(q16, st * 2 + h2, mt, t_row, t_col), dsf[h2], acc_k[mt]);
        }
      __builtin_amdgcn_s_setprio(0);
    }
  }

  // Edge tiles left out above (Q or dO rows with an inf or NaN): fold their valid queries one by one.
  if (skipped) {
#pragma unroll 1
    for (int t = 0; t < tiles; ++t) {
      const int q0 = tile_q0(t);
      if ((causal && q0 + kTile - 1 < wk0) || !edge_tile(q0)) continue;
      const int hq = tile_head(t);
      const uint16_t *qbase = Q + b * g.q[0] + hq * g.q[1];
      const uint16_t *gbase = G + b * g.dout[0] + hq * g.dout[1];
      if (!((kDoK && rows_nonfinite<D>(qbase, g.q[2], q0, sq - 1, lane)) ||
            (kDoV && rows_nonfinite<D>(gbase, g.dout[2], q0, sq - 1, lane))))
        continue;
      const int first = causal ? lane_k - q0 : 0, last = sq - 1 - q0;   // valid tile rows of this key
#pragma unroll 1
      for (int j = 0; j < kTile; ++j) {
        const int q = min(q0 + j, sq - 1);
        const uint16_t *qrow = qbase + static_cast<int64_t>(q) * g.q[2];
        const uint16_t *grow = gbase + static_cast<int64_t>(q) * g.dout[2];
        const float s = pair_dot<D>(kf, qrow, half);
        float dp = 0.0f;
        if constexpr (kDoK) dp = pair_dot<D>(vf, grow, half);
        if (j < first || j > last) continue;
        const float p = __builtin_amdgcn_exp2f(
            fmaf(s, c1, -LSE[b * g.lse[0] + hq * g.lse[1] + static_cast<int64_t>(q) * g.lse[2]] * kLog2e));
        if constexpr (kDoV) add_row<D>(acc_v, static_cast<float>(static_cast<_Float16>(p)), grow, half);
        if constexpr (kDoK) {
          const float dl = DELTA[b * g.delta[0] + hq * g.delta[1] + static_cast<int64_t>(q) * g.delta[2]];
          add_row<D>(acc_k, static_cast<float>(round_to<_Float16>(p * (dp - dl))), qrow, half);
        }
      }
    }
  }

  if (!k_ok) return;
  if constexpr (kSplit) {
    const int64_t rows = static_cast<int64_t>(gridDim.x / (k_blocks * head_group * qsplits)) * sk;   // batch * kv_heads * sk
    const int64_t row = (static_cast<int64_t>(b) * kv_heads + kh) * sk + lane_k;
    const int parts = head_group * qsplits, part = split * qsplits + qs;
    float *pk = partial + part * rows * D + row * 8 + 4 * half;
    float *pv = partial + (parts + part) * rows * D + row * 8 + 4 * half;
#pragma unroll
    for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int64_t block = (mt * 4 + gq) * rows * 8;   // partial layout: [column / 8][row][column % 8]
        if constexpr (kDoK)
          *reinterpret_cast<float4 *>(pk + block) =
              make_float4(acc_k[mt][4 * gq], acc_k[mt][4 * gq + 1], acc_k[mt][4 * gq + 2], acc_k[mt][4 * gq + 3]);
        if constexpr (kDoV)
          *reinterpret_cast<float4 *>(pv + block) =
              make_float4(acc_v[mt][4 * gq], acc_v[mt][4 * gq + 1], acc_v[mt][4 * gq + 2], acc_v[mt][4 * gq + 3]);
      }
    return;
  }
  uint16_t *krow = DK + b * g.out0[0] + kh * g.out0[1] + static_cast<int64_t>(lane_k) * g.out0[2];
  uint16_t *vrow = DV + b * g.out1[0] + kh * g.out1[1] + static_cast<int64_t>(lane_k) * g.out1[2];
#pragma unroll
  for (int mt = 0; mt < D / 32; ++mt)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int col = mt * 32 + 8 * gq + 4 * half;
      if constexpr (kDoK)
        *reinterpret_cast<uint2 *>(krow + col) =
            make_uint2(pack_f16x2(acc_k[mt][4 * gq] * scale, acc_k[mt][4 * gq + 1] * scale),
                       pack_f16x2(acc_k[mt][4 * gq + 2] * scale, acc_k[mt][4 * gq + 3] * scale));
      if constexpr (kDoV)
        *reinterpret_cast<uint2 *>(vrow + col) = make_uint2(pack_f16x2(acc_v[mt][4 * gq], acc_v[mt][4 * gq + 1]),
                                                            pack_f16x2(acc_v[mt][4 * gq + 2], acc_v[mt][4 * gq + 3]));
    }
}

template <int D, bool kSplit, int kPart, int kW>
__global__ __launch_bounds__(kW * 64, 1) void attention_bwd_dkdv(
    const uint16_t *__restrict__ Q, const uint16_t *__restrict__ K, const uint16_t *__restrict__ V,
    const uint16_t *__restrict__ G, const float *__restrict__ LSE, const float *__restrict__ DELTA,
    uint16_t *__restrict__ DK, uint16_t *__restrict__ DV, float *__restrict__ partial, int kv_heads,
    int head_group, int sq, int sk, BwdGeometry g, float scale, int causal, int k_blocks, int qsplits) {
  constexpr int kStage = 2 * (kTile * D / 8) + 2 * (kTile / 4);
  __shared__ uint4 lds[kStages * kStage];
  attention_bwd_dkdv_body<D, kSplit, kPart, kW>(Q, K, V, G, LSE, DELTA, DK, DV, partial, kv_heads, head_group, sq, sk, g,
                                     scale, causal, k_blocks, qsplits, lds);
}

// dK = f16(scale * sum of the `parts` partial dK), dV = f16(sum of the partial dV); four columns
// per thread, in part order (query head of the group, then query-tile range).
template <int D>
__global__ __launch_bounds__(kThreads) void attention_bwd_dkdv_reduce(const float *__restrict__ partial,
                                                                      uint16_t *__restrict__ DK,
                                                                      uint16_t *__restrict__ DV, int kv_heads,
                                                                      int parts, int sk, int64_t rows,
                                                                      BwdGeometry g, float scale) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (t >= rows * (D / 4)) return;
  const int64_t e = 4 * t, row = e % (rows * 8) / 8;   // partial layout: [column / 8][row][column % 8]
  const int col = static_cast<int>(e / (rows * 8)) * 8 + static_cast<int>(e % 8);
  const int64_t k = row % sk, bh = row / sk;
  const int64_t b = bh / kv_heads, kh = bh % kv_heads;
  float4 sk4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), sv4 = sk4;
  for (int i = 0; i < parts; ++i) {
    const float4 a = *reinterpret_cast<const float4 *>(partial + i * rows * D + e);
    const float4 c = *reinterpret_cast<const float4 *>(partial + (parts + i) * rows * D + e);
    sk4 = make_float4(sk4.x + a.x, sk4.y + a.y, sk4.z + a.z, sk4.w + a.w);
    sv4 = make_float4(sv4.x + c.x, sv4.y + c.y, sv4.z + c.z, sv4.w + c.w);
  }
  uint16_t *krow = DK + b * g.out0[0] + kh * g.out0[1] + k * g.out0[2];
  uint16_t *vrow = DV + b * g.out1[0] + kh * g.out1[1] + k * g.out1[2];
  *reinterpret_cast<uint2 *>(krow + col) =
      make_uint2(pack_f16x2(sk4.x * scale, sk4.y * scale), pack_f16x2(sk4.z * scale, sk4.w * scale));
  *reinterpret_cast<uint2 *>(vrow + col) = make_uint2(pack_f16x2(sv4.x, sv4.y), pack_f16x2(sv4.z, sv4.w));
}

}  // namespace
}  // namespace intent_hip

namespace intent_hip {

// rows: batch x heads x sequence of the call (query heads and queries for dQ, key heads and keys
// for dK/dV); it selects the variant as the launch does. Wide dK/dV launches two kernels; the
// first (dK) is described.
int attention_bwd_resources(int64_t which, int64_t rows, int64_t d, IntentHipKernelResources *out) {
  const bool d64 = d == 64, wide = rows >= kWideRows;
  const auto describe = [out](const void *kernel, const char *name, int threads) {
    return describe_kernel(kernel, name, threads, out);
  };
  switch (which) {
    case 0:
      return d64 ? describe(reinterpret_cast<const void *>(&attention_bwd_delta<64>), "attention_bwd_delta<64>", kThreads)
                 : describe(reinterpret_cast<const void *>(&attention_bwd_delta<128>), "attention_bwd_delta<128>",
                            kThreads);
    case 1:
      if (wide)
        return d64 ? describe(reinterpret_cast<const void *>(&attention_bwd_dq<64, 8>), "attention_bwd_dq<64,8>", 512)
                   : describe(reinterpret_cast<const void *>(&attention_bwd_dq<128, 8>), "attention_bwd_dq<128,8>", 512);
      return d64 ? describe(reinterpret_cast<const void *>(&attention_bwd_dq<64, 4>), "attention_bwd_dq<64,4>", kThreads)
                 : describe(reinterpret_cast<const void *>(&attention_bwd_dq<128, 4>), "attention_bwd_dq<128,4>",
                            kThreads);
    default:
      if (wide)
        return d64 ? describe(reinterpret_cast<const void *>(&attention_bwd_dkdv<64, false, kOnlyDk, 8>),
                              "attention_bwd_dk<64,8>", 512)
                   : describe(reinterpret_cast<const void *>(&attention_bwd_dkdv<128, false, kOnlyDk, 8>),
                              "attention_bwd_dk<128,8>", 512);
      return d64 ? describe(reinterpret_cast<const void *>(&attention_bwd_dkdv<64, false, kBoth, 4>),
                            "attention_bwd_dkdv<64,4>", kThreads)
                 : describe(reinterpret_cast<const void *>(&attention_bwd_dkdv<128, false, kBoth, 4>),
                            "attention_bwd_dkdv<128,4>", kThreads);
  }
}

namespace {

// Shared checks of the 4-D f16 operands: unit inner stride, other strides multiples of 8
// elements, 16-byte aligned starts (8-byte for outputs written 4 elements at a time).
int check_operand(const void *p, const int64_t *st, int out, const char *name) {
  if (st[3] != 1) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "%s needs unit inner stride", name);
  for (int i = 0; i < 3; ++i)
    if (st[i] % (out ? 4 : 8))
      return fail(INTENT_HIP_ERR_UNSUPPORTED, "%s strides must be multiples of %d elements", name, out ? 4 : 8);
  if (!aligned(p, out ? 8 : 16)) return fail(INTENT_HIP_ERR_UNSUPPORTED, "%s must be %d-byte aligned", name, out ? 8 : 16);
  return INTENT_HIP_OK;
}

int check_common(int64_t batch, int64_t q_heads, int64_t head_group, int64_t sq, int64_t sk, int64_t d) {
  if (batch < 0 || q_heads < 0 || sq < 0 || sk < 0 || d < 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (head_group < 1 || (q_heads > 0 && q_heads % head_group != 0))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "head_group %lld must be positive and divide the %lld query heads",
                static_cast<long long>(head_group), static_cast<long long>(q_heads));
  if (d != 64 && d != 128)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "attention backward supports head dimension 64 or 128 (got %lld)",
                static_cast<long long>(d));
  if (sq > INT32_MAX / 2 || sk > INT32_MAX / 2 || batch * q_heads > INT32_MAX / 64)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "attention extents too large for one launch");
  return INTENT_HIP_OK;
}

void load_geometry(BwdGeometry &g, const int64_t *s, bool two_outputs) {
  for (int i = 0; i < 4; ++i) {
    g.q[i] = s[i];
    g.k[i] = s[4 + i];
    g.v[i] = s[8 + i];
    g.dout[i] = s[12 + i];
    g.out0[i] = s[22 + i];
    g.out1[i] = two_outputs ? s[26 + i] : 0;
  }
  for (int i = 0; i < 3; ++i) {
    g.lse[i] = s[16 + i];
    g.delta[i] = s[19 + i];
  }
}

}  // namespace
}  // namespace intent_hip

using namespace intent_hip;

extern "C" int intent_hip_attention_bwd_delta(const void *o, const void *dout, float *delta, int64_t batch,
                                              int64_t heads, int64_t sq, int64_t d, const int64_t *strides,
                                              void *stream) {
  if (const int rc = check_common(batch, heads, 1, sq, 0, d)) return rc;
  if (batch == 0 || heads == 0 || sq == 0) return INTENT_HIP_OK;
  if (o == nullptr || dout == nullptr || delta == nullptr || strides == nullptr)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null pointer");
  if (int rc = check_operand(o, strides, 0, "output")) return rc;
  if (int rc = check_operand(dout, strides + 4, 0, "grad_output")) return rc;
  BwdGeometry g{};
  for (int i = 0; i < 4; ++i) {
    g.q[i] = strides[i];
    g.dout[i] = strides[4 + i];
  }
  for (int i = 0; i < 3; ++i) g.delta[i] = strides[8 + i];
  const int64_t rows = batch * heads * sq;
  const int64_t threads = rows * (d / 8);
  const dim3 grid(static_cast<unsigned>((threads + kThreads - 1) / kThreads));
  const auto *O = static_cast<const uint16_t *>(o);
  const auto *G = static_cast<const uint16_t *>(dout);
  if (d == 64)
    attention_bwd_delta<64><<<grid, dim3(kThreads), 0, as_stream(stream)>>>(O, G, delta, static_cast<int>(heads),
                                                                            static_cast<int>(sq), rows, g);
  else
    attention_bwd_delta<128><<<grid, dim3(kThreads), 0, as_stream(stream)>>>(O, G, delta, static_cast<int>(heads),
                                                                             static_cast<int>(sq), rows, g);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("attention_bwd_delta");
  return INTENT_HIP_OK;
}

namespace {

// Narrow grids split their work over more workgroups, which write f32 partial sums to a
// caller-owned workspace that a second kernel folds: with fewer than kSplitBelow workgroups of
// the 4-wave kernel, CUs stay idle while one workgroup walks the longest range of tiles alone.
// The split aims at kSplitTarget workgroups (two per CU fit at D = 64), at most kMaxSplits ranges.
// Reference example (B2 HQ8 HK2 S1024 D64 causal, delta + dK/dV + dQ): 88.8 us unsplit except by
// head, 64.3 us aiming at 256 workgroups with up to 4 ranges, 61.5 us with 512 and 8.
constexpr int64_t kSplitBelow = 256;
constexpr int64_t kSplitTarget = 512;
constexpr int64_t kMaxSplits = 8;

// dQ: the number of key-tile ranges per query block (1 = no split).
int dq_splits(int64_t batch, int64_t q_heads, int64_t sq, int64_t sk) {
  if (batch <= 0 || q_heads <= 0 || sq <= 0 || sk <= 0 || batch * q_heads * sq >= kWideRows) return 1;
  const int64_t blocks = batch * q_heads * ((sq + kRows - 1) / kRows);
  if (blocks >= kSplitBelow) return 1;
  int64_t splits = (kSplitTarget + blocks - 1) / blocks;
  splits = splits < kMaxSplits ? splits : kMaxSplits;
  const int64_t key_tiles = (sk + kTile - 1) / kTile;
  return static_cast<int>(splits < key_tiles ? splits : key_tiles);
}

int64_t dq_workspace(int splits, int64_t batch, int64_t q_heads, int64_t sq, int64_t d) {
  return splits > 1 ? splits * batch * q_heads * sq * d * static_cast<int64_t>(sizeof(float)) : 0;
}

// dK/dV: split by query head of the group and by query-tile range; returns the number of ranges
// per head (0 = no split).
int dkdv_qsplits(int64_t batch, int64_t q_heads, int64_t head_group, int64_t sq, int64_t sk) {
  if (batch <= 0 || q_heads <= 0 || sq <= 0 || sk <= 0) return 0;
  const int64_t blocks = batch * (q_heads / head_group) * ((sk + kRows - 1) / kRows);
  if (blocks >= kSplitBelow) return 0;
  int64_t qsplits = (kSplitTarget + blocks * head_group - 1) / (blocks * head_group);
  qsplits = qsplits < kMaxSplits ? qsplits : kMaxSplits;
  const int64_t query_tiles = (sq + kTile - 1) / kTile;
  qsplits = qsplits < query_tiles ? qsplits : query_tiles;
  if (head_group == 1 && qsplits <= 1) return 0;
  return static_cast<int>(qsplits < 1 ? 1 : qsplits);
}

int64_t dkdv_workspace(int qsplits, int64_t batch, int64_t q_heads, int64_t head_group, int64_t sk, int64_t d) {
  return qsplits > 0 ? 2 * head_group * qsplits * batch * (q_heads / head_group) * sk * d *
                           static_cast<int64_t>(sizeof(float))
                     : 0;
}

// attention_bwd_dq<D, kW> over every (batch, query head), block of 32 kW queries and key range;
// with splits > 1 the partial sums in `partial` are then folded by attention_bwd_dq_reduce.
template <int D, int kW>
int launch_dq(const uint16_t *Q, const uint16_t *K, const uint16_t *V, const uint16_t *G, const float *lse,
              const float *delta, uint16_t *DQ, float *partial, int splits, int64_t batch, int64_t q_heads,
              int64_t head_group, int64_t sq, int64_t sk, const BwdGeometry &g, float scale, int causal,
              hipStream_t s) {
  const int q_blocks = static_cast<int>((sq + kW * 32 - 1) / (kW * 32));
  const int64_t blocks = batch * q_heads * q_blocks * splits;
  if (blocks > INT32_MAX) return fail(INTENT_HIP_ERR_UNSUPPORTED, "too many workgroups");
  attention_bwd_dq<D, kW><<<dim3(static_cast<unsigned>(blocks)), dim3(kW * 64), 0, s>>>(
      Q, K, V, G, lse, delta, DQ, splits > 1 ? partial : nullptr, static_cast<int>(q_heads),
      static_cast<int>(head_group), static_cast<int>(sq), static_cast<int>(sk), g, scale, causal, q_blocks, splits);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("attention_bwd_dq");
  if (splits == 1) return INTENT_HIP_OK;
  const int64_t rows = batch * q_heads * sq;
  const dim3 rgrid(static_cast<unsigned>((rows * (D / 4) + kThreads - 1) / kThreads));
  attention_bwd_dq_reduce<D><<<rgrid, dim3(kThreads), 0, s>>>(partial, DQ, static_cast<int>(q_heads),
                                                              static_cast<int>(sq), splits, rows, g, scale);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("attention_bwd_dq_reduce");
  return INTENT_HIP_OK;
}

// attention_bwd_dkdv<D, kSplit, kPart, kW> over every (batch, key head) and block of 32 kW keys
// (times head_group when split).
template <int D, bool kSplit, int kPart, int kW>
int launch_dkdv(const uint16_t *Q, const uint16_t *K, const uint16_t *V, const uint16_t *G, const float *lse,
                const float *delta, uint16_t *DK, uint16_t *DV, float *partial, int64_t batch, int64_t kv_heads,
                int64_t head_group, int64_t sq, int64_t sk, const BwdGeometry &g, float scale, int causal,
                int qsplits, hipStream_t s) {
  const int k_blocks = static_cast<int>((sk + kW * 32 - 1) / (kW * 32));
  const int64_t blocks = batch * kv_heads * k_blocks * (kSplit ? head_group * qsplits : 1);
  if (blocks > INT32_MAX) return fail(INTENT_HIP_ERR_UNSUPPORTED, "too many workgroups");
  attention_bwd_dkdv<D, kSplit, kPart, kW><<<dim3(static_cast<unsigned>(blocks)), dim3(kW * 64), 0, s>>>(
      Q, K, V, G, lse, delta, DK, DV, partial, static_cast<int>(kv_heads), static_cast<int>(head_group),
      static_cast<int>(sq), static_cast<int>(sk), g, scale, causal, k_blocks, qsplits);
  if (hipPeekAtLastError() != hipSuccess)
    return launch_status(kPart == kOnlyDk ? "attention_bwd_dk" : kPart == kOnlyDv ? "attention_bwd_dv" : "attention_bwd_dkdv");
  return INTENT_HIP_OK;
}

// dK and dV of one call: split by query head and query-tile range with a workspace (qsplits > 0;
// then folded), as two 8-wave kernels on wide grids, or as one 4-wave kernel.
template <int D>
int run_dkdv(const uint16_t *Q, const uint16_t *K, const uint16_t *V, const uint16_t *G, const float *lse,
             const float *delta, uint16_t *DK, uint16_t *DV, float *partial, int qsplits, int64_t batch,
             int64_t kv_heads, int64_t head_group, int64_t sq, int64_t sk, const BwdGeometry &g, float scale,
             int causal, hipStream_t s) {
  if (qsplits > 0) {
    if (int rc = launch_dkdv<D, true, kBoth, 4>(Q, K, V, G, lse, delta, DK, DV, partial, batch, kv_heads, head_group,
                                                sq, sk, g, scale, causal, qsplits, s))
      return rc;
    const int64_t rows = batch * kv_heads * sk;
    const dim3 rgrid(static_cast<unsigned>((rows * (D / 4) + kThreads - 1) / kThreads));
    attention_bwd_dkdv_reduce<D><<<rgrid, dim3(kThreads), 0, s>>>(partial, DK, DV, static_cast<int>(kv_heads),
                                                                  static_cast<int>(head_group * qsplits),
                                                                  static_cast<int>(sk), rows, g, scale);
    if (hipPeekAtLastError() != hipSuccess) return launch_status("attention_bwd_dkdv_reduce");
    return INTENT_HIP_OK;
  }
  if (batch * kv_heads * sk >= kWideRows) {
    if (int rc = launch_dkdv<D, false, kOnlyDk, 8>(Q, K, V, G, lse, delta, DK, DV, nullptr, batch, kv_heads,
                                                   head_group, sq, sk, g, scale, causal, 1, s))
      return rc;
    return launch_dkdv<D, false, kOnlyDv, 8>(Q, K, V, G, lse, delta, DK, DV, nullptr, batch, kv_heads, head_group, sq,
                                             sk, g, scale, causal, 1, s);
  }
  return launch_dkdv<D, false, kBoth, 4>(Q, K, V, G, lse, delta, DK, DV, nullptr, batch, kv_heads, head_group, sq, sk,
                                         g, scale, causal, 1, s);
}

}  // namespace

extern "C" int intent_hip_attention_bwd_dq_workspace_bytes(int64_t batch, int64_t q_heads, int64_t head_group,
                                                           int64_t sq, int64_t sk, int64_t d, size_t *bytes) {
  if (bytes == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null output");
  if (const int rc = check_common(batch, q_heads, head_group, sq, sk, d)) return rc;
  *bytes = static_cast<size_t>(dq_workspace(dq_splits(batch, q_heads, sq, sk), batch, q_heads, sq, d));
  return INTENT_HIP_OK;
}

extern "C" int intent_hip_attention_bwd_dq_ws(const void *q, const void *k, const void *v, const void *dout,
                                              const float *lse, const float *delta, void *dq, int64_t batch,
                                              int64_t q_heads, int64_t head_group, int64_t sq, int64_t sk, int64_t d,
                                              const int64_t *strides, float scale, int causal, void *workspace,
                                              size_t workspace_bytes, void *stream) {
  if (const int rc = check_common(batch, q_heads, head_group, sq, sk, d)) return rc;
  if (batch == 0 || q_heads == 0 || sq == 0) return INTENT_HIP_OK;
  if (strides == nullptr || q == nullptr || dout == nullptr || lse == nullptr || delta == nullptr || dq == nullptr ||
      (sk > 0 && (k == nullptr || v == nullptr)))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null pointer");
  if (int rc = check_operand(q, strides, 0, "q")) return rc;
  if (int rc = check_operand(k, strides + 4, 0, "k")) return rc;
  if (int rc = check_operand(v, strides + 8, 0, "v")) return rc;
  if (int rc = check_operand(dout, strides + 12, 0, "grad_output")) return rc;
  if (int rc = check_operand(dq, strides + 22, 1, "grad_q")) return rc;
  BwdGeometry g{};
  load_geometry(g, strides, false);
  int splits = dq_splits(batch, q_heads, sq, sk);
  const int64_t need = dq_workspace(splits, batch, q_heads, sq, d);
  if (need > 0 && workspace != nullptr && (workspace_bytes < static_cast<size_t>(need) || !aligned(workspace, 16)))
    return fail(INTENT_HIP_ERR_WORKSPACE, "dQ needs %lld 16-byte aligned workspace bytes, got %zu",
                static_cast<long long>(need), workspace_bytes);
  if (workspace == nullptr) splits = 1;
  const auto *Q = static_cast<const uint16_t *>(q);
  const auto *K = static_cast<const uint16_t *>(k);
  const auto *V = static_cast<const uint16_t *>(v);
  const auto *G = static_cast<const uint16_t *>(dout);
  auto *DQ = static_cast<uint16_t *>(dq);
  auto *P = static_cast<float *>(workspace);
  const bool wide = batch * q_heads * sq >= kWideRows;
  const int c = causal ? 1 : 0;
  const hipStream_t s = as_stream(stream);
  if (d == 64)
    return wide ? launch_dq<64, 8>(Q, K, V, G, lse, delta, DQ, P, 1, batch, q_heads, head_group, sq, sk, g, scale, c, s)
                : launch_dq<64, 4>(Q, K, V, G, lse, delta, DQ, P, splits, batch, q_heads, head_group, sq, sk, g, scale,
                                   c, s);
  return wide ? launch_dq<128, 8>(Q, K, V, G, lse, delta, DQ, P, 1, batch, q_heads, head_group, sq, sk, g, scale, c, s)
              : launch_dq<128, 4>(Q, K, V, G, lse, delta, DQ, P, splits, batch, q_heads, head_group, sq, sk, g, scale,
                                  c, s);
}

extern "C" int intent_hip_attention_bwd_dq(const void *q, const void *k, const void *v, const void *dout,
                                           const float *lse, const float *delta, void *dq, int64_t batch,
                                           int64_t q_heads, int64_t head_group, int64_t sq, int64_t sk, int64_t d,
                                           const int64_t *strides, float scale, int causal, void *stream) {
  return intent_hip_attention_bwd_dq_ws(q, k, v, dout, lse, delta, dq, batch, q_heads, head_group, sq, sk, d, strides,
                                        scale, causal, nullptr, 0, stream);
}

extern "C" int intent_hip_attention_bwd_dkdv_workspace_bytes(int64_t batch, int64_t q_heads, int64_t head_group,
                                                             int64_t sq, int64_t sk, int64_t d, size_t *bytes) {
  if (bytes == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null output");
  if (const int rc = check_common(batch, q_heads, head_group, sq, sk, d)) return rc;
  *bytes = static_cast<size_t>(
      dkdv_workspace(dkdv_qsplits(batch, q_heads, head_group, sq, sk), batch, q_heads, head_group, sk, d));
  return INTENT_HIP_OK;
}

extern "C" int intent_hip_attention_bwd_dkdv_ws(const void *q, const void *k, const void *v, const void *dout,
                                                const float *lse, const float *delta, void *dk, void *dv,
                                                int64_t batch, int64_t q_heads, int64_t head_group, int64_t sq,
                                                int64_t sk, int64_t d, const int64_t *strides, float scale,
                                                int causal, void *workspace, size_t workspace_bytes, void *stream) {
  if (const int rc = check_common(batch, q_heads, head_group, sq, sk, d)) return rc;
  if (batch == 0 || q_heads == 0 || sk == 0) return INTENT_HIP_OK;
  if (strides == nullptr || k == nullptr || v == nullptr || dk == nullptr || dv == nullptr ||
      (sq > 0 && (q == nullptr || dout == nullptr || lse == nullptr || delta == nullptr)))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null pointer");
  if (int rc = check_operand(q, strides, 0, "q")) return rc;
  if (int rc = check_operand(k, strides + 4, 0, "k")) return rc;
  if (int rc = check_operand(v, strides + 8, 0, "v")) return rc;
  if (int rc = check_operand(dout, strides + 12, 0, "grad_output")) return rc;
  if (int rc = check_operand(dk, strides + 22, 1, "grad_k")) return rc;
  if (int rc = check_operand(dv, strides + 26, 1, "grad_v")) return rc;
  BwdGeometry g{};
  load_geometry(g, strides, true);
  const int64_t kv_heads = q_heads / head_group;
  int qsplits = dkdv_qsplits(batch, q_heads, head_group, sq, sk);
  const int64_t need = dkdv_workspace(qsplits, batch, q_heads, head_group, sk, d);
  if (need > 0 && workspace != nullptr && (workspace_bytes < static_cast<size_t>(need) || !aligned(workspace, 16)))
    return fail(INTENT_HIP_ERR_WORKSPACE, "dK/dV needs %lld 16-byte aligned workspace bytes, got %zu",
                static_cast<long long>(need), workspace_bytes);
  if (workspace == nullptr) qsplits = 0;
  const auto *Q = static_cast<const uint16_t *>(q);
  const auto *K = static_cast<const uint16_t *>(k);
  const auto *V = static_cast<const uint16_t *>(v);
  const auto *G = static_cast<const uint16_t *>(dout);
  auto *DK = static_cast<uint16_t *>(dk);
  auto *DV = static_cast<uint16_t *>(dv);
  auto *P = static_cast<float *>(workspace);
  const hipStream_t s = as_stream(stream);
  const int c = causal ? 1 : 0;
  if (d == 64)
    return run_dkdv<64>(Q, K, V, G, lse, delta, DK, DV, P, qsplits, batch, kv_heads, head_group, sq, sk, g, scale,
                        c, s);
  return run_dkdv<128>(Q, K, V, G, lse, delta, DK, DV, P, qsplits, batch, kv_heads, head_group, sq, sk, g, scale, c,
                       s);
}

extern "C" int intent_hip_attention_bwd_dkdv(const void *q, const void *k, const void *v, const void *dout,
                                             const float *lse, const float *delta, void *dk, void *dv, int64_t batch,
                                             int64_t q_heads, int64_t head_group, int64_t sq, int64_t sk, int64_t d,
                                             const int64_t *strides, float scale, int causal, void *stream) {
  return intent_hip_attention_bwd_dkdv_ws(q, k, v, dout, lse, delta, dk, dv, batch, q_heads, head_group, sq, sk, d,
                                          strides, scale, causal, nullptr, 0, stream);
}
