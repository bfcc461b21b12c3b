// Fused attention forward (f16 in/out, f32 softmax and accumulation) for gfx950.
//
// Semantics: flash_attention_fwd (python/intent/examples/kernels/streaming/attention.py:428-466)
// with summarize_attention_chunk_f16 (:152-191), merge_attention_summaries (:82-114) and
// normalize_attention_summary (:417-425): scores s = (q . k) * (scale * log2 e) in f32, causal
// validity q_idx >= k_idx on absolute indices, masked scores -inf, maximum_num maxima,
// p = exp2(s - max) (approximate, flush-to-zero: v_exp_f32), P rounded to f16 before P @ V
// (f32 accumulation), output acc * rcp(den) (approximate: v_rcp_f32), cast to f16 (RNE).
// The key axis is folded in 64-key chunks, each summarised as the definition's author summarizer
// does: weights against the chunk's own maximum, rounded to the element type, P @ V of the chunk
// from zero, then merged into the running state with exp2 factors on both sides. (The running-
// maximum rewrite of online softmax, which moves where P is rounded, is the compiler's
// relaxed_normalization rewrite; it never applies to author summarizers,
// doc/dsl/types-numerics-and-effects.en.md:142-152.)
//
// Design (d and dv each 64 or 128, independently):
//   * a workgroup owns 256 query rows of one (batch, head): 8 waves x 32 rows, two per SIMD;
//     key tiles of 64 keys stream through LDS in four stages (K: 16 KB, V: 16 KB per stage),
//     written by global_load_lds_dwordx4, two tiles per barrier: the next two are fetched while
//     the waves fold the current two, so the waves synchronise once per 128 keys. Each K/V tile
//     serves 256 queries, which halves the L2 -> LDS traffic of 128-query workgroups (4.3 GB
//     at config 4) and measured 0.609 against 0.631 ms;
//   * scores are computed transposed, S^T = K Q^T (v_mfma_f32_32x32x16_f16, the wave's Q
//     fragments stay in registers): lane l then holds 16 scores of query l % 32 per 32-key
//     tile, so the running max/denominator of a query live in one lane pair (l, l ^ 32);
//   * the output is accumulated transposed as well, O^T = V^T P^T: lane l holds dv values of
//     query l % 32, so the online-softmax rescale of O is lane-local and P goes from the
//     score registers to the MFMA B operand without leaving registers;
//   * V stays in its natural [key][dv] layout; the V^T operand is read with ds_read_b64_tr_b16
//     (in each 16-lane group, lane i receives element i % 4 of the 8-byte segments addressed by
//     lanes i / 4, 4 + i / 4, 8 + i / 4, 12 + i / 4), so no transpose passes through registers;
//   * each wave raises its priority (s_setprio 1) while it issues an MFMA loop, so of the two
//     waves on a SIMD the one with matrix work issues first and the other's exp and LDS work
//     fills the gaps (0.621 against 0.638 ms at config 4);
//   * the softmax scale is folded into one FMA per score. A chunk's maximum spans the lane pair
//     (l, l ^ 32), exchanged with v_permlane32_swap (a VALU op, no LDS round trip); the chunk's
//     P @ V runs one 32-dv block at a time from a zero accumulator and joins O with one FMA per
//     element (O is first scaled only when some query's maximum rises);
//   * causal: a workgroup visits key tiles up to its last query only, a wave skips tiles
//     beyond its own last query, and only tiles crossing the diagonal are masked; the
//     heaviest query blocks are dispatched first. All query blocks of one head share an
//     XCD (blocks of a head are 128 apart, a multiple of the 8 XCDs) and so its L2.
//
// The same kernel serves three modes: batched [B,H,S,D] tensors; packed sequences
// (flash_varlen_attention_fwd / flash_varlen_gqa_prefill, attention.py:839-924), where a
// workgroup's item names a sequence of rows in [U,H,D] tensors; and a per-key additive bias
// (flash_attention_bias_fwd, attention.py:800-836), whose 64 floats per tile are DMA'd beside K
// and V and enter each score as s (scale log2 e) + bias log2 e.
#include "common.hpp"

namespace intent_hip {
namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// Element type of q, k, v, o and of the rounded weights P: _Float16 (flash_attention_fwd,
// flash_gqa_attention_fwd) or __bf16 (flash_attention_bf16_fwd).
template <typename E> struct Elem;
template <> struct Elem<_Float16> {
  typedef _Float16 x8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x16_t mma(x8 a, x8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct Elem<__bf16> {
  typedef __bf16 x8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x16_t mma(x8 a, x8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <typename E>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, round_to<E>(lo))) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, round_to<E>(hi))) << 16);
}

constexpr int kBQ = 256;     // query rows per workgroup
constexpr int kBK = 64;      // keys per tile
constexpr int kThreads = 512;
constexpr float kLog2e = 1.4426950408889634f;

// LDS layouts of the K and V tiles: rows of D / 8 16-byte chunks, logical chunk c of row r stored
// at c ^ swz(r). D = 128: K rows at c ^ (r & 15), V rows at c ^ 4 (r & 3). D = 64 (two rows per
// 64-bank row): both at c ^ ((r >> 1) & 7) in the bit order below, a bijection of the 8 chunk
// slots over each 16 consecutive rows (the K fragment reads) that also sends the transposing V
// reads of 4 consecutive rows to 4 distinct chunk groups. Plain functions of d (constant after
// inlining), not templates: called as swz<D>(...) from the lambdas of the kernel template, hipcc
// (ROCm 7.2) compiled the device code but silently emitted no host stubs for the kernel, so the
// library failed to load with undefined kernel symbols.
__host__ __device__ __forceinline__ int swz_k(int d, int row) {
  if (d == 192) return (row >> 1) & 7;   // 24 chunks per row: the xor stays inside each group of 8
  return d == 128 ? (row & 15) : ((((row >> 1) & 1) << 2) | ((row >> 2) & 3));
}
__host__ __device__ __forceinline__ int swz_v(int d, int row) {
  return d == 128 ? 4 * (row & 3) : ((((row >> 1) & 1) << 2) | ((row >> 2) & 3));
}

__device__ __forceinline__ uint4 select(bool keep, uint4 v) {
  return make_uint4(keep ? v.x : 0u, keep ? v.y : 0u, keep ? v.z : 0u, keep ? v.w : 0u);
}

struct Geometry {
  int64_t qs[4], ks[4], vs[4], os[4];  // element strides (batch, head, row, col)
};

// Packed sequences (flash_varlen_attention_fwd, flash_varlen_gqa_prefill): rows cu[s] .. cu[s + 1]
// of q, k, v and the output belong to sequence s. Workgroup item * heads + h runs query head h of
// items[item] = (sequence, query block); attention_varlen_items writes the items on the device.
struct Ragged {
  const int32_t *cu;      // [sequences + 1] row offsets
  const int2 *items;      // [capacity]
  const int32_t *count;   // items written
  int total;              // rows of q, k, v and the output
};

// Per-key additive bias (flash_attention_bias_fwd): row (batch b, head h) at p + b bs + h hs, unit
// key stride; each tile's 64 floats are DMA'd beside its K and V.
struct KeyBias {
  const float *p;
  int64_t bs, hs;
};

// The position parts of latent attention (mla_prefill): query rows qpe [B,H,Q,P] at strides qs
// (batch, head, row) and key rows kpe [B,1,K,P], shared by every head, at strides ks (batch, row).
struct RopeRows {
  const uint16_t *qpe, *kpe;
  int64_t qs[3], ks[2];
};

// Key split for small grids: with count > 1, workgroup (item, split) folds its query block against
// the split-th share of the block's key tiles and writes each query row's unnormalised state
// (maximum in the exp2 domain, denominator, DV sums) at slot (split * rows + row) of m, den and
// acc, rows = batch * heads * sq; the sums are laid out [column / 8][slot][column % 8], so the 32
// rows of a wave store 1 KB contiguously per instruction. attention_split_merge combines the
// splits. Batched modes only. With `grouped`, workgroup x folds split x / items of item
// x % items (items = grid / count), else split x % count of item x / count.
struct KeySplit {
  int count;
  float *m, *den, *acc;
  int64_t rows;
  int grouped;
};

// Kernel modes: batched [B,H,S,D] tensors, packed sequences, batched with a key bias, or batched
// latent attention, whose score dimensions are the DV content dimensions of q and k followed by
// the position dimensions of qpe and kpe (D = DV + P).
constexpr int kBatched = 0, kPacked = 1, kBiased = 2, kLatent = 3;

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
typedef __attribute__((address_space(3))) void lds_void_t;

// s_waitcnt with only the vector-memory counter constrained (vmcnt <= n).
#define INTENT_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt((((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8)))

// How far a chunk maximum may exceed the reference maximum of the running O^T and denominator
// before they are rescaled to it (exp2 domain): chunk factors stay <= 2^8.
constexpr float kRefSlack = 8.0f;

// The values of lanes l % 32 (lo) and l % 32 + 32 (hi) of v, on every lane l: one
// v_permlane32_swap_b32 of two copies (it swaps the upper 32 lanes of its first operand with the
// lower 32 of its second). Inline assembly: hipcc's builtin for it returns both results from one
// register. The s_nop 1 on each side gives the two wait states the instruction needs after a VALU
// write of its operands, and before its results are read.
__device__ __forceinline__ void lane_halves(float v, float &lo, float &hi) {
  float a = v, b = v;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  lo = a;
  hi = b;
}

template <typename E, int D, int DV, int kMode>
__global__ __launch_bounds__(kThreads, 2) void attention_fwd(const uint16_t *__restrict__ Q,
                                                                  const uint16_t *__restrict__ K,
                                                                  const uint16_t *__restrict__ V,
                                                                  uint16_t *__restrict__ O, int heads,
                                                                  int head_group, int sq_all, int sk_all,
                                                                  Geometry g, float scale, int causal,
                                                                  int q_blocks, Ragged r, KeyBias kb, RopeRows rr,
                                                                  KeySplit split) {
  // Every rounding of the softmax and merge is the one written: no product is fused into a later
  // sum by the compiler (which it may otherwise do differently in different instantiations or
  // copies of the loop, e.g. a rescale acc *= left joined into the next fmaf).
#pragma clang fp contract(off)
  constexpr bool kVarlen = kMode == kPacked, kBias = kMode == kBiased, kRope = kMode == kLatent;
  typedef typename Elem<E>::x8 f16x8_t;   // operand fragments of 8 elements of E
  constexpr int kD = D, kDV = DV;
  constexpr int kKRow = kD / 8;               // 16-byte chunks per K row
  constexpr int kContent = kRope ? kDV / 8 : kKRow;   // chunks of a K row read from k (the rest: kpe)
  constexpr int kVRow = kDV / 8;              // 16-byte chunks per V row
  constexpr int kKChunks = kBK * kKRow;       // 16-byte chunks of a K tile (row = key)
  constexpr int kVChunks = kBK * kVRow;       // 16-byte chunks of a V tile (row = key)
  constexpr int kBiasChunks = kBias ? kBK / 4 : 0;   // 16-byte chunks of the tile's key bias
  constexpr int kStageChunks = kKChunks + kVChunks + kBiasChunks;
  // Key tiles per barrier: the waves synchronise once per kGroup tiles, with kGroup more in flight,
  // so 2 kGroup LDS stages. Two against one (interleaved, bit-identical): config 4 0.697 -> 0.690
  // ms, D = 64 at config 4's extents 0.427 -> 0.406 ms; four at D = 64 (eight 16 KB stages) lost
  // that gain again (0.418 ms).
  constexpr int kGroup = 2;
  constexpr int kStages = 2 * kGroup;
  static_assert(kStages * kStageChunks * 16 <= 160 * 1024, "LDS stages");
  static_assert(kKChunks % kThreads == 0 && kVChunks % kThreads == 0, "DMA split");
  __shared__ uint4 lds[kStages * kStageChunks];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform, kept in a scalar register
  int qb, b = 0, h, sq, sk;   // query block, batch entry, query head, rows of q and of k/v
  int part = 0;               // the key split this workgroup folds (batched modes)
  int64_t row0 = 0;           // first row of the sequence (packed sequences)
  if constexpr (kVarlen) {
    const int item = static_cast<int>(blockIdx.x) / heads;   // the heads of an item are neighbours
    h = static_cast<int>(blockIdx.x) % heads;
    if (item >= *r.count) return;                            // the grid covers the item capacity
    const int2 work = r.items[item];
    const int start = min(max(r.cu[work.x], 0), r.total);
    const int end = min(max(r.cu[work.x + 1], start), r.total);
    qb = work.y;
    sq = sk = end - start;
    row0 = start;
  } else {
    // With a key split the splits of one item are neighbours, or (grouped) `items` workgroups
    // apart: then, when items is a multiple of 8, on one XCD (dispatch goes round-robin over the 8
    // XCDs), where they share the item's query rows in L2. The launch groups only grids the device
    // holds at once, so the order changes no workgroup's start. Without a split, item = workgroup.
    const int items = gridDim.x / split.count;
    const int x = static_cast<int>(blockIdx.x);
    const int item = split.grouped ? x % items : x / split.count;
    part = split.grouped ? x / items : x % split.count;
    const int bh_count = items / q_blocks;
    qb = q_blocks - 1 - item / bh_count;   // heaviest blocks first
    const int bh = item % bh_count;
    b = bh / heads;
    h = bh % heads;
    sq = sq_all;
    sk = sk_all;
  }
  const uint16_t *qbase = Q + b * g.qs[0] + h * g.qs[1] + row0 * g.qs[2];
  const int kh = h / head_group;   // query head h reads key/value head h / head_group
  const uint16_t *kbase = K + b * g.ks[0] + kh * g.ks[1] + row0 * g.ks[2];
  const uint16_t *vbase = V + b * g.vs[0] + kh * g.vs[1] + row0 * g.vs[2];
  uint16_t *obase = O + b * g.os[0] + h * g.os[1] + row0 * g.os[2];
  const float *bias_row = kBias ? kb.p + b * kb.bs + h * kb.hs : nullptr;
  const uint16_t *qpe_base = kRope ? rr.qpe + b * rr.qs[0] + h * rr.qs[1] : nullptr;
  const uint16_t *kpe_base = kRope ? rr.kpe + b * rr.ks[0] : nullptr;

  const int q0 = qb * kBQ;
  const int wq0 = q0 + wave * 32;             // this wave's first query row
  const int lane_q = wq0 + (lane & 31);       // the query row this lane tracks
  const int half = lane >> 5;

  // Q fragments (MFMA B operand of S^T): q = lane_q, d = 16 ks + 8 half + 0..7.
  f16x8_t qf[kD / 16];
  {
    const bool ok = lane_q < sq;
    const uint16_t *row = qbase + static_cast<int64_t>(ok ? lane_q : 0) * g.qs[2];
    const uint16_t *pe_row = kRope ? qpe_base + static_cast<int64_t>(ok ? lane_q : 0) * rr.qs[2] : nullptr;
#pragma unroll
    for (int ks = 0; ks < kD / 16; ++ks) {
      const uint16_t *src = ks * 2 < kContent ? row + ks * 16 + half * 8 : pe_row + (ks * 16 - kContent * 8) + half * 8;
      qf[ks] = __builtin_bit_cast(f16x8_t, select(ok, *reinterpret_cast<const uint4 *>(src)));
    }
  }

  const int q_last_block = min(q0 + kBQ, sq) - 1;
  const int k_end = causal ? min(sk, q_last_block + 1) : sk;
  const int tiles_all = (k_end + kBK - 1) / kBK;
  // This workgroup's key tiles [t_begin, tiles): all of them, or its split's share.
  const int share = (tiles_all + split.count - 1) / split.count;
  const int t_begin = kVarlen ? 0 : min(tiles_all, part * share);
  const int tiles = kVarlen ? tiles_all : min(tiles_all, t_begin + share);
  const int wave_q_last = min(wq0 + 31, sq - 1);

  // DMA roles: each wave moves D / 32 x 64 chunks of K and DV / 32 x 64 chunks of V per tile.
  // LDS chunk slot p of a tile is row p / (row chunks) (a key), physical chunk p % (row chunks);
  // rows store logical chunk pc ^ swz(key). Keys beyond sk read row sk - 1 (finite data that the
  // mask zeroes out; V tail rows are cleared in LDS below).
  // Element offsets of this thread's chunks inside a full tile (key0 + row for every row): only
  // the tile's base, a wave-uniform scalar, changes from tile to tile. The last tile of a row that
  // ends inside it, and the latent mode (K chunks from two sources), take the clamped path below.
  // (The DMA builtin takes each source as a named pointer: given the sum `k_tile + k_off[i]`
  // directly, hipcc's host pass rejected the kernel template as a substitution failure.)
  int64_t k_off[kKChunks / kThreads], v_off[kVChunks / kThreads];
#pragma unroll
  for (int i = 0; i < kKChunks / kThreads; ++i) {
    const int p = (wave * (kKChunks / kThreads) + i) * 64 + lane;
    const int row = p / kKRow, pc = p % kKRow;
    k_off[i] = static_cast<int64_t>(row) * g.ks[2] + (pc ^ swz_k(D, row)) * 8;
  }
#pragma unroll
  for (int i = 0; i < kVChunks / kThreads; ++i) {
    const int p = (wave * (kVChunks / kThreads) + i) * 64 + lane;
    const int row = p / kVRow, pc = p % kVRow;
    v_off[i] = static_cast<int64_t>(row) * g.vs[2] + (pc ^ swz_v(DV, row)) * 8;
  }
  auto issue = [&](int kt) {
    uint4 *stage = lds + (kt & (kStages - 1)) * kStageChunks;
    const int key0 = kt * kBK;
    if (!kRope && key0 + kBK <= sk) {   // wave-uniform: a full tile
      const uint16_t *k_tile = kbase + static_cast<int64_t>(key0) * g.ks[2];
      const uint16_t *v_tile = vbase + static_cast<int64_t>(key0) * g.vs[2];
#pragma unroll
      for (int i = 0; i < kKChunks / kThreads; ++i)
      {
        const uint16_t *src = k_tile + k_off[i];
        __builtin_amdgcn_global_load_lds(src, (lds_void_t *)(stage + (wave * (kKChunks / kThreads) + i) * 64), 16, 0,
                                         0);
      }
#pragma unroll
      for (int i = 0; i < kVChunks / kThreads; ++i)
      {
        const uint16_t *src = v_tile + v_off[i];
        __builtin_amdgcn_global_load_lds(src, (lds_void_t *)(stage + kKChunks + (wave * (kVChunks / kThreads) + i) * 64),
                                         16, 0, 0);
      }
      if constexpr (kBias) {   // wave 0, one key per lane
        if (wave == 0)
          __builtin_amdgcn_global_load_lds(bias_row + key0 + lane, (lds_void_t *)(stage + kKChunks + kVChunks), 4, 0,
                                           0);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < kKChunks / kThreads; ++i) {
      const int p = (wave * (kKChunks / kThreads) + i) * 64 + lane;
      const int row = p / kKRow, pc = p % kKRow;
      const int key = min(key0 + row, sk - 1);
      const int lc = pc ^ swz_k(D, row);   // the logical chunk this slot holds
      const uint16_t *src = kbase + static_cast<int64_t>(key) * g.ks[2] + lc * 8;
      if constexpr (kRope)
        if (lc >= kContent) src = kpe_base + static_cast<int64_t>(key) * rr.ks[1] + (lc - kContent) * 8;
      __builtin_amdgcn_global_load_lds(src, (lds_void_t *)(stage + (wave * (kKChunks / kThreads) + i) * 64), 16, 0,
                                       0);
    }
#pragma unroll
    for (int i = 0; i < kVChunks / kThreads; ++i) {
      const int p = (wave * (kVChunks / kThreads) + i) * 64 + lane;
      const int row = p / kVRow, pc = p % kVRow;
      const int key = min(key0 + row, sk - 1);
      __builtin_amdgcn_global_load_lds(vbase + static_cast<int64_t>(key) * g.vs[2] + (pc ^ swz_v(DV, row)) * 8,
                                       (lds_void_t *)(stage + kKChunks + (wave * (kVChunks / kThreads) + i) * 64), 16,
                                       0, 0);
    }
    if constexpr (kBias) {   // wave 0, one key per lane (past the row's end, its last key: masked below)
      if (wave == 0)
        __builtin_amdgcn_global_load_lds(bias_row + min(key0 + lane, sk - 1),
                                         (lds_void_t *)(stage + kKChunks + kVChunks), 4, 0, 0);
    }
  };

  f32x16_t acc[kDV / 32];   // O^T: dv tile mt (32 dv) x 32 queries
#pragma unroll
  for (int mt = 0; mt < kDV / 32; ++mt)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[mt][e] = 0.0f;
  // Running summary of this lane's query (merge_attention_summaries' record): validity, and the
  // denominator (the same on both lanes of the pair) and O^T against the reference maximum row_ref,
  // which stays within kRefSlack below the running maximum of valid scaled scores (exp2 domain).
  bool row_valid = false;
  float row_ref = 0.0f;   // reference maximum of row_den and acc (see the merge below)
  float row_den = 0.0f;
  const float factor = scale * kLog2e;
  const int frag_row = lane & 31;
  // V^T transposed-read roles: group g16 = lane / 16, source index i16 = lane % 16.
  const int g16 = lane >> 4, i16 = lane & 15;
  const int v_key = 4 * (g16 >> 1) + (i16 >> 2);      // + 16 sl + 8 r
  const int v_dv = 16 * (g16 & 1) + 4 * (i16 & 3);    // + 32 mt

  for (int i = 0; i < kGroup && t_begin + i < tiles; ++i) issue(t_begin + i);
  for (int kt = t_begin; kt < tiles; ++kt) {
    if ((kt - t_begin) % kGroup == 0) {   // workgroup-uniform
      INTENT_WAIT_VMCNT(0);
      __syncthreads();   // tiles kt .. kt + kGroup - 1 are in LDS; every wave is done with the group before
      for (int i = 0; i < kGroup; ++i)
        if (kt + kGroup + i < tiles) issue(kt + kGroup + i);   // into the stages of the group before
    }
    const int key0 = kt * kBK;
    const uint4 *sk_tile = lds + (kt & (kStages - 1)) * kStageChunks;
    const uint16_t *sv_tile = reinterpret_cast<const uint16_t *>(sk_tile + kKChunks);
    if (key0 + kBK > sk) {
      // Tail tile: clear the V rows past the last key so masked weights meet zeros.
      uint4 *vt = const_cast<uint4 *>(sk_tile + kKChunks);
      for (int c = tid; c < kVChunks; c += kThreads)
        if (key0 + c / kVRow >= sk) vt[c] = make_uint4(0, 0, 0, 0);
      __syncthreads();
    }
    const bool active = !causal || key0 <= wave_q_last;      // wave-uniform
    if (!active || wq0 >= sq) continue;
    // S^T for two 32-key tiles: s[st][e] is key 8 (e / 4) + 4 half + e % 4 of tile st. The K
    // fragments of step ks + 1 are read while the two MFMAs of step ks run.
    f32x16_t s[2];
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 16; ++e) s[st][e] = 0.0f;
    {
      f16x8_t kf[2][2];
      auto read_k = [&](int ks, int buf) {
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const int row = st * 32 + frag_row;
          kf[buf][st] = __builtin_bit_cast(f16x8_t, sk_tile[row * kKRow + ((ks * 2 + half) ^ swz_k(D, row))]);
        }
      };
      read_k(0, 0);
      __builtin_amdgcn_iglp_opt(0);   // hipcc's DS/MFMA interleave for the loop below
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int ks = 0; ks < kD / 16; ++ks) {
        if (ks + 1 < kD / 16) read_k(ks + 1, (ks + 1) & 1);
#pragma unroll
        for (int st = 0; st < 2; ++st)
          s[st] = Elem<E>::mma(kf[ks & 1][st], qf[ks], s[st]);
      }
      __builtin_amdgcn_s_setprio(0);
    }
    // With a key bias the scores become (s scale + bias) log2 e here, as one FMA each; lane keys
    // 8 j + 4 half + 0..3 of each 32-key tile are one 16-byte LDS read.
    if constexpr (kBias) {
      const float *sbias = reinterpret_cast<const float *>(sk_tile + kKChunks + kVChunks);
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float4 b4 = *reinterpret_cast<const float4 *>(sbias + st * 32 + 8 * j + 4 * half);
          s[st][4 * j] = fmaf(s[st][4 * j], factor, b4.x * kLog2e);
          s[st][4 * j + 1] = fmaf(s[st][4 * j + 1], factor, b4.y * kLog2e);
          s[st][4 * j + 2] = fmaf(s[st][4 * j + 2], factor, b4.z * kLog2e);
          s[st][4 * j + 3] = fmaf(s[st][4 * j + 3], factor, b4.w * kLog2e);
        }
    }
    // Mask (only tiles that cross the diagonal or the end) and the chunk maximum of raw scores
    // (scale * log2 e > 0, so the maximum commutes with the scaling, rounding included; biased
    // scores are final).
    const bool edge = causal ? (key0 + kBK - 1 > wq0) : false;
    const bool partial = edge || key0 + kBK > sk;               // wave-uniform
    if (partial) {
      const int limit = causal ? min(sk - 1, lane_q) : sk - 1;  // last valid key of this lane's query
      // Key key0 + 4 half + o of element (st, e), o = 32 st + 8 (e / 4) + e % 4 an immediate: one
      // compare against the lane's room per element.
      const int room = limit - key0 - 4 * half;
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          s[st][e] = st * 32 + 8 * (e >> 2) + (e & 3) <= room ? s[st][e] : -INFINITY;
    }
    // This lane's 32 keys in four independent chains (maximum_num: NaN-ignoring, exact, any order),
    // then the other half's from lane l ^ 32.
    float part[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 16; ++e) part[e & 3] = fmaxf(part[e & 3], s[st][e]);
    float max_lo, max_hi;
    lane_halves(fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3])), max_lo, max_hi);
    // The chunk summary (summarize_attention_chunk_*): weights against the chunk maximum, 0 at
    // masked keys. Every chunk this wave visits holds a valid key for each of its queries (tiles
    // start at multiples of 64 keys and waves at multiples of 32 queries, and a wave visits tile key0
    // only when key0 <= its last query, hence key0 <= its first; without the causal mask, key0 < sk),
    // so the summarizer's empty-chunk case (maximum 0, accumulator selected to 0) never arises here.
    // A masked key's score is -inf, so its weight exp2(-inf - max) is 0 for a finite or +inf chunk
    // maximum, without a select. With a -inf or NaN chunk maximum (only from infinite or NaN
    // inputs) the chunk's valid weights are NaN as the summarizer's are, and so is the row's output
    // whatever the masked keys' weights.
    const float chunk_max = fmaxf(max_lo, max_hi) * (kBias ? 1.0f : factor);
    f16x8_t pf[4];   // P^T fragments: slice sl = 2 st + (e / 8), slot j = e % 8
    float den_part = 0.0f;
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float p = __builtin_amdgcn_exp2f(kBias ? s[st][e] - chunk_max : fmaf(s[st][e], factor, -chunk_max));
        den_part += p;
        pf[st * 2 + (e >> 3)][e & 7] = static_cast<E>(p);
      }
    float den_lo, den_hi;
    lane_halves(den_part, den_lo, den_hi);
    // Merge (running summary, chunk), merge_attention_summaries' algebra: O^T and the denominator are
    // kept against a reference maximum `row_ref` instead of the running maximum itself, and the
    // chunk joins with the factor exp2(chunk max - row_ref). The reference rises to the running
    // maximum only when a chunk maximum exceeds it by more than kRefSlack, so the factors stay
    // <= 2^kRefSlack and O^T is rescaled (exp2(old - new) on both, as the merge's left factor) only
    // then. Normalisation divides out the common factor exp2(running maximum - row_ref). The weights
    // P above are rounded against the chunk's own maximum either way: the reference only moves the
    // f32 products of the merge, not where the 16-bit rounding happens.
    // A chunk maximum above row_ref + kRefSlack is above the running maximum too (that never rose
    // more than kRefSlack above row_ref without a rescale), so it is the new running maximum.
    if (__any(!row_valid || chunk_max > row_ref + kRefSlack)) {   // wave-uniform, rare
      const float ref = !row_valid || chunk_max > row_ref + kRefSlack ? chunk_max : row_ref;
      const float left = row_valid ? __builtin_amdgcn_exp2f(row_ref - ref) : 0.0f;
      row_ref = ref;
      row_den *= left;
#pragma unroll
      for (int mt = 0; mt < kDV / 32; ++mt)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[mt][e] *= left;
    }
    row_valid = true;
    const float right = __builtin_amdgcn_exp2f(chunk_max - row_ref);
    row_den = fmaf(right, den_lo + den_hi, row_den);
    // The chunk's O^T = V^T P^T, one 32-dv tile at a time from zero, joined as acc + right * chunk.
    // The A operand (V^T rows dv, keys in slot order) comes from V's natural [key][dv] layout through
    // ds_read_b64_tr_b16: read r of slice sl gives the lane keys 16 sl + 8 r + 4 half + 0..3 of its
    // dv. Steps q = 4 mt + sl run over the dv tiles and key slices; fragment q lives in vf[q % 4] and
    // is read two steps before its MFMA.
    {
      constexpr int kSteps = kDV / 32 * 4;
      f16x8_t vf[4];
      auto read_v = [&](int q) {
        const int mt = q >> 2, sl = q & 3;
        i16x4_t parts[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int key = sl * 16 + 8 * r + v_key;
          const int dv = mt * 32 + v_dv;
          const int chunk = (dv >> 3) ^ swz_v(DV, key);
          parts[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(sv_tile + key * kDV + chunk * 8 + (dv & 7)));
        }
        vf[q & 3] = __builtin_bit_cast(f16x8_t, parts);
      };
      read_v(0);
      read_v(1);
      __builtin_amdgcn_iglp_opt(0);
      __builtin_amdgcn_s_setprio(1);
      f32x16_t chunk_acc;
#pragma unroll
      for (int q = 0; q < kSteps; ++q) {
        if (q + 2 < kSteps) read_v(q + 2);
        const int mt = q >> 2, sl = q & 3;
        chunk_acc = Elem<E>::mma(vf[q & 3], pf[sl], sl == 0 ? f32x16_t{} : chunk_acc);
        if (sl == 3)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[mt][e] = fmaf(right, chunk_acc[e], acc[mt][e]);
      }
      __builtin_amdgcn_s_setprio(0);
    }
  }

  // Normalise and store: acc[mt][4 gq + e] is dv = 32 mt + 8 gq + 4 half + e of query lane_q.
  if (lane_q >= sq) return;
  const float den = row_den;
  if (!kVarlen && split.count > 1) {
    // This split's state, unnormalised: the denominator and O^T with the maximum they are taken
    // against (row_ref; -inf for a split with no key), which is what attention_split_merge's exp2
    // factors need.
    const int64_t slot = static_cast<int64_t>(part) * split.rows +
                         (static_cast<int64_t>(b) * heads + h) * sq + lane_q;
    if (half == 0) {
      split.m[slot] = row_valid ? row_ref : -INFINITY;
      split.den[slot] = den;
    }
    // The sums of a row with no key in this split are never read (the merge skips a split whose
    // maximum is -inf), so they are not written.
    if (!row_valid) return;
    const int64_t slots = split.count * split.rows;
    float *arow = split.acc + slot * 8 + 4 * half;
#pragma unroll
    for (int mt = 0; mt < kDV / 32; ++mt)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq)
        *reinterpret_cast<float4 *>(arow + (mt * 4 + gq) * slots * 8) =
            make_float4(acc[mt][4 * gq], acc[mt][4 * gq + 1], acc[mt][4 * gq + 2], acc[mt][4 * gq + 3]);
    return;
  }
  const bool valid = row_valid;
  const float inv = valid ? __builtin_amdgcn_rcpf(den) : 0.0f;
  uint16_t *orow = obase + static_cast<int64_t>(lane_q) * g.os[2];
#pragma unroll
  for (int mt = 0; mt < kDV / 32; ++mt)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const uint32_t w0 = pack2<E>(acc[mt][4 * gq] * inv, acc[mt][4 * gq + 1] * inv);
      const uint32_t w1 = pack2<E>(acc[mt][4 * gq + 2] * inv, acc[mt][4 * gq + 3] * inv);
      *reinterpret_cast<uint2 *>(orow + mt * 32 + 8 * gq + 4 * half) = make_uint2(w0, w1);
    }
}

// Items of the packed sequences, one workgroup: sequence s has ceil(rows / kBQ) query blocks, listed
// from the last (the most keys under a causal mask) to the first, sequence after sequence. Offsets
// are clamped into [0, total] and the list into its capacity, so no offsets can send a later
// workgroup out of bounds.
__global__ __launch_bounds__(1024) void attention_varlen_items(const int32_t *__restrict__ cu, int sequences,
                                                               int total, int2 *__restrict__ items,
                                                               int32_t *__restrict__ count, int capacity) {
  __shared__ int s_wave[16];
  __shared__ int s_carry;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid == 0) s_carry = 0;
  __syncthreads();
  for (int s0 = 0; s0 < sequences; s0 += 1024) {
    const int s = s0 + tid;
    int blocks = 0;
    if (s < sequences) {
      const int start = min(max(cu[s], 0), total);
      const int end = min(max(cu[s + 1], start), total);
      blocks = (end - start + kBQ - 1) / kBQ;
    }
    int incl = blocks;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int up = __shfl_up(incl, d);
      incl += lane >= d ? up : 0;
    }
    if (lane == 63) s_wave[wave] = incl;
    __syncthreads();
    int first = s_carry + incl - blocks;
    for (int w = 0; w < wave; ++w) first += s_wave[w];
    for (int j = 0; j < blocks; ++j)
      if (first + j < capacity) items[first + j] = make_int2(s, blocks - 1 - j);
    __syncthreads();
    if (tid == 0) {
      int sum = s_carry;
      for (int w = 0; w < 16; ++w) sum += s_wave[w];
      s_carry = sum;
    }
    __syncthreads();
  }
  if (tid == 0) *count = min(s_carry, capacity);
}

}  // namespace

// Key splits per query block: at most kMaxKeySplits (key_splits below).
constexpr int kMaxKeySplits = 8;

// The key splits of one query row merged as merge_attention_summaries does (exp2 factors against
// the largest maximum), normalised by an approximate reciprocal and stored in the element type E;
// a row with no admitted key in any split is 0. One thread per row and 8-column block, threads in
// the order of the sums' layout ([column / 8][row][column % 8] within each split), so a wave reads
// 2 KB of every split contiguously. The splits are unrolled (at most kMaxKeySplits): the maxima
// are loaded first (indices clamped, the splits past `splits` masked), then the denominator and
// sums of each split that holds a key for the row.
template <typename E, int DV>
__global__ __launch_bounds__(256) void attention_split_merge(const float *__restrict__ m, const float *__restrict__ den,
                                                             const float *__restrict__ acc, int splits, int64_t rows,
                                                             int heads, int sq, uint16_t *__restrict__ O, int64_t os_b,
                                                             int64_t os_h, int64_t os_q) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= rows * (DV / 8)) return;
  const int64_t row = t % rows, block = t / rows;
  const float *a = acc + (block * splits * rows + row) * 8;   // split s at + s * rows * 8
  float ms[kMaxKeySplits];
  float top = -INFINITY;
#pragma unroll
  for (int s = 0; s < kMaxKeySplits; ++s) {
    const float v = m[min(s, splits - 1) * rows + row];
    ms[s] = s < splits ? v : -INFINITY;
    top = fmaxf(top, ms[s]);
  }
  const bool valid = top != -INFINITY;
  float total = 0.0f;
  float4 lo = make_float4(0.0f, 0.0f, 0.0f, 0.0f), hi = lo;
#pragma unroll
  for (int s = 0; s < kMaxKeySplits; ++s) {
    // A split with no key for this row (maximum -inf) adds nothing; its sums were not written.
    if (s < splits && ms[s] != -INFINITY) {
      const int64_t at = s * rows;
      const float d = den[at + row];
      const float4 v0 = *reinterpret_cast<const float4 *>(a + at * 8);
      const float4 v1 = *reinterpret_cast<const float4 *>(a + at * 8 + 4);
      const float f = __builtin_amdgcn_exp2f(ms[s] - top);
      total = fmaf(f, d, total);
      lo = make_float4(fmaf(f, v0.x, lo.x), fmaf(f, v0.y, lo.y), fmaf(f, v0.z, lo.z), fmaf(f, v0.w, lo.w));
      hi = make_float4(fmaf(f, v1.x, hi.x), fmaf(f, v1.y, hi.y), fmaf(f, v1.z, hi.z), fmaf(f, v1.w, hi.w));
    }
  }
  const float inv = valid ? __builtin_amdgcn_rcpf(total) : 0.0f;
  const int64_t q = row % sq, bh = row / sq;
  uint16_t *orow = O + (bh / heads) * os_b + (bh % heads) * os_h + q * os_q + block * 8;
  auto pack = [&](float x, float y) {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, round_to<E>(x * inv))) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, round_to<E>(y * inv))) << 16);
  };
  reinterpret_cast<uint2 *>(orow)[0] = make_uint2(pack(lo.x, lo.y), pack(lo.z, lo.w));
  reinterpret_cast<uint2 *>(orow)[1] = make_uint2(pack(hi.x, hi.y), pack(hi.z, hi.w));
}

// The kernel of a (dtype, d, dv, mode) choice; d and dv are each 64 or 128 (checked by the callers).
template <typename E, int kMode>
const void *attention_kernel(int64_t d, int64_t dv) {
  if (d == 64) return dv == 64 ? reinterpret_cast<const void *>(&attention_fwd<E, 64, 64, kMode>)
                               : reinterpret_cast<const void *>(&attention_fwd<E, 64, 128, kMode>);
  return dv == 64 ? reinterpret_cast<const void *>(&attention_fwd<E, 128, 64, kMode>)
                  : reinterpret_cast<const void *>(&attention_fwd<E, 128, 128, kMode>);
}

int attention_resources(int dtype, int64_t sq, int64_t d, int64_t dv, int mode, IntentHipKernelResources *out) {
  (void)sq;
  if (mode == kLatent) {   // d: content dimensions (= dv), dv: position dimensions
    if ((d != 64 && d != 128) || dv != 64)
      return fail(INTENT_HIP_ERR_UNSUPPORTED, "latent attention takes D in {64, 128} and P = 64");
    return describe_kernel(d == 128 ? reinterpret_cast<const void *>(&attention_fwd<_Float16, 192, 128, kLatent>)
                                    : reinterpret_cast<const void *>(&attention_fwd<_Float16, 128, 64, kLatent>),
                           d == 128 ? "attention_fwd<f16,192,128,latent>" : "attention_fwd<f16,128,64,latent>",
                           kThreads, out);
  }
  if ((d != 64 && d != 128) || (dv != 64 && dv != 128))
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "attention kernels take d, dv in {64, 128}");
  char name[64];
  snprintf(name, sizeof name, "attention_fwd<%s,%d,%d%s>", dtype == INTENT_HIP_BF16 ? "bf16" : "f16",
           static_cast<int>(d), static_cast<int>(dv), mode == kPacked ? ",packed" : mode == kBiased ? ",bias" : "");
  const void *kernel;
  if (mode == kBiased)
    kernel = attention_kernel<_Float16, kBiased>(d, dv);
  else if (dtype == INTENT_HIP_BF16)
    kernel = mode == kPacked ? attention_kernel<__bf16, kPacked>(d, dv) : attention_kernel<__bf16, kBatched>(d, dv);
  else
    kernel = mode == kPacked ? attention_kernel<_Float16, kPacked>(d, dv) : attention_kernel<_Float16, kBatched>(d, dv);
  return describe_kernel(kernel, name, kThreads, out);
}

}  // namespace intent_hip

using namespace intent_hip;

namespace {

template <typename E, int D, int DV, int kMode>
void launch_fwd(dim3 grid, hipStream_t s, const uint16_t *Q, const uint16_t *K, const uint16_t *V, uint16_t *O,
                int heads, int head_group, int sq, int sk, const Geometry &g, float scale, int causal, int q_blocks,
                const Ragged &r, const KeyBias &kb, const RopeRows &rr = RopeRows{},
                const KeySplit &split = KeySplit{1, nullptr, nullptr, nullptr}) {
  attention_fwd<E, D, DV, kMode><<<grid, dim3(kThreads), 0, s>>>(Q, K, V, O, heads, head_group, sq, sk, g, scale,
                                                                 causal, q_blocks, r, kb, rr, split);
}

// One launch of the (dtype, d, dv) instantiation.
template <int kMode>
void launch_variant(int dtype, int64_t d, int64_t dv, dim3 grid, hipStream_t s, const uint16_t *Q, const uint16_t *K,
                    const uint16_t *V, uint16_t *O, int heads, int head_group, int sq, int sk, const Geometry &g,
                    float scale, int causal, int q_blocks, const Ragged &r,
                    const KeyBias &kb = KeyBias{}, const KeySplit &ks = KeySplit{1, nullptr, nullptr, nullptr}) {
  if (kMode != kBiased && dtype == INTENT_HIP_BF16) {
    if (d == 64)
      dv == 64 ? launch_fwd<__bf16, 64, 64, kMode>(grid, s, Q, K, V, O, heads, head_group, sq, sk, g, scale, causal, q_blocks, r, kb, RopeRows{}, ks)
               : launch_fwd<__bf16, 64, 128, kMode>(grid, s, Q, K, V, O, heads, head_group, sq, sk, g, scale, causal, q_blocks, r, kb, RopeRows{}, ks);
    else
      dv == 64 ? launch_fwd<__bf16, 128, 64, kMode>(grid, s, Q, K, V, O, heads, head_group, sq, sk, g, scale, causal, q_blocks, r, kb, RopeRows{}, ks)
               : launch_fwd<__bf16, 128, 128, kMode>(grid, s, Q, K, V, O, heads, head_group, sq, sk, g, scale, causal, q_blocks, r, kb, RopeRows{}, ks);
  } else {
    if (d == 64)
      dv == 64 ? launch_fwd<_Float16, 64, 64, kMode>(grid, s, Q, K, V, O, heads, head_group, sq, sk, g, scale, causal, q_blocks, r, kb, RopeRows{}, ks)
               : launch_fwd<_Float16, 64, 128, kMode>(grid, s, Q, K, V, O, heads, head_group, sq, sk, g, scale, causal, q_blocks, r, kb, RopeRows{}, ks);
    else
      dv == 64 ? launch_fwd<_Float16, 128, 64, kMode>(grid, s, Q, K, V, O, heads, head_group, sq, sk, g, scale, causal, q_blocks, r, kb, RopeRows{}, ks)
               : launch_fwd<_Float16, 128, 128, kMode>(grid, s, Q, K, V, O, heads, head_group, sq, sk, g, scale, causal, q_blocks, r, kb, RopeRows{}, ks);
  }
}

// Key splits for a grid of `blocks` workgroups: 1 when the grid fills the 256 CUs or the keys are
// fewer than 8 tiles, else enough to reach about 512 workgroups, at most 8 and at most half the key
// tiles (two tiles per split). With fewer tiles the merge launch costs more than the split saves
// (the reference streaming example, 4 tiles: 14.8 us split in two against 13.2 us unsplit).
int64_t key_splits(int64_t blocks, int64_t sk) {
  const int64_t tiles = (sk + kBK - 1) / kBK;
  if (blocks <= 0 || blocks >= 256 || tiles < 8) return 1;
  int64_t s = (512 + blocks - 1) / blocks;
  s = s > kMaxKeySplits ? kMaxKeySplits : s;
  s = s > tiles / 2 ? tiles / 2 : s;
  return s < 1 ? 1 : s;
}

// Split state: maxima and denominators (each from a 256-byte boundary), then the sums.
struct SplitLayout {
  int64_t splits, rows;
  size_t den, acc, bytes;
};
SplitLayout split_layout(int64_t batch, int64_t heads, int64_t sq, int64_t sk, int64_t dv) {
  const int64_t q_blocks = (sq + kBQ - 1) / kBQ;
  const int64_t splits = key_splits(batch * heads * q_blocks, sk);
  if (splits == 1) return SplitLayout{1, 0, 0, 0, 0};
  const size_t n = static_cast<size_t>(batch * heads * sq * splits);
  const size_t part = (4 * n + 255) / 256 * 256;
  return SplitLayout{splits, batch * heads * sq, part, 2 * part, 2 * part + 4 * n * static_cast<size_t>(dv)};
}

// The split state of a launch, when the grid is small enough to split and the workspace holds it
// (256-byte aligned); else a single split.
KeySplit key_split(const SplitLayout &layout, void *workspace, size_t workspace_bytes) {
  if (layout.splits <= 1 || workspace == nullptr || workspace_bytes < layout.bytes || !aligned(workspace, 256))
    return KeySplit{1, nullptr, nullptr, nullptr};
  char *ws = static_cast<char *>(workspace);
  return KeySplit{static_cast<int>(layout.splits), reinterpret_cast<float *>(ws),
                  reinterpret_cast<float *>(ws + layout.den), reinterpret_cast<float *>(ws + layout.acc), layout.rows};
}

// attention_split_merge<E, dv> over every query row of a split launch.
void launch_merge(int dtype, int64_t dv, const KeySplit &ks, int heads, int sq, uint16_t *O, const Geometry &g,
                  hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((ks.rows * (dv / 8) + 255) / 256)), block(256);
  if (dtype == INTENT_HIP_BF16) {
    if (dv == 128)
      attention_split_merge<__bf16, 128><<<grid, block, 0, s>>>(ks.m, ks.den, ks.acc, ks.count, ks.rows, heads, sq, O,
                                                                g.os[0], g.os[1], g.os[2]);
    else
      attention_split_merge<__bf16, 64><<<grid, block, 0, s>>>(ks.m, ks.den, ks.acc, ks.count, ks.rows, heads, sq, O,
                                                               g.os[0], g.os[1], g.os[2]);
  } else {
    if (dv == 128)
      attention_split_merge<_Float16, 128><<<grid, block, 0, s>>>(ks.m, ks.den, ks.acc, ks.count, ks.rows, heads, sq,
                                                                  O, g.os[0], g.os[1], g.os[2]);
    else
      attention_split_merge<_Float16, 64><<<grid, block, 0, s>>>(ks.m, ks.den, ks.acc, ks.count, ks.rows, heads, sq,
                                                                 O, g.os[0], g.os[1], g.os[2]);
  }
}

// Batched attention; with kb, the key-biased form (f16, non-causal). A workspace of
// split_layout(...).bytes lets a small batched grid split its keys (merged by a second launch).
int launch_attention(int dtype, const void *q, const void *k, const void *v, void *o, int64_t batch, int64_t heads,
                     int64_t head_group, int64_t sq, int64_t sk, int64_t d, int64_t dv, const int64_t *strides,
                     float scale, int causal, void *stream, const KeyBias *kb = nullptr, void *workspace = nullptr,
                     size_t workspace_bytes = 0) {
  if (batch < 0 || heads < 0 || sq < 0 || sk < 0 || d < 0 || dv < 0)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (head_group < 1 || (heads > 0 && heads % head_group != 0))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "head_group %lld must be positive and divide the %lld query heads",
                static_cast<long long>(head_group), static_cast<long long>(heads));
  if (dtype != INTENT_HIP_F16 && dtype != INTENT_HIP_BF16)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "attention dtype code %d (1 = f16, 2 = bf16)", dtype);
  if (batch == 0 || heads == 0 || sq == 0 || dv == 0) return INTENT_HIP_OK;
  if ((d != 64 && d != 128) || (dv != 64 && dv != 128))
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "attention kernels take D and DV in {64, 128} (got d=%lld, dv=%lld)",
                static_cast<long long>(d), static_cast<long long>(dv));
  if (strides == nullptr || q == nullptr || o == nullptr || (sk > 0 && (k == nullptr || v == nullptr)))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null pointer");
  if (sq > INT32_MAX / 2 || sk > INT32_MAX / 2 || batch * heads > INT32_MAX / 64)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "attention extents too large for one launch");
  Geometry g;
  for (int i = 0; i < 4; ++i) {
    g.qs[i] = strides[i];
    g.ks[i] = strides[4 + i];
    g.vs[i] = strides[8 + i];
    g.os[i] = strides[12 + i];
  }
  if (g.qs[3] != 1 || g.ks[3] != 1 || g.vs[3] != 1 || g.os[3] != 1)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "attention tensors need unit inner stride");
  for (int i = 0; i < 3; ++i)
    if (g.qs[i] % 8 || g.ks[i] % 8 || g.vs[i] % 8 || g.os[i] % 4)
      return fail(INTENT_HIP_ERR_UNSUPPORTED, "attention strides must be multiples of 8 elements");
  if (!aligned(q, 16) || (sk > 0 && (!aligned(k, 16) || !aligned(v, 16))) || !aligned(o, 8))
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "attention tensors must be 16-byte aligned");
  const int q_blocks = static_cast<int>((sq + kBQ - 1) / kBQ);
  KeySplit ks = kb == nullptr ? key_split(split_layout(batch, heads, sq, sk, dv), workspace, workspace_bytes)
                              : KeySplit{1, nullptr, nullptr, nullptr};
  const int64_t blocks = batch * heads * q_blocks * ks.count;
  if (blocks > INT32_MAX) return fail(INTENT_HIP_ERR_UNSUPPORTED, "too many attention workgroups");
  ks.grouped = ks.count > 1 && blocks <= device_cus();
  const auto *Qp = static_cast<const uint16_t *>(q);
  const auto *Kp = static_cast<const uint16_t *>(k);
  const auto *Vp = static_cast<const uint16_t *>(v);
  auto *Op = static_cast<uint16_t *>(o);
  const dim3 grid(static_cast<unsigned>(blocks));
  const hipStream_t s = as_stream(stream);
  const int h = static_cast<int>(heads), grp = static_cast<int>(head_group);
  const int iq = static_cast<int>(sq), ik = static_cast<int>(sk), c = causal ? 1 : 0;
  if (kb != nullptr)
    launch_variant<kBiased>(dtype, d, dv, grid, s, Qp, Kp, Vp, Op, h, grp, iq, ik, g, scale, c, q_blocks, Ragged{}, *kb);
  else
    launch_variant<kBatched>(dtype, d, dv, grid, s, Qp, Kp, Vp, Op, h, grp, iq, ik, g, scale, c, q_blocks, Ragged{},
                             KeyBias{}, ks);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("attention_fwd");
  if (ks.count > 1) {
    launch_merge(dtype, dv, ks, h, iq, Op, g, s);
    if (hipPeekAtLastError() != hipSuccess) return launch_status("attention_split_merge");
  }
  return INTENT_HIP_OK;
}

}  // namespace

extern "C" int intent_hip_attention_fwd_f16(const void *q, const void *k, const void *v, void *o, int64_t batch,
                                            int64_t heads, int64_t sq, int64_t sk, int64_t d, int64_t dv,
                                            const int64_t *strides, float scale, int causal, void *stream) {
  return launch_attention(INTENT_HIP_F16, q, k, v, o, batch, heads, 1, sq, sk, d, dv, strides, scale, causal, stream);
}

extern "C" int intent_hip_attention_fwd(int dtype, const void *q, const void *k, const void *v, void *o,
                                        int64_t batch, int64_t q_heads, int64_t head_group, int64_t sq, int64_t sk,
                                        int64_t d, int64_t dv, const int64_t *strides, float scale, int causal,
                                        void *stream) {
  return launch_attention(dtype, q, k, v, o, batch, q_heads, head_group, sq, sk, d, dv, strides, scale, causal,
                          stream);
}

extern "C" int intent_hip_attention_fwd_workspace_bytes(int64_t batch, int64_t q_heads, int64_t sq, int64_t sk,
                                                        int64_t dv, size_t *bytes) {
  if (bytes == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null output");
  if (batch < 0 || q_heads < 0 || sq < 0 || sk < 0 || dv < 0)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  *bytes = split_layout(batch, q_heads, sq, sk, dv).bytes;
  return INTENT_HIP_OK;
}

extern "C" int intent_hip_attention_fwd_ws(int dtype, const void *q, const void *k, const void *v, void *o,
                                           int64_t batch, int64_t q_heads, int64_t head_group, int64_t sq,
                                           int64_t sk, int64_t d, int64_t dv, const int64_t *strides, float scale,
                                           int causal, void *workspace, size_t workspace_bytes, void *stream) {
  return launch_attention(dtype, q, k, v, o, batch, q_heads, head_group, sq, sk, d, dv, strides, scale, causal,
                          stream, nullptr, workspace, workspace_bytes);
}

extern "C" int intent_hip_attention_bias_fwd(const void *q, const void *k, const void *v, const float *bias, void *o,
                                             int64_t batch, int64_t heads, int64_t sq, int64_t sk, int64_t d,
                                             int64_t dv, const int64_t *strides, const int64_t *bias_strides,
                                             float scale, void *stream) {
  if (bias_strides == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null pointer");
  if (batch > 0 && heads > 0 && sq > 0 && sk > 0) {
    if (bias == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null pointer");
    if (bias_strides[2] != 1) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "bias needs unit key stride");
    if (bias_strides[0] < 0 || bias_strides[1] < 0)
      return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative bias stride");
    if (!aligned(bias, 4)) return fail(INTENT_HIP_ERR_UNSUPPORTED, "bias must be 4-byte aligned");
  }
  const KeyBias kb{bias, bias_strides[0], bias_strides[1]};
  return launch_attention(INTENT_HIP_F16, q, k, v, o, batch, heads, 1, sq, sk, d, dv, strides, scale, 0, stream,
                          &kb);
}

// ---------------------------------------------------------------- packed sequences
namespace {

int64_t varlen_capacity(int64_t sequences, int64_t total) { return (total + kBQ - 1) / kBQ + sequences; }
size_t varlen_workspace(int64_t sequences, int64_t total) {
  return 256 + 8 * static_cast<size_t>(varlen_capacity(sequences, total));
}

}  // namespace

extern "C" int intent_hip_attention_varlen_workspace_bytes(int64_t sequences, int64_t total, size_t *bytes) {
  if (bytes == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null output");
  if (sequences < 0 || total < 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  *bytes = varlen_workspace(sequences, total);
  return INTENT_HIP_OK;
}

extern "C" int intent_hip_attention_varlen_fwd(int dtype, const void *q, const void *k, const void *v,
                                               const int32_t *cu_seqlens, void *o, int64_t sequences, int64_t total,
                                               int64_t q_heads, int64_t head_group, int64_t d, int64_t dv,
                                               const int64_t *strides, float scale, int causal, void *workspace,
                                               size_t workspace_bytes, void *stream) {
  if (sequences < 0 || total < 0 || q_heads < 0 || d < 0 || dv < 0)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (head_group < 1 || (q_heads > 0 && q_heads % head_group != 0))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "head_group %lld must be positive and divide the %lld query heads",
                static_cast<long long>(head_group), static_cast<long long>(q_heads));
  if (dtype != INTENT_HIP_F16 && dtype != INTENT_HIP_BF16)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "attention dtype code %d (1 = f16, 2 = bf16)", dtype);
  if (sequences == 0 || total == 0 || q_heads == 0 || dv == 0) return INTENT_HIP_OK;
  if ((d != 64 && d != 128) || (dv != 64 && dv != 128))
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "attention kernels take D and DV in {64, 128} (got d=%lld, dv=%lld)",
                static_cast<long long>(d), static_cast<long long>(dv));
  if (strides == nullptr || q == nullptr || k == nullptr || v == nullptr || o == nullptr || cu_seqlens == nullptr)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null pointer");
  const int64_t capacity = varlen_capacity(sequences, total);
  if (total > INT32_MAX / 2 || sequences > INT32_MAX / 2 || capacity * q_heads > INT32_MAX)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "packed attention extents too large for one launch");
  if (workspace == nullptr || workspace_bytes < varlen_workspace(sequences, total) || !aligned(workspace, 256))
    return fail(INTENT_HIP_ERR_WORKSPACE, "packed attention needs %zu workspace bytes (256-byte aligned), got %zu",
                varlen_workspace(sequences, total), workspace_bytes);
  Geometry g{};   // batch strides stay 0: the sequence start moves the row
  // strides[] lists (row, head, inner) per tensor; the kernel's geometry is (batch, head, row, col).
  for (int t = 0; t < 4; ++t) {
    int64_t *dst = t == 0 ? g.qs : t == 1 ? g.ks : t == 2 ? g.vs : g.os;
    dst[2] = strides[3 * t];
    dst[1] = strides[3 * t + 1];
    dst[3] = strides[3 * t + 2];
  }
  if (g.qs[3] != 1 || g.ks[3] != 1 || g.vs[3] != 1 || g.os[3] != 1)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "attention tensors need unit inner stride");
  for (int i = 1; i < 3; ++i)
    if (g.qs[i] % 8 || g.ks[i] % 8 || g.vs[i] % 8 || g.os[i] % 4)
      return fail(INTENT_HIP_ERR_UNSUPPORTED, "attention strides must be multiples of 8 elements");
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(o, 8))
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "attention tensors must be 16-byte aligned");
  char *ws = static_cast<char *>(workspace);
  Ragged r{cu_seqlens, reinterpret_cast<const int2 *>(ws + 256), reinterpret_cast<const int32_t *>(ws),
           static_cast<int>(total)};
  const hipStream_t s = as_stream(stream);
  attention_varlen_items<<<1, 1024, 0, s>>>(cu_seqlens, static_cast<int>(sequences), static_cast<int>(total),
                                            reinterpret_cast<int2 *>(ws + 256), reinterpret_cast<int32_t *>(ws),
                                            static_cast<int>(capacity));
  if (hipPeekAtLastError() != hipSuccess) return launch_status("attention_varlen_items");
  const dim3 grid(static_cast<unsigned>(capacity * q_heads));
  launch_variant<kPacked>(dtype, d, dv, grid, s, static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k),
                       static_cast<const uint16_t *>(v), static_cast<uint16_t *>(o), static_cast<int>(q_heads),
                       static_cast<int>(head_group), 0, 0, g, scale, causal ? 1 : 0, 1, r);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("attention_fwd (packed)");
  return INTENT_HIP_OK;
}

// ---------------------------------------------------------------- latent attention
extern "C" int intent_hip_mla_prefill_workspace_bytes(int64_t batch, int64_t heads, int64_t sq, int64_t sk, int64_t d,
                                                      size_t *bytes) {
  if (bytes == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null output");
  if (batch < 0 || heads < 0 || sq < 0 || sk < 0 || d < 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  *bytes = split_layout(batch, heads, sq, sk, d).bytes;
  return INTENT_HIP_OK;
}

extern "C" int intent_hip_mla_prefill(const void *q, const void *qpe, const void *k, const void *kpe, const void *v,
                                      void *o, int64_t batch, int64_t heads, int64_t head_group, int64_t sq,
                                      int64_t sk, int64_t d, int64_t p, const int64_t *strides, float scale,
                                      void *workspace, size_t workspace_bytes, void *stream) {
  if (batch < 0 || heads < 0 || sq < 0 || sk < 0 || d < 0 || p < 0)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (head_group < 1 || (heads > 0 && heads % head_group != 0))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "head_group %lld must be positive and divide the %lld query heads",
                static_cast<long long>(head_group), static_cast<long long>(heads));
  if (batch == 0 || heads == 0 || sq == 0 || d == 0) return INTENT_HIP_OK;
  if ((d != 64 && d != 128) || p != 64)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "latent attention takes D in {64, 128} and P = 64 (got D=%lld, P=%lld)",
                static_cast<long long>(d), static_cast<long long>(p));
  if (strides == nullptr || q == nullptr || qpe == nullptr || o == nullptr ||
      (sk > 0 && (k == nullptr || kpe == nullptr || v == nullptr)))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null pointer");
  if (sq > INT32_MAX / 2 || sk > INT32_MAX / 2 || batch * heads > INT32_MAX / 64)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "attention extents too large for one launch");
  // strides: q[4], qpe[4], k[4], kpe[4], v[4], o[4], each (batch, head, row, col)
  Geometry g;
  RopeRows rr{static_cast<const uint16_t *>(qpe), static_cast<const uint16_t *>(kpe), {strides[4], strides[5], strides[6]},
              {strides[12], strides[14]}};
  for (int i = 0; i < 4; ++i) {
    g.qs[i] = strides[i];
    g.ks[i] = strides[8 + i];
    g.vs[i] = strides[16 + i];
    g.os[i] = strides[20 + i];
  }
  for (int t = 0; t < 6; ++t)
    if (strides[4 * t + 3] != 1) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "attention tensors need unit inner stride");
  for (int t = 0; t < 6; ++t)
    for (int i = 0; i < 3; ++i)
      if (strides[4 * t + i] % (t == 5 ? 4 : 8))
        return fail(INTENT_HIP_ERR_UNSUPPORTED, "attention strides must be multiples of 8 elements");
  if (!aligned(q, 16) || !aligned(qpe, 16) || (sk > 0 && (!aligned(k, 16) || !aligned(kpe, 16) || !aligned(v, 16))) ||
      !aligned(o, 8))
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "attention tensors must be 16-byte aligned");
  const int q_blocks = static_cast<int>((sq + kBQ - 1) / kBQ);
  // A key split needs the workspace intent_hip_mla_prefill_workspace_bytes names; without it (or
  // when the grid fills the chip) the launch is unsplit.
  KeySplit ks = key_split(split_layout(batch, heads, sq, sk, d), workspace, workspace_bytes);
  const int64_t blocks = batch * heads * q_blocks * ks.count;
  if (blocks > INT32_MAX) return fail(INTENT_HIP_ERR_UNSUPPORTED, "too many attention workgroups");
  ks.grouped = ks.count > 1 && blocks <= device_cus();
  const dim3 grid(static_cast<unsigned>(blocks));
  const hipStream_t s = as_stream(stream);
  const auto *Qp = static_cast<const uint16_t *>(q);
  const auto *Kp = static_cast<const uint16_t *>(k);
  const auto *Vp = static_cast<const uint16_t *>(v);
  auto *Op = static_cast<uint16_t *>(o);
  const int h = static_cast<int>(heads), grp = static_cast<int>(head_group);
  const int iq = static_cast<int>(sq), ik = static_cast<int>(sk);
  if (d == 128)
    launch_fwd<_Float16, 192, 128, kLatent>(grid, s, Qp, Kp, Vp, Op, h, grp, iq, ik, g, scale, 1, q_blocks, Ragged{},
                                            KeyBias{}, rr, ks);
  else
    launch_fwd<_Float16, 128, 64, kLatent>(grid, s, Qp, Kp, Vp, Op, h, grp, iq, ik, g, scale, 1, q_blocks, Ragged{},
                                           KeyBias{}, rr, ks);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("attention_fwd (latent)");
  if (ks.count > 1) {
    launch_merge(INTENT_HIP_F16, d, ks, h, iq, Op, g, s);
    if (hipPeekAtLastError() != hipSuccess) return launch_status("attention_split_merge");
  }
  return INTENT_HIP_OK;
}
