// Paged grouped-query decode attention, split over page ranges, and the split-K merge, for gfx950.
//
// Semantics:
//   paged_gqa_decode_partials (python/intent/examples/kernels/streaming/paged_attention.py:77-165)
//     with summarize_masked_attention_chunk (streaming/attention.py:250-285): for job
//     j = batch * SPLITS + split and key head kh, the HEAD_GROUP query heads kh * G + g attend over
//     the job's tokens t: page position first + t / PS (first = split_offsets[j]), physical page
//     page_indices[position], offset t % PS, logical token (position - page_offsets[batch]) *
//     PAGE_SIZE + offset, active while below sequence_lengths[batch]. Scores in the exp2 domain,
//     weights rounded to f16 before P @ V (f32 accumulation); partial_lse = max + ln(den) * log2 e
//     (-inf for an empty job), partial_output = acc * (1 / den) (0 for an empty job).
//   splitk_attention_f32_to_f16_reduce (streaming/splitk_reduce.py:129-155): per (batch, head)
//     m = maximum_num over splits of lse, w = exp(lse - m) (natural exponential, as the
//     definition writes it), out = f16(sum w * partial * rcp_approx(sum w)).
// P is rounded against each 64-token chunk's own maximum, as the definition's chunk summary does;
// the chunk's merge factor exp2(chunk max - running max) is folded into the stored weights, and
// the summed axes are reassociated. Scores use v_dot2_f32_f16 (f16 pair products summed in f32).
// Page positions and physical pages are clamped into their arrays (the definition assumes them in
// bounds), so a bad index cannot fault.
//
// Design (both kernels memory-bound):
//   * partials: one workgroup per (job, key head), 4 waves taking 64-token chunks in turn. Per
//     chunk, groups of up to 4 query heads load K as V is loaded below (16 bytes per lane, D / 8
//     lanes per token row, non-temporal) with this lane's 8 dimensions of every query in
//     registers, and fold the lanes' partial dot products by a reduce-scatter over the lane bits
//     (DPP and ds_swizzle), so each lane ends with the full scores of one token. Larger groups
//     score lane t = token t against the queries in LDS (read as broadcasts), each lane reading
//     its own K row. Chunk maxima and sums are wave reductions; P goes through LDS to the P @ V
//     phase, where each lane loads 16 bytes of a V row (D / 8 lanes per token, the chunk's loads
//     in flight together) and accumulates 8 output dimensions. Lanes sharing dimensions are
//     folded once per job, then the four waves' states are merged in wave order.
//   * merge: one single-wave workgroup per (batch, head) row; lanes own output dimensions, the
//     split loop is unrolled so its loads overlap.
#include "common.hpp"

namespace intent_hip {
namespace {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kChunk = 64;            // tokens per wave step
constexpr int kMaxGroup = 16;          // query heads per key head
constexpr float kLog2e = 1.4426950408889634f;

struct DecodeGeometry {
  int64_t q[3], k[4], v[4], lse[3], out[4];
};

// Where a job's tokens live (the partials kernel's kSrc):
//   kPaged  paged_gqa_decode_partials: job (batch, split) reads pages split_offsets[job] ..
//           split_offsets[job + 1]; k and v strides (page, offset, head).
//   kDense  k/v rows at b k[0] + key k[1] + head k[2]; job (batch, split) covers keys split * span
//           .. + span below `keys`, active where the optional u8 mask [b, key, head] is nonzero.
//   kPacked k/v [U, HK, D] rows; sequence b is rows cu[b] .. cu[b + 1] (clamped into [0, rows]),
//           of which the first `keys` count; job (b, split) covers split * span .. + span of them.
constexpr int kPaged = 0, kDense = 1, kPacked = 2;
// What the partials kernel writes (kOut): normalised f32 or element-type partials with their
// log2-sum-exp2 (partial_lse, partial_output), or the unnormalised state (maximum, denominator,
// sums) of each split for decode_merge.
constexpr int kOutF32 = 0, kOutElem = 1, kOutState = 2;

struct DecodeSource {
  const int32_t *page_offsets, *page_indices, *lengths, *split_offsets;   // kPaged
  int64_t pages, positions;
  int ps, page_size;
  const uint8_t *mask;   // kDense: validity of (batch, key, head), or null for every key
  int64_t mask_s[3];
  const int32_t *cu;     // kPacked: row offsets of the sequences
  int rows;              // kPacked: rows of k and v
  int keys;              // kDense: K; kPacked: keys per sequence taken at most
  int span;              // kDense, kPacked: keys per split (a multiple of the 64-key chunk)
};

struct DecodeTarget {
  float *lse;            // kOutF32, kOutElem: [B, HQ, S] (strides g.lse)
  void *out;             // kOutF32, kOutElem: [B, HQ, S, D] (strides g.out)
  float *state_m, *state_den, *state_acc;   // kOutState: [B HQ S], [B HQ S], [B HQ S][D]
  float *block_max;      // kPacked: each 64-key block's score maximum [B, HQ, block] (strides bm), or null
  int64_t bm[3];
};

template <typename E>
__device__ __forceinline__ float dot8(uint4 a, uint4 b, float t) {
  if constexpr (__is_same(E, _Float16)) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    t = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a.x), __builtin_bit_cast(h2, b.x), t, false);
    t = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a.y), __builtin_bit_cast(h2, b.y), t, false);
    t = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a.z), __builtin_bit_cast(h2, b.z), t, false);
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a.w), __builtin_bit_cast(h2, b.w), t, false);
  } else {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    t = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, a.x), __builtin_bit_cast(b2, b.x), t, false);
    t = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, a.y), __builtin_bit_cast(b2, b.y), t, false);
    t = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, a.z), __builtin_bit_cast(b2, b.z), t, false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, a.w), __builtin_bit_cast(b2, b.w), t, false);
  }
}

// The value of lane (lane ^ m), m in {1, 2, 4, 8}: quad permutes and row_ror:8 (DPP, within 16-lane
// rows) for 1, 2 and 8; ds_swizzle in bit mode (xor within 32 lanes) for 4. Every lane active.
__device__ __forceinline__ float lane_xor(float v, int m) {
  if (m == 1) return dpp_move<0xB1>(v);
  if (m == 2) return dpp_move<0x4E>(v);
  if (m == 8) return dpp_move<0x128>(v);
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x101F));
}

// kG bounds the query heads per key head (the group runs 1..kG; register arrays are sized by kG
// and every loop over them is unrolled with a uniform guard, so nothing is indexed dynamically).
template <typename E, int D, int kG, int kSrc, int kOut>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kG <= 4 ? 4 : 2))) void decode_partials(
    const uint16_t *__restrict__ Q, const uint16_t *__restrict__ KC, const uint16_t *__restrict__ VC, int kv_heads,
    int group, int splits, DecodeSource src, DecodeTarget dst, DecodeGeometry g, float scale) {
  typedef E e8_t __attribute__((ext_vector_type(8)));
  constexpr int kLanesPerToken = D / 8;            // 16 bytes of a row per lane
  constexpr int kTokensPerLoad = 64 / kLanesPerToken;
  constexpr int kSlots = kChunk / kTokensPerLoad;   // loads per lane for a whole chunk
  constexpr int kBatch = kG >= 16 ? kSlots / 4 : kSlots / 2;
  __shared__ __attribute__((aligned(16))) uint16_t q_s[kG * D];
  __shared__ float p_s[kWaves][kG][kChunk];
  __shared__ int64_t row_s[kWaves][kChunk];   // per token: physical row offset (elements) in the caches
  __shared__ float m_s[kWaves][kG], den_s[kWaves][kG];
  __shared__ float acc_s[kWaves][kG][D];
  __shared__ int valid_s[kWaves];
  // Groups of up to four query heads score with coalesced K loads (kLanesPerToken lanes per token
  // row, 16 bytes each) and fold the lanes' partial dot products by a reduce-scatter in registers.
  constexpr bool kCoalesced = kG <= 4;
  __shared__ int64_t key_s[kWaves][kCoalesced ? kChunk : 1];   // per token: K row offset, -1 if inactive

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Workgroups go to the 8 XCDs round-robin; give each XCD a contiguous run of (job, key head)
  // items so every key head of a job runs on one XCD together and the 2 KB token rows of the
  // interleaved caches are read whole, close in time.
  const int n = static_cast<int>(gridDim.x), xcd = static_cast<int>(blockIdx.x) % 8;
  const int item = xcd * (n / 8) + (xcd < n % 8 ? xcd : n % 8) + static_cast<int>(blockIdx.x) / 8;
  const int kh = item % kv_heads;
  const int job = item / kv_heads;
  const int b = job / splits, split = job % splits;
  int first = 0, tokens = 0;
  int64_t length = 0, page_begin = 0;
  if constexpr (kSrc == kPaged) {
    first = src.split_offsets[job];
    int64_t count = static_cast<int64_t>(src.split_offsets[job + 1]) - first;
    count = count < 0 ? 0 : (count > src.positions ? src.positions : count);
    tokens = static_cast<int>(count * src.ps);     // host checks positions * ps < 2^31
    length = src.lengths[b];
    page_begin = src.page_offsets[b];
  } else {
    // first: the job's first key (kDense) or row (kPacked); host checks splits * span < 2^31.
    int available = src.keys;
    first = split * src.span;
    if constexpr (kSrc == kPacked) {
      const int lo = min(max(src.cu[b], 0), src.rows), hi = min(max(src.cu[b + 1], lo), src.rows);
      available = min(hi - lo, src.keys);
      tokens = max(0, min(available - first, src.span));
      first += lo;
    } else {
      tokens = max(0, min(available - first, src.span));
    }
  }
  const float c1 = scale * kLog2e;

  for (int i = tid; i < group * D; i += kThreads) {
    const int gq = i / D, c = i % D;
    q_s[i] = Q[b * g.q[0] + (kh * group + gq) * g.q[1] + c];
  }
  __syncthreads();

  const int token_lane = lane / kLanesPerToken, dim0 = (lane % kLanesPerToken) * 8;
  float m[kG], den[kG], acc[kG][8];
#pragma unroll
  for (int gq = 0; gq < kG; ++gq) {
    m[gq] = -INFINITY;
    den[gq] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[gq][e] = 0.0f;
  }
  bool valid = false;
  uint4 qr[kCoalesced ? kG : 1];   // this lane's 8 dimensions of each query head of the group
  if constexpr (kCoalesced) {
#pragma unroll
    for (int gq = 0; gq < kG; ++gq)
      qr[gq] = gq < group ? *reinterpret_cast<const uint4 *>(q_s + gq * D + dim0) : make_uint4(0, 0, 0, 0);
  }

  for (int c0 = wave * kChunk; c0 < tokens; c0 += kWaves * kChunk) {
    // Addresses: lane t <-> token c0 + t (its K row offset, and its V row offset for P @ V).
    const int flat = c0 + lane;
    bool active = false;
    float s[kG];
#pragma unroll
    for (int gq = 0; gq < kG; ++gq) s[gq] = 0.0f;
    int64_t key_row = 0;
    if (flat < tokens) {
      if constexpr (kSrc == kPaged) {
        int64_t position = first + flat / src.ps;
        position = position < 0 ? 0 : (position >= src.positions ? src.positions - 1 : position);
        const int offset = flat % src.ps;
        int64_t physical = src.page_indices[position];
        physical = physical < 0 ? 0 : (physical >= src.pages ? src.pages - 1 : physical);
        active = (position - page_begin) * src.page_size + offset < length;
        key_row = physical * g.k[0] + offset * g.k[1] + kh * g.k[2];
        row_s[wave][lane] = physical * g.v[0] + offset * g.v[1] + kh * g.v[2];
      } else {
        const int64_t key = first + flat;
        active = true;
        if constexpr (kSrc == kDense)
          if (src.mask != nullptr) active = src.mask[b * src.mask_s[0] + key * src.mask_s[1] + kh * src.mask_s[2]] != 0;
        key_row = b * g.k[0] + key * g.k[1] + kh * g.k[2];
        row_s[wave][lane] = b * g.v[0] + key * g.v[1] + kh * g.v[2];
      }
    }
    int mine = lane;                               // the chunk token whose scores this lane holds
    if constexpr (kCoalesced) {
      key_s[wave][lane] = active ? key_row : -1;
      if (!__any(active)) continue;
      __builtin_amdgcn_wave_barrier();
      // Slot j of a lane is token j * kTokensPerLoad + token_lane, dimensions dim0 .. dim0 + 8. The
      // kSlots loads go in kNB batches of kB. Each batch's partial sums are folded over the lane
      // bits below kB: at each step a lane keeps the half of its slots that its lane bit selects
      // and adds the partner's sums for them. The batches are then folded the same way over the
      // lane bits kB .. kSlots / 2. Lane (token_lane, dc) ends with the full scores of slot dc,
      // i.e. of token dc * kTokensPerLoad + token_lane (measured against 2 batches of 8 and one
      // of 16: 52.0, 53.1 and 73.5 us at the B8 HQ32 HK8 D128 decode shape).
      constexpr int kNB = 4;
      constexpr int kB = kSlots / kNB;
      float red[kNB][kG];
#pragma unroll
      for (int h = 0; h < kNB; ++h) {
        uint4 kv[kB];
#pragma unroll
        for (int j = 0; j < kB; ++j) {
          const int64_t r = key_s[wave][(h * kB + j) * kTokensPerLoad + token_lane];
          kv[j] = make_uint4(0, 0, 0, 0);
          if (r >= 0) kv[j] = __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const e8_t *>(KC + r + dim0)));
        }
        float v[kB][kG];
#pragma unroll
        for (int j = 0; j < kB; ++j)
#pragma unroll
          for (int gq = 0; gq < kG; ++gq) {
            v[j][gq] = gq < group ? dot8<E>(qr[gq], kv[j], 0.0f) : 0.0f;
          }
#pragma unroll
        for (int n = kB; n > 1; n /= 2) {
          const bool upper = (lane & (n / 2)) != 0;
#pragma unroll
          for (int j = 0; j < n / 2; ++j)
#pragma unroll
            for (int gq = 0; gq < kG; ++gq)
              if (gq < group) {
                const float keep = upper ? v[j + n / 2][gq] : v[j][gq];
                const float give = upper ? v[j][gq] : v[j + n / 2][gq];
                v[j][gq] = keep + lane_xor(give, n / 2);
              }
        }
#pragma unroll
        for (int gq = 0; gq < kG; ++gq) red[h][gq] = v[0][gq];
      }
#pragma unroll
      for (int n = kNB; n > 1; n /= 2) {
        const bool upper = (lane & (kB * n / 2)) != 0;
#pragma unroll
        for (int h = 0; h < n / 2; ++h)
#pragma unroll
          for (int gq = 0; gq < kG; ++gq)
            if (gq < group) {
              const float keep = upper ? red[h + n / 2][gq] : red[h][gq];
              const float give = upper ? red[h][gq] : red[h + n / 2][gq];
              red[h][gq] = keep + lane_xor(give, kB * n / 2);
            }
      }
#pragma unroll
      for (int gq = 0; gq < kG; ++gq) s[gq] = red[0][gq];
      mine = (lane % kLanesPerToken) * kTokensPerLoad + token_lane;
      active = key_s[wave][mine] >= 0;
    } else {
      if (active) {                                  // inactive tokens are never read for scores
        // q.k with v_dot2_f32_f16 (products of f16 pairs summed in f32), half a row at a time.
        const uint4 *krow = reinterpret_cast<const uint4 *>(KC + key_row);
  #pragma unroll
        for (int half = 0; half < 2; ++half) {
          uint4 kv[D / 16];
  #pragma unroll
          for (int c = 0; c < D / 16; ++c) kv[c] = krow[half * (D / 16) + c];
  #pragma unroll
          for (int c = 0; c < D / 16; ++c) {
  #pragma unroll
            for (int gq = 0; gq < kG; ++gq) {
              if (gq < group) {
                const uint4 qv = *reinterpret_cast<const uint4 *>(q_s + gq * D + (half * (D / 16) + c) * 8);
                s[gq] = dot8<E>(qv, kv[c], s[gq]);
              }
            }
          }
        }
      }
      if (!__any(active)) continue;
    }
    valid = true;
    // Chunk summary as the definition forms it: weights against the chunk's own maximum, rounded
    // to the element type for P @ V; the chunk joins the running state with exp2 factors (left for the state,
    // right for the chunk, folded into the stored weights).
    float left[kG];
#pragma unroll
    for (int gq = 0; gq < kG; ++gq) {
      left[gq] = 1.0f;
      if (gq < group) {
        const float score = active ? s[gq] * c1 : -INFINITY;
        const float chunk_max = wave_max(score);
        const float p = active ? __builtin_amdgcn_exp2f(score - chunk_max) : 0.0f;
        const float chunk_den = wave_sum(p);
        const float next = fmaxf(m[gq], chunk_max);
        left[gq] = m[gq] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m[gq] - next);
        const float right = __builtin_amdgcn_exp2f(chunk_max - next);
        m[gq] = next;
        den[gq] = left[gq] * den[gq] + right * chunk_den;
        p_s[wave][gq][mine] = right * static_cast<float>(round_to<E>(p));
        if constexpr (kSrc == kPacked)
          if (dst.block_max != nullptr && lane == 0)
            dst.block_max[b * dst.bm[0] + (kh * group + gq) * dst.bm[1] +
                          static_cast<int64_t>((split * src.span + c0) / kChunk) * dst.bm[2]] = chunk_max;
      }
    }
#pragma unroll
    for (int gq = 0; gq < kG; ++gq)
      if (gq < group)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[gq][j] *= left[gq];
    __builtin_amdgcn_wave_barrier();
    // P @ V: lane l reads dimensions 8 (l % kLanesPerToken) .. + 8 of token
    // slot * kTokensPerLoad + l / kLanesPerToken; one load per slot, all slots of a batch in flight.
    const int chunk_tokens = tokens - c0 < kChunk ? tokens - c0 : kChunk;
#pragma unroll
    for (int base = 0; base < kSlots; base += kBatch) {
      e8_t vv[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int token = (base + j) * kTokensPerLoad + token_lane;
        vv[j] = e8_t{};
        if (token < chunk_tokens)
          vv[j] = __builtin_nontemporal_load(reinterpret_cast<const e8_t *>(VC + row_s[wave][token] + dim0));
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int token = (base + j) * kTokensPerLoad + token_lane;
#pragma unroll
        for (int gq = 0; gq < kG; ++gq) {
          if (gq < group) {
            const float p = p_s[wave][gq][token];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[gq][e] = fmaf(p, static_cast<float>(vv[j][e]), acc[gq][e]);
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }

  // Lanes that share dimensions hold sums over different tokens: fold them once.
#pragma unroll
  for (int gq = 0; gq < kG; ++gq)
    if (gq < group)
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int x = kLanesPerToken; x < 64; x <<= 1) acc[gq][e] += __shfl_xor(acc[gq][e], x);

  // Merge the waves' states in wave order.
  if (lane == 0) valid_s[wave] = valid ? 1 : 0;
#pragma unroll
  for (int gq = 0; gq < kG; ++gq) {
    if (gq < group) {
      if (lane == 0) {
        m_s[wave][gq] = m[gq];
        den_s[wave][gq] = den[gq];
      }
      if (lane < kLanesPerToken)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc_s[wave][gq][dim0 + e] = acc[gq][e];
    }
  }
  __syncthreads();
  for (int i = tid; i < group * D; i += kThreads) {
    const int gq = i / D, c = i % D;
    float top = -INFINITY;
    bool any = false;
    for (int w = 0; w < kWaves; ++w)
      if (valid_s[w]) {
        any = true;
        top = fmaxf(top, m_s[w][gq]);
      }
    float total = 0.0f, value = 0.0f;
    for (int w = 0; w < kWaves; ++w)
      if (valid_s[w]) {
        const float f = __builtin_amdgcn_exp2f(m_s[w][gq] - top);
        total = fmaf(f, den_s[w][gq], total);
        value = fmaf(f, acc_s[w][gq][c], value);
      }
    const int h = kh * group + gq;
    if constexpr (kOut == kOutState) {
      const int64_t slot = (static_cast<int64_t>(b) * kv_heads * group + h) * splits + split;
      dst.state_acc[slot * D + c] = any ? value : 0.0f;
      if (c == 0) {
        dst.state_m[slot] = any ? top : -INFINITY;
        dst.state_den[slot] = any ? total : 0.0f;
      }
    } else {
      const float normalised = any ? value * (1.0f / total) : 0.0f;
      const int64_t at = b * g.out[0] + h * g.out[1] + split * g.out[2] + c;
      if constexpr (kOut == kOutF32)
        static_cast<float *>(dst.out)[at] = normalised;
      else
        static_cast<uint16_t *>(dst.out)[at] = __builtin_bit_cast(uint16_t, round_to<E>(normalised));
      if (c == 0) dst.lse[b * g.lse[0] + h * g.lse[1] + split * g.lse[2]] = any ? top + logf(total) * kLog2e : -INFINITY;
    }
  }
}

// One wave per (batch, head) row, one workgroup per row so the rows spread over every CU. Lanes
// own output dimensions; the split loop is unrolled so its loads are in flight together.
__global__ __launch_bounds__(64) void splitk_reduce_f32_to_f16(const float *__restrict__ P,
                                                              const float *__restrict__ LSE,
                                                              uint16_t *__restrict__ OUT, int heads, int splits,
                                                              int d, DecodeGeometry g) {
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t b = row / heads, h = row % heads;
  const float *lse = LSE + b * g.lse[0] + h * g.lse[1];
  float top = -INFINITY;
  for (int s = lane; s < splits; s += 64) top = fmaxf(top, lse[s * g.lse[2]]);
  top = wave_max(top);
  float den = 0.0f;
  for (int s = lane; s < splits; s += 64) den += expf(lse[s * g.lse[2]] - top);
  den = wave_sum(den);
  const float inv = __builtin_amdgcn_rcpf(den);
  const float *prow = P + b * g.q[0] + h * g.q[1];
  for (int c = lane; c < d; c += 64) {
    float num = 0.0f;
#pragma unroll 8
    for (int s = 0; s < splits; ++s) num = fmaf(expf(lse[s * g.lse[2]] - top), prow[s * g.q[2] + c], num);
    OUT[b * g.out[0] + h * g.out[1] + c] = __builtin_bit_cast(uint16_t, round_to<_Float16>(num * inv));
  }
}

// The split states of one (batch, head) row merged as merge_attention_summaries does: weights
// exp2(m_s - M) against the largest maximum M (approximate, as the definition's), the denominator
// plus an optional per-head sink (varlen_gqa_decode_with_sink_logits adds sink[head] to the merged
// denominator), normalised by an approximate reciprocal and cast to f16; 0 for a row with no valid
// key. With block maxima, block j's entry becomes exp2(max_j - M) / denominator for j below the
// sequence's block count ceil(length / 64) and 0 above it. One wave per row; lanes own columns.
template <int D>
__global__ __launch_bounds__(64) void decode_merge(const float *__restrict__ state_m, const float *__restrict__ state_den,
                                                   const float *__restrict__ state_acc, int heads, int splits,
                                                   const float *__restrict__ sink, uint16_t *__restrict__ OUT,
                                                   int64_t out_b, int64_t out_h, float *__restrict__ block_max,
                                                   int64_t bm_b, int64_t bm_h, int64_t bm_k,
                                                   const int32_t *__restrict__ cu, int rows, int max_blocks) {
  constexpr int kPer = D / 64;   // columns per lane
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int b = static_cast<int>(row / heads), h = static_cast<int>(row % heads);
  const int64_t base = row * splits;
  float top = -INFINITY;
  for (int s = lane; s < splits; s += 64) top = fmaxf(top, state_m[base + s]);
  top = wave_max(top);
  const bool valid = top != -INFINITY;
  float den = 0.0f;
  for (int s = lane; s < splits; s += 64) {
    const float m = state_m[base + s];
    if (m != -INFINITY) den = fmaf(__builtin_amdgcn_exp2f(m - top), state_den[base + s], den);
  }
  den = wave_sum(den);
  if (sink != nullptr) den += sink[h];
  const float inv = __builtin_amdgcn_rcpf(valid ? den : 1.0f);
  float acc[kPer];
#pragma unroll
  for (int e = 0; e < kPer; ++e) acc[e] = 0.0f;
  // Empty splits hold m = -inf and zero sums; no branch in the loop, so its loads issue together.
  if (valid) {
#pragma unroll 8
    for (int s = 0; s < splits; ++s) {
      const float m = state_m[base + s];   // the same for every lane
      const float f = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - top);
      const float *part = state_acc + (base + s) * D;
#pragma unroll
      for (int e = 0; e < kPer; ++e) acc[e] = fmaf(f, part[lane + 64 * e], acc[e]);
    }
  }
  uint16_t *orow = OUT + b * out_b + h * out_h;
#pragma unroll
  for (int e = 0; e < kPer; ++e)
    orow[lane + 64 * e] = __builtin_bit_cast(uint16_t, round_to<_Float16>(valid ? acc[e] * inv : 0.0f));
  if (block_max != nullptr) {
    const int lo = min(max(cu[b], 0), rows), hi = min(max(cu[b + 1], lo), rows);
    const int count = (hi - lo + kChunk - 1) / kChunk;
    float *blocks = block_max + b * bm_b + h * bm_h;
    for (int j = lane; j < max_blocks; j += 64)
      blocks[j * bm_k] = j < count && valid ? __builtin_amdgcn_exp2f(blocks[j * bm_k] - top) * inv : 0.0f;
  }
}

}  // namespace

template <typename E, int D, int kSrc, int kOut>
const void *partials_kernel(int64_t group) {
  if (group <= 4) return reinterpret_cast<const void *>(&decode_partials<E, D, 4, kSrc, kOut>);
  if (group <= 8) return reinterpret_cast<const void *>(&decode_partials<E, D, 8, kSrc, kOut>);
  return reinterpret_cast<const void *>(&decode_partials<E, D, 16, kSrc, kOut>);
}

// The instantiation serving one definition: paged (f16 partials in f32), dense bf16 partials
// (grouped_flash_decode_partials), dense f16 with a mask (continuous_gqa_decode) or packed f16
// (varlen_gqa_decode_with_sink_logits), the last two into split states.
enum DecodeVariant { kVariantPaged = 0, kVariantGroupedBf16 = 1, kVariantContinuous = 2, kVariantPackedSink = 3 };

const void *variant_kernel(int variant, int64_t d, int64_t group, char *name, size_t size) {
  static const char *const names[] = {"paged_decode_partials", "decode_partials<bf16,dense>",
                                      "decode_partials<f16,dense,state>", "decode_partials<f16,packed,state>"};
  const int g = group <= 4 ? 4 : group <= 8 ? 8 : 16;
  snprintf(name, size, "%s<%d,%d>", names[variant], static_cast<int>(d), g);
  const bool wide = d == 128;
  switch (variant) {
    case kVariantGroupedBf16:
      return wide ? partials_kernel<__bf16, 128, kDense, kOutElem>(group)
                  : partials_kernel<__bf16, 64, kDense, kOutElem>(group);
    case kVariantContinuous:
      return wide ? partials_kernel<_Float16, 128, kDense, kOutState>(group)
                  : partials_kernel<_Float16, 64, kDense, kOutState>(group);
    case kVariantPackedSink:
      return wide ? partials_kernel<_Float16, 128, kPacked, kOutState>(group)
                  : partials_kernel<_Float16, 64, kPacked, kOutState>(group);
    default:
      return wide ? partials_kernel<_Float16, 128, kPaged, kOutF32>(group)
                  : partials_kernel<_Float16, 64, kPaged, kOutF32>(group);
  }
}

// which: 0 paged partials, 1 split-K merge, 2 grouped bf16 partials, 3 continuous partials,
// 4 packed (sink) partials, 5 decode_merge.
int decode_resources(int64_t which, int64_t d, int64_t group, IntentHipKernelResources *out) {
  if (which == 1)
    return describe_kernel(reinterpret_cast<const void *>(&splitk_reduce_f32_to_f16), "splitk_reduce_f32_to_f16",
                           64, out);
  if (which == 5)
    return describe_kernel(d == 64 ? reinterpret_cast<const void *>(&decode_merge<64>)
                                   : reinterpret_cast<const void *>(&decode_merge<128>),
                           d == 64 ? "decode_merge<64>" : "decode_merge<128>", 64, out);
  if (d != 64 && d != 128) return fail(INTENT_HIP_ERR_UNSUPPORTED, "decode kernels take D = 64 or 128");
  char name[64];
  const int variant = which == 0 ? kVariantPaged : static_cast<int>(which) - 1;
  const void *kernel = variant_kernel(variant, d, group, name, sizeof name);
  return describe_kernel(kernel, name, kThreads, out);
}

// Splits of a dense or packed decode: enough (batch, key head, split) workgroups to fill the chip
// (2048, eight per CU) with at least 256 keys (one chunk per wave) per split; spans are whole
// 64-key chunks, so packed splits start on block boundaries.
void decode_splits(int64_t jobs, int64_t keys, int64_t *splits, int64_t *span) {
  int64_t s = jobs > 0 ? (2048 + jobs - 1) / jobs : 1;
  const int64_t most = keys > 256 ? (keys + 255) / 256 : 1;
  s = s < 1 ? 1 : (s > most ? most : s);
  int64_t sp = (keys + s - 1) / s;
  sp = sp < 1 ? kChunk : (sp + kChunk - 1) / kChunk * kChunk;
  *span = sp;
  *splits = keys > 0 ? (keys + sp - 1) / sp : 1;
}

// Split states in a workspace: maxima, denominators (each from a 256-byte boundary), then sums.
struct StateLayout {
  size_t den, acc, bytes;
};
StateLayout state_layout(int64_t rows_heads, int64_t splits, int64_t dv) {
  const size_t n = static_cast<size_t>(rows_heads) * static_cast<size_t>(splits);
  const size_t part = (4 * n + 255) / 256 * 256;
  return StateLayout{part, 2 * part, 2 * part + 4 * n * static_cast<size_t>(dv)};
}

int launch_partials(int variant, int64_t d, const uint16_t *Q, const uint16_t *K, const uint16_t *V, int64_t kv_heads,
                    int64_t group, int64_t splits, int64_t blocks, const DecodeSource &src, const DecodeTarget &dst,
                    const DecodeGeometry &g, float scale, void *stream) {
  char name[64];
  const void *kernel = variant_kernel(variant, d, group, name, sizeof name);
  int kv = static_cast<int>(kv_heads), grp = static_cast<int>(group), spl = static_cast<int>(splits);
  DecodeSource s = src;
  DecodeTarget t = dst;
  DecodeGeometry geometry = g;
  void *args[] = {&Q, &K, &V, &kv, &grp, &spl, &s, &t, &geometry, &scale};
  const hipError_t rc = hipLaunchKernel(kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), args, 0,
                                        as_stream(stream));
  if (rc != hipSuccess) return launch_status(name);
  return INTENT_HIP_OK;
}

}  // namespace intent_hip

using namespace intent_hip;

extern "C" int intent_hip_paged_decode_partials(const void *q, const void *key_cache, const void *value_cache,
                                                const int32_t *page_offsets, const int32_t *page_indices,
                                                const int32_t *lengths, const int32_t *split_offsets,
                                                float *partial_lse, float *partial_output, int64_t batch,
                                                int64_t q_heads, int64_t d, int64_t pages, int64_t ps,
                                                int64_t kv_heads, int64_t dv, int64_t positions,
                                                int64_t page_size, int64_t head_group, int64_t splits,
                                                const int64_t *strides, float scale, void *stream) {
  if (batch < 0 || q_heads < 0 || d < 0 || pages < 0 || ps < 0 || kv_heads < 0 || dv < 0 || positions < 0 ||
      splits < 0)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (head_group < 1 || head_group > kMaxGroup || q_heads != kv_heads * head_group)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT,
                "query heads (%lld) must equal key heads (%lld) * HEAD_GROUP (%lld), HEAD_GROUP in 1..%d",
                static_cast<long long>(q_heads), static_cast<long long>(kv_heads),
                static_cast<long long>(head_group), kMaxGroup);
  if (batch == 0 || q_heads == 0 || splits == 0) return INTENT_HIP_OK;
  if ((d != 64 && d != 128) || dv != d)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "paged decode supports D = DV = 64 or 128 (got %lld, %lld)",
                static_cast<long long>(d), static_cast<long long>(dv));
  if (page_size < 1 || ps < 1) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "page sizes must be positive");
  if (pages < 1 || positions < 1) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "empty page cache or page table");
  if (strides == nullptr || q == nullptr || key_cache == nullptr || value_cache == nullptr ||
      page_offsets == nullptr || page_indices == nullptr || lengths == nullptr || split_offsets == nullptr ||
      partial_lse == nullptr || partial_output == nullptr)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null pointer");
  DecodeGeometry g{};
  for (int i = 0; i < 3; ++i) g.q[i] = strides[i];
  for (int i = 0; i < 4; ++i) {
    g.k[i] = strides[3 + i];
    g.v[i] = strides[7 + i];
    g.out[i] = strides[14 + i];
  }
  for (int i = 0; i < 3; ++i) g.lse[i] = strides[11 + i];
  if (g.q[2] != 1 || g.k[3] != 1 || g.v[3] != 1 || g.out[3] != 1)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "q, caches and partial_output need unit inner stride");
  for (int i = 0; i < 3; ++i)
    if (g.k[i] % 8 || g.v[i] % 8)
      return fail(INTENT_HIP_ERR_UNSUPPORTED, "cache strides must be multiples of 8 elements");
  if (!aligned(key_cache, 16) || !aligned(value_cache, 16))
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "key and value caches must be 16-byte aligned");
  const int64_t blocks = batch * splits * kv_heads;
  if (blocks > INT32_MAX || ps > INT32_MAX || page_size > INT32_MAX || positions * ps >= INT32_MAX)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "extents too large");
  const auto *Q = static_cast<const uint16_t *>(q);
  const auto *K = static_cast<const uint16_t *>(key_cache);
  const auto *V = static_cast<const uint16_t *>(value_cache);
  DecodeSource src{};
  src.page_offsets = page_offsets;
  src.page_indices = page_indices;
  src.lengths = lengths;
  src.split_offsets = split_offsets;
  src.pages = pages;
  src.positions = positions;
  src.ps = static_cast<int>(ps);
  src.page_size = static_cast<int>(page_size);
  DecodeTarget dst{};
  dst.lse = partial_lse;
  dst.out = partial_output;
  return launch_partials(kVariantPaged, d, Q, K, V, kv_heads, head_group, splits, blocks, src, dst, g, scale, stream);
}

extern "C" int intent_hip_splitk_reduce_f32_to_f16(const float *partial, const float *lse, void *out, int64_t batch,
                                                   int64_t heads, int64_t splits, int64_t d, const int64_t *strides,
                                                   void *stream) {
  if (batch < 0 || heads < 0 || splits < 0 || d < 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (batch == 0 || heads == 0 || d == 0) return INTENT_HIP_OK;
  if (partial == nullptr || lse == nullptr || out == nullptr || strides == nullptr)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null pointer");
  if (splits > INT32_MAX || d > INT32_MAX || heads > INT32_MAX) return fail(INTENT_HIP_ERR_UNSUPPORTED, "extents too large");
  DecodeGeometry g{};
  for (int i = 0; i < 3; ++i) g.q[i] = strides[i];
  for (int i = 0; i < 3; ++i) g.lse[i] = strides[4 + i];
  for (int i = 0; i < 3; ++i) g.out[i] = strides[7 + i];
  if ((strides[3] != 1 || strides[9] != 1) && d > 1)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "partial and output need unit inner stride");
  const int64_t rows = batch * heads;
  if (rows > INT32_MAX) return fail(INTENT_HIP_ERR_UNSUPPORTED, "extents too large");
  splitk_reduce_f32_to_f16<<<dim3(static_cast<unsigned>(rows)), dim3(64), 0, as_stream(stream)>>>(
      partial, lse, static_cast<uint16_t *>(out), static_cast<int>(heads), static_cast<int>(splits),
      static_cast<int>(d), g);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("splitk_reduce_f32_to_f16");
  return INTENT_HIP_OK;
}

// ---------------------------------------------------------------- dense and packed decode

namespace {

bool decode_shape_ok(int64_t d, int64_t dv) { return (d == 64 || d == 128) && dv == d; }

int check_group(int64_t q_heads, int64_t kv_heads, int64_t head_group) {
  if (head_group < 1 || head_group > kMaxGroup || q_heads != kv_heads * head_group)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT,
                "query heads (%lld) must equal key heads (%lld) * HEAD_GROUP (%lld), HEAD_GROUP in 1..%d",
                static_cast<long long>(q_heads), static_cast<long long>(kv_heads),
                static_cast<long long>(head_group), kMaxGroup);
  return INTENT_HIP_OK;
}

// k and v geometry (row of a key: b k[0] + key k[1] + head k[2]) with the loads' requirements.
int rows_geometry(const int64_t *ks, const int64_t *vs, const void *k, const void *v, DecodeGeometry *g) {
  for (int i = 0; i < 3; ++i) {
    g->k[i] = ks[i];
    g->v[i] = vs[i];
    if (ks[i] % 8 || vs[i] % 8) return fail(INTENT_HIP_ERR_UNSUPPORTED, "key and value strides must be multiples of 8 elements");
  }
  if (!aligned(k, 16) || !aligned(v, 16)) return fail(INTENT_HIP_ERR_UNSUPPORTED, "keys and values must be 16-byte aligned");
  return INTENT_HIP_OK;
}

int launch_merge(int64_t dv, const StateLayout &layout, char *ws, int64_t rows, int64_t heads, int64_t splits,
                 const float *sink, void *out, int64_t out_b, int64_t out_h, float *block_max, const int64_t *bm,
                 const int32_t *cu, int64_t total_rows, int64_t max_blocks, void *stream) {
  const float *m = reinterpret_cast<const float *>(ws), *den = reinterpret_cast<const float *>(ws + layout.den);
  const float *acc = reinterpret_cast<const float *>(ws + layout.acc);
  auto *o = static_cast<uint16_t *>(out);
  const int h = static_cast<int>(heads), spl = static_cast<int>(splits), r = static_cast<int>(total_rows);
  const int mb = static_cast<int>(max_blocks);
  const int64_t b0 = bm ? bm[0] : 0, b1 = bm ? bm[1] : 0, b2 = bm ? bm[2] : 0;
  if (dv == 64)
    decode_merge<64><<<dim3(static_cast<unsigned>(rows)), dim3(64), 0, as_stream(stream)>>>(
        m, den, acc, h, spl, sink, o, out_b, out_h, block_max, b0, b1, b2, cu, r, mb);
  else
    decode_merge<128><<<dim3(static_cast<unsigned>(rows)), dim3(64), 0, as_stream(stream)>>>(
        m, den, acc, h, spl, sink, o, out_b, out_h, block_max, b0, b1, b2, cu, r, mb);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("decode_merge");
  return INTENT_HIP_OK;
}

}  // namespace

extern "C" int intent_hip_grouped_decode_partials(const void *q, const void *k, const void *v, float *partial_lse,
                                                  void *partial_output, int64_t batch, int64_t q_heads,
                                                  int64_t kv_heads, int64_t head_group, int64_t keys, int64_t d,
                                                  int64_t dv, int64_t parts, int64_t split_size,
                                                  const int64_t *strides, float scale, void *stream) {
  if (batch < 0 || q_heads < 0 || kv_heads < 0 || keys < 0 || d < 0 || dv < 0 || parts < 0 || split_size < 1)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent or SPLIT_SIZE below 1");
  if (int rc = check_group(q_heads, kv_heads, head_group)) return rc;
  if (batch == 0 || q_heads == 0 || parts == 0) return INTENT_HIP_OK;
  if (!decode_shape_ok(d, dv))
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "decode supports D = DV = 64 or 128 (got %lld, %lld)",
                static_cast<long long>(d), static_cast<long long>(dv));
  if (strides == nullptr || q == nullptr || partial_lse == nullptr || partial_output == nullptr ||
      (keys > 0 && (k == nullptr || v == nullptr)))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null pointer");
  if (keys > INT32_MAX / 2 || parts * split_size > INT32_MAX / 2 || batch * parts * kv_heads > INT32_MAX)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "extents too large");
  // strides: q [B,HQ,1,D], k [B,HK,K,D], v [B,HK,K,DV], partial_lse [B,HQ,P], partial_output [B,HQ,P,DV]
  const int64_t *qs = strides, *ks = strides + 4, *vs = strides + 8, *ls = strides + 12, *os = strides + 15;
  if (qs[3] != 1 || ks[3] != 1 || vs[3] != 1 || os[3] != 1)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "q, k, v and partial_output need unit inner stride");
  DecodeGeometry g{};
  g.q[0] = qs[0];
  g.q[1] = qs[1];
  g.q[2] = 1;
  const int64_t kr[3] = {ks[0], ks[2], ks[1]}, vr[3] = {vs[0], vs[2], vs[1]};
  if (keys > 0)
    if (int rc = rows_geometry(kr, vr, k, v, &g)) return rc;
  for (int i = 0; i < 3; ++i) {
    g.lse[i] = ls[i];
    g.out[i] = os[i];
  }
  g.out[3] = 1;
  DecodeSource src{};
  src.keys = static_cast<int>(keys);
  src.span = static_cast<int>(split_size);
  DecodeTarget dst{};
  dst.lse = partial_lse;
  dst.out = partial_output;
  return launch_partials(kVariantGroupedBf16, d, static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k),
                         static_cast<const uint16_t *>(v), kv_heads, head_group, parts, batch * parts * kv_heads, src,
                         dst, g, scale, stream);
}

extern "C" int intent_hip_dense_decode_workspace_bytes(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t keys,
                                                       int64_t dv, size_t *bytes) {
  if (bytes == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null output");
  if (batch < 0 || q_heads < 0 || kv_heads < 0 || keys < 0 || dv < 0)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  int64_t splits, span;
  decode_splits(batch * kv_heads, keys, &splits, &span);
  *bytes = state_layout(batch * q_heads, splits, dv).bytes;
  return INTENT_HIP_OK;
}

extern "C" int intent_hip_continuous_gqa_decode(const void *q, const void *k, const void *v, const uint8_t *valid_mask,
                                                void *out, int64_t batch, int64_t q_heads, int64_t kv_heads,
                                                int64_t head_group, int64_t keys, int64_t d, int64_t dv,
                                                const int64_t *strides, float scale, void *workspace,
                                                size_t workspace_bytes, void *stream) {
  if (batch < 0 || q_heads < 0 || kv_heads < 0 || keys < 0 || d < 0 || dv < 0)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (int rc = check_group(q_heads, kv_heads, head_group)) return rc;
  if (batch == 0 || q_heads == 0) return INTENT_HIP_OK;
  if (!decode_shape_ok(d, dv))
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "decode supports D = DV = 64 or 128 (got %lld, %lld)",
                static_cast<long long>(d), static_cast<long long>(dv));
  if (strides == nullptr || q == nullptr || out == nullptr ||
      (keys > 0 && (k == nullptr || v == nullptr || valid_mask == nullptr)))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null pointer");
  int64_t splits, span;
  decode_splits(batch * kv_heads, keys, &splits, &span);
  const StateLayout layout = state_layout(batch * q_heads, splits, dv);
  if (workspace == nullptr || workspace_bytes < layout.bytes || !aligned(workspace, 256))
    return fail(INTENT_HIP_ERR_WORKSPACE, "continuous decode needs %zu workspace bytes (256-byte aligned), got %zu",
                layout.bytes, workspace_bytes);
  if (keys > INT32_MAX / 2 || batch * splits * kv_heads > INT32_MAX || batch * q_heads > INT32_MAX)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "extents too large");
  // strides: q [B,HQ,D], k [B,K,HK,D], v [B,K,HK,DV], valid_mask [B,K,HK], output [B,HQ,DV]
  const int64_t *qs = strides, *ks = strides + 3, *vs = strides + 7, *ms = strides + 11, *os = strides + 14;
  if (qs[2] != 1 || ks[3] != 1 || vs[3] != 1 || os[2] != 1)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "q, k, v and output need unit inner stride");
  DecodeGeometry g{};
  g.q[0] = qs[0];
  g.q[1] = qs[1];
  g.q[2] = 1;
  if (keys > 0)
    if (int rc = rows_geometry(ks, vs, k, v, &g)) return rc;
  char *ws = static_cast<char *>(workspace);
  DecodeSource src{};
  src.keys = static_cast<int>(keys);
  src.span = static_cast<int>(span);
  src.mask = valid_mask;
  for (int i = 0; i < 3; ++i) src.mask_s[i] = ms[i];
  DecodeTarget dst{};
  dst.state_m = reinterpret_cast<float *>(ws);
  dst.state_den = reinterpret_cast<float *>(ws + layout.den);
  dst.state_acc = reinterpret_cast<float *>(ws + layout.acc);
  if (int rc = launch_partials(kVariantContinuous, d, static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k),
                               static_cast<const uint16_t *>(v), kv_heads, head_group, splits,
                               batch * splits * kv_heads, src, dst, g, scale, stream))
    return rc;
  return launch_merge(dv, layout, ws, batch * q_heads, q_heads, splits, nullptr, out, os[0], os[1], nullptr, nullptr,
                      nullptr, 0, 0, stream);
}

extern "C" int intent_hip_varlen_decode_workspace_bytes(int64_t sequences, int64_t q_heads, int64_t kv_heads,
                                                        int64_t max_blocks, int64_t dv, size_t *bytes) {
  if (bytes == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null output");
  if (sequences < 0 || q_heads < 0 || kv_heads < 0 || max_blocks < 0 || dv < 0)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  int64_t splits, span;
  decode_splits(sequences * kv_heads, max_blocks * kChunk, &splits, &span);
  *bytes = state_layout(sequences * q_heads, splits, dv).bytes;
  return INTENT_HIP_OK;
}

extern "C" int intent_hip_varlen_decode_sink(const void *q, const void *k, const void *v, const int32_t *cu_seqlens,
                                             const float *sink, void *out, float *block_logits, int64_t sequences,
                                             int64_t rows, int64_t q_heads, int64_t kv_heads, int64_t head_group,
                                             int64_t d, int64_t dv, int64_t max_blocks, const int64_t *strides,
                                             float scale, void *workspace, size_t workspace_bytes, void *stream) {
  if (sequences < 0 || rows < 0 || q_heads < 0 || kv_heads < 0 || d < 0 || dv < 0 || max_blocks < 0)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (int rc = check_group(q_heads, kv_heads, head_group)) return rc;
  if (sequences == 0 || q_heads == 0) return INTENT_HIP_OK;
  if (!decode_shape_ok(d, dv))
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "decode supports D = DV = 64 or 128 (got %lld, %lld)",
                static_cast<long long>(d), static_cast<long long>(dv));
  if (strides == nullptr || q == nullptr || out == nullptr || cu_seqlens == nullptr || sink == nullptr ||
      (max_blocks > 0 && block_logits == nullptr) || (rows > 0 && (k == nullptr || v == nullptr)))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null pointer");
  if (rows > INT32_MAX / 2 || max_blocks > (INT32_MAX / 2) / kChunk || sequences * q_heads > INT32_MAX)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "extents too large");
  int64_t splits, span;
  decode_splits(sequences * kv_heads, max_blocks * kChunk, &splits, &span);
  const StateLayout layout = state_layout(sequences * q_heads, splits, dv);
  if (workspace == nullptr || workspace_bytes < layout.bytes || !aligned(workspace, 256))
    return fail(INTENT_HIP_ERR_WORKSPACE, "packed decode needs %zu workspace bytes (256-byte aligned), got %zu",
                layout.bytes, workspace_bytes);
  if (sequences * splits * kv_heads > INT32_MAX) return fail(INTENT_HIP_ERR_UNSUPPORTED, "extents too large");
  // strides: q [B,HQ,D], k [U,HK,D], v [U,HK,DV], output [B,HQ,DV], block_logits [B,HQ,MAX_BLOCKS]
  const int64_t *qs = strides, *ks = strides + 3, *vs = strides + 6, *os = strides + 9, *bs = strides + 12;
  if (qs[2] != 1 || ks[2] != 1 || vs[2] != 1 || os[2] != 1)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "q, k, v and output need unit inner stride");
  DecodeGeometry g{};
  g.q[0] = qs[0];
  g.q[1] = qs[1];
  g.q[2] = 1;
  const int64_t kr[3] = {0, ks[0], ks[1]}, vr[3] = {0, vs[0], vs[1]};
  if (rows > 0)
    if (int rc = rows_geometry(kr, vr, k, v, &g)) return rc;
  char *ws = static_cast<char *>(workspace);
  DecodeSource src{};
  src.cu = cu_seqlens;
  src.rows = static_cast<int>(rows);
  src.keys = static_cast<int>(max_blocks * kChunk);
  src.span = static_cast<int>(span);
  DecodeTarget dst{};
  dst.state_m = reinterpret_cast<float *>(ws);
  dst.state_den = reinterpret_cast<float *>(ws + layout.den);
  dst.state_acc = reinterpret_cast<float *>(ws + layout.acc);
  dst.block_max = max_blocks > 0 ? block_logits : nullptr;
  for (int i = 0; i < 3; ++i) dst.bm[i] = bs[i];
  if (int rc = launch_partials(kVariantPackedSink, d, static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k),
                               static_cast<const uint16_t *>(v), kv_heads, head_group, splits,
                               sequences * splits * kv_heads, src, dst, g, scale, stream))
    return rc;
  return launch_merge(dv, layout, ws, sequences * q_heads, q_heads, splits, sink, out, os[0], os[1], dst.block_max, bs,
                      cu_seqlens, rows, max_blocks, stream);
}
