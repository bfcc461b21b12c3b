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
template <int D, int kG>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kG <= 4 ? 4 : 2))) void paged_decode_partials(
    const uint16_t *__restrict__ Q, const uint16_t *__restrict__ KC, const uint16_t *__restrict__ VC,
    const int32_t *__restrict__ page_offsets, const int32_t *__restrict__ page_indices,
    const int32_t *__restrict__ lengths, const int32_t *__restrict__ split_offsets, float *__restrict__ LSE,
    float *__restrict__ OUT, int kv_heads, int group, int splits, int64_t pages, int ps, int64_t positions,
    int page_size, DecodeGeometry g, float scale) {
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
  const int first = split_offsets[job];
  int64_t count = static_cast<int64_t>(split_offsets[job + 1]) - first;
  count = count < 0 ? 0 : (count > positions ? positions : count);
  const int tokens = static_cast<int>(count * ps);     // host checks positions * ps < 2^31
  const int64_t length = lengths[b], page_begin = page_offsets[b];
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
      int64_t position = first + flat / ps;
      position = position < 0 ? 0 : (position >= positions ? positions - 1 : position);
      const int offset = flat % ps;
      int64_t physical = page_indices[position];
      physical = physical < 0 ? 0 : (physical >= pages ? pages - 1 : physical);
      active = (position - page_begin) * page_size + offset < length;
      key_row = physical * g.k[0] + offset * g.k[1] + kh * g.k[2];
      row_s[wave][lane] = physical * g.v[0] + offset * g.v[1] + kh * g.v[2];
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
          if (r >= 0) kv[j] = __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const f16x8_t *>(KC + r + dim0)));
        }
        float v[kB][kG];
#pragma unroll
        for (int j = 0; j < kB; ++j)
#pragma unroll
          for (int gq = 0; gq < kG; ++gq) {
            float t = 0.0f;
            if (gq < group) {
              t = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, qr[gq].x), __builtin_bit_cast(f16x2_t, kv[j].x), t, false);
              t = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, qr[gq].y), __builtin_bit_cast(f16x2_t, kv[j].y), t, false);
              t = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, qr[gq].z), __builtin_bit_cast(f16x2_t, kv[j].z), t, false);
              t = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, qr[gq].w), __builtin_bit_cast(f16x2_t, kv[j].w), t, false);
            }
            v[j][gq] = t;
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
                float t = s[gq];
                t = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, qv.x), __builtin_bit_cast(f16x2_t, kv[c].x), t, false);
                t = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, qv.y), __builtin_bit_cast(f16x2_t, kv[c].y), t, false);
                t = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, qv.z), __builtin_bit_cast(f16x2_t, kv[c].z), t, false);
                t = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, qv.w), __builtin_bit_cast(f16x2_t, kv[c].w), t, false);
                s[gq] = t;
              }
            }
          }
        }
      }
      if (!__any(active)) continue;
    }
    valid = true;
    // Chunk summary as the definition forms it: weights against the chunk's own maximum, rounded
    // to f16 for P @ V; the chunk joins the running state with exp2 factors (left for the state,
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
        p_s[wave][gq][mine] = right * static_cast<float>(static_cast<_Float16>(p));
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
      f16x8_t vv[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int token = (base + j) * kTokensPerLoad + token_lane;
        vv[j] = f16x8_t{};
        if (token < chunk_tokens)
          vv[j] = __builtin_nontemporal_load(reinterpret_cast<const f16x8_t *>(VC + row_s[wave][token] + dim0));
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
    float *orow = OUT + b * g.out[0] + h * g.out[1] + split * g.out[2];
    orow[c] = any ? value * (1.0f / total) : 0.0f;
    if (c == 0) LSE[b * g.lse[0] + h * g.lse[1] + split * g.lse[2]] = any ? top + logf(total) * kLog2e : -INFINITY;
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

}  // namespace

template <int D>
const void *partials_kernel(int64_t group, const char **name) {
  if (group <= 4) {
    *name = D == 64 ? "paged_decode_partials<64,4>" : "paged_decode_partials<128,4>";
    return reinterpret_cast<const void *>(&paged_decode_partials<D, 4>);
  }
  if (group <= 8) {
    *name = D == 64 ? "paged_decode_partials<64,8>" : "paged_decode_partials<128,8>";
    return reinterpret_cast<const void *>(&paged_decode_partials<D, 8>);
  }
  *name = D == 64 ? "paged_decode_partials<64,16>" : "paged_decode_partials<128,16>";
  return reinterpret_cast<const void *>(&paged_decode_partials<D, 16>);
}

int decode_resources(int64_t which, int64_t d, int64_t group, IntentHipKernelResources *out) {
  if (which == 1)
    return describe_kernel(reinterpret_cast<const void *>(&splitk_reduce_f32_to_f16), "splitk_reduce_f32_to_f16",
                           64, out);
  const char *name = nullptr;
  const void *kernel = d == 64 ? partials_kernel<64>(group, &name) : partials_kernel<128>(group, &name);
  return describe_kernel(kernel, name, kThreads, out);
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
  const char *name = nullptr;
  const void *kernel = d == 64 ? partials_kernel<64>(head_group, &name) : partials_kernel<128>(head_group, &name);
  int kv = static_cast<int>(kv_heads), grp = static_cast<int>(head_group), spl = static_cast<int>(splits);
  int ps32 = static_cast<int>(ps), psize = static_cast<int>(page_size);
  void *args[] = {&Q, &K, &V, &page_offsets, &page_indices, &lengths, &split_offsets, &partial_lse, &partial_output,
                  &kv, &grp, &spl, &pages, &ps32, &positions, &psize, &g, &scale};
  const hipError_t rc = hipLaunchKernel(kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), args, 0,
                                        as_stream(stream));
  if (rc != hipSuccess) return launch_status(name);
  return INTENT_HIP_OK;
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
