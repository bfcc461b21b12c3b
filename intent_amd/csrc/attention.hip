// Fused attention forward (f16 in/out, f32 softmax and accumulation) for gfx950.
//
// Semantics: flash_attention_fwd (python/intent/examples/kernels/streaming/attention.py:428-466)
// with summarize_attention_chunk_f16 (:152-191), merge_attention_summaries (:82-114) and
// normalize_attention_summary (:417-425): scores s = (q . k) * (scale * log2 e) in f32, causal
// validity q_idx >= k_idx on absolute indices, masked scores -inf, maximum_num maxima,
// p = exp2(s - max) (approximate, flush-to-zero: v_exp_f32), P rounded to f16 before P @ V
// (f32 accumulation), output acc * rcp(den) (approximate: v_rcp_f32), cast to f16 (RNE).
// The key axis is folded in 64-key chunks; the running maximum replaces the chunk maximum
// before P is rounded (online softmax), which the 16-bit tolerance covers.
//
// Design (d = dv = 128):
//   * a workgroup owns 128 query rows of one (batch, head): 4 waves x 32 rows; key tiles of
//     64 keys stream through LDS in two stages (K: 16 KB, V^T: 16 KB per stage), so two
//     workgroups share a CU;
//   * scores are computed transposed, S^T = K Q^T (v_mfma_f32_32x32x16_f16, the wave's Q
//     fragments stay in registers): lane l then holds 16 scores of query l % 32 per 32-key
//     tile, so the running max/denominator of a query live in one lane pair (l, l ^ 32);
//   * the output is accumulated transposed as well, O^T = V^T P^T: lane l holds dv values of
//     query l % 32, so the online-softmax rescale of O is lane-local and P goes from the
//     score registers to the MFMA B operand without leaving registers;
//   * V^T lives in LDS with the keys of every 16-key slice permuted (bits 2 and 3 of the key
//     swapped), so the 8 keys a lane needs for one MFMA k-slice are one 16-byte read;
//   * causal: a workgroup visits key tiles up to its last query only, a wave skips tiles
//     beyond its own last query, and only tiles crossing the diagonal are masked; the
//     heaviest query blocks are dispatched first. All query blocks of one head share an
//     XCD (blocks of a head are 128 apart, a multiple of the 8 XCDs) and so its L2.
#include "common.hpp"

namespace intent_hip {
namespace {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kD = 128;
constexpr int kBQ = 128;     // query rows per workgroup
constexpr int kBK = 64;      // keys per tile
constexpr int kThreads = 256;
constexpr int kKChunks = kBK * kD / 8;      // 16-byte chunks of a K tile (row = key, 16 chunks)
constexpr int kVChunks = kD * kBK / 8;      // 16-byte chunks of a V^T tile (row = dv, 8 chunks)
constexpr int kStageChunks = kKChunks + kVChunks;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ int swizzle(int row) { return (row & 7) ^ ((row >> 3) & 1); }

__device__ __forceinline__ uint4 select(bool keep, uint4 v) {
  return make_uint4(keep ? v.x : 0u, keep ? v.y : 0u, keep ? v.z : 0u, keep ? v.w : 0u);
}

__device__ __forceinline__ uint32_t word(const uint4 &v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

struct Geometry {
  int64_t qs[4], ks[4], vs[4], os[4];  // element strides (batch, head, row, col)
};

__global__ __launch_bounds__(kThreads, 2) void attention_fwd_d128(const uint16_t *__restrict__ Q,
                                                                  const uint16_t *__restrict__ K,
                                                                  const uint16_t *__restrict__ V,
                                                                  uint16_t *__restrict__ O, int heads,
                                                                  int sq, int sk, Geometry g, float scale,
                                                                  int causal, int q_blocks) {
  __shared__ uint4 lds[2 * kStageChunks];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int bh_count = gridDim.x / q_blocks;
  const int qb = q_blocks - 1 - static_cast<int>(blockIdx.x) / bh_count;   // heaviest blocks first
  const int bh = static_cast<int>(blockIdx.x) % bh_count;
  const int b = bh / heads, h = bh % heads;
  const uint16_t *qbase = Q + b * g.qs[0] + h * g.qs[1];
  const uint16_t *kbase = K + b * g.ks[0] + h * g.ks[1];
  const uint16_t *vbase = V + b * g.vs[0] + h * g.vs[1];
  uint16_t *obase = O + b * g.os[0] + h * g.os[1];

  const int q0 = qb * kBQ;
  const int wq0 = q0 + wave * 32;             // this wave's first query row
  const int lane_q = wq0 + (lane & 31);       // the query row this lane tracks
  const int half = lane >> 5;

  // Q fragments (MFMA B operand of S^T): q = lane_q, d = 16 ks + 8 half + 0..7.
  f16x8_t qf[kD / 16];
  {
    const bool ok = lane_q < sq;
    const uint16_t *row = qbase + static_cast<int64_t>(ok ? lane_q : 0) * g.qs[2];
#pragma unroll
    for (int ks = 0; ks < kD / 16; ++ks)
      qf[ks] = __builtin_bit_cast(f16x8_t, select(ok, *reinterpret_cast<const uint4 *>(row + ks * 16 + half * 8)));
  }

  // Key range of this workgroup and of this wave.
  const int q_last_block = min(q0 + kBQ, sq) - 1;
  const int k_end = causal ? min(sk, q_last_block + 1) : sk;
  const int tiles = (k_end + kBK - 1) / kBK;
  const int wave_q_last = min(wq0 + 31, sq - 1);

  // Loader roles: waves 0-1 copy K (row = key, chunk kc), waves 2-3 copy V (8 keys x 8 dv
  // blocks) and transpose them into V^T rows.
  const bool loads_k = wave < 2;
  const int lt = tid & 127;
  const int k_chunk = lt & 15, k_row = lt >> 4;   // K: rows k_row + 8 i, chunk k_chunk
  const int v_kg = lt & 7, v_dc = lt >> 3;        // V: keys v_kg*8 + j, dv chunk v_dc (0..15)
  uint4 r[8];

  auto load = [&](int kt) {
    const int key0 = kt * kBK;
    if (loads_k) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int key = key0 + k_row + 8 * i;
        const bool ok = key < sk;
        r[i] = select(ok, *reinterpret_cast<const uint4 *>(kbase + static_cast<int64_t>(ok ? key : 0) * g.ks[2] +
                                                           k_chunk * 8));
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int key = key0 + v_kg * 8 + j;
        const bool ok = key < sk;
        r[j] = select(ok, *reinterpret_cast<const uint4 *>(vbase + static_cast<int64_t>(ok ? key : 0) * g.vs[2] +
                                                           v_dc * 8));
      }
    }
  };

  auto store = [&](int stage) {
    uint4 *sk_tile = lds + stage * kStageChunks;
    uint4 *sv_tile = sk_tile + kKChunks;
    if (loads_k) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int row = k_row + 8 * i;
        sk_tile[row * 16 + (k_chunk ^ swizzle(row))] = r[i];
      }
    } else {
      // r[j] word p = (dv = 2p, 2p + 1) at key v_kg*8 + j. V^T row dv gets the 8 keys, split
      // into two 4-key halves by the slice permutation (bits 2 and 3 of the key swapped).
      uint2 *sv2 = reinterpret_cast<uint2 *>(sv_tile);
      const int slice = v_kg >> 1;                         // 16-key slice of these keys
      const int pos_lo = slice * 16 + ((v_kg & 1) ? 4 : 0);   // keys +0..3 of this group
      const int pos_hi = pos_lo + 8;                          // keys +4..7
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        uint32_t even[4], odd[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t a = word(r[2 * q], p), c = word(r[2 * q + 1], p);
          even[q] = (a & 0xffffu) | (c << 16);
          odd[q] = (a >> 16) | (c & 0xffff0000u);
        }
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int dv = v_dc * 8 + 2 * p + e;
          const uint32_t *w = e ? odd : even;
          const int sw = swizzle(dv);
          // 16-byte chunk (pos / 8) of row dv, swizzled; 8-byte half (pos % 8) / 4.
          sv2[(dv * 8 + ((pos_lo >> 3) ^ sw)) * 2 + ((pos_lo & 7) >> 2)] = make_uint2(w[0], w[1]);
          sv2[(dv * 8 + ((pos_hi >> 3) ^ sw)) * 2 + ((pos_hi & 7) >> 2)] = make_uint2(w[2], w[3]);
        }
      }
    }
  };

  f32x16_t acc[4];   // O^T: dv tile mt (32 dv) x 32 queries
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[mt][e] = 0.0f;
  float row_max = -INFINITY;   // running maximum of valid scaled scores (exp2 domain)
  float row_den = 0.0f;        // this lane's share of the denominator
  const float factor = scale * kLog2e;
  const int frag_row = lane & 31;
  const int frag_swz = swizzle(frag_row);

  if (tiles > 0) {
    load(0);
    store(0);
  }
  __syncthreads();
  for (int kt = 0; kt < tiles; ++kt) {
    const bool more = kt + 1 < tiles;
    if (more) load(kt + 1);
    const int key0 = kt * kBK;
    const bool active = !causal || key0 <= wave_q_last;      // wave-uniform
    if (active && wq0 < sq) {
      const uint4 *sk_tile = lds + (kt & 1) * kStageChunks;
      const uint4 *sv_tile = sk_tile + kKChunks;
      // S^T for two 32-key tiles: s[st][e] is key 8 (e / 4) + 4 half + e % 4 of tile st.
      f32x16_t s[2];
#pragma unroll
      for (int st = 0; st < 2; ++st) {
#pragma unroll
        for (int e = 0; e < 16; ++e) s[st][e] = 0.0f;
        const int row = st * 32 + frag_row;
#pragma unroll
        for (int ks = 0; ks < kD / 16; ++ks) {
          const f16x8_t kf = __builtin_bit_cast(f16x8_t, sk_tile[row * 16 + ((ks * 2 + half) ^ frag_swz)]);
          s[st] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[ks], s[st], 0, 0, 0);
        }
      }
      // Scale, mask and this tile's maximum.
      const bool edge = causal ? (key0 + kBK - 1 > wq0) : false;
      const bool tail = key0 + kBK > sk;
      float tile_max = -INFINITY;
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float v = s[st][e] * factor;
          if (edge || tail) {
            const int key = key0 + st * 32 + 8 * (e >> 2) + 4 * half + (e & 3);
            const bool valid = key < sk && (!causal || key <= lane_q);
            v = valid ? v : -INFINITY;
          }
          s[st][e] = v;
          tile_max = fmaxf(tile_max, v);
        }
      tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32));
      const float new_max = fmaxf(row_max, tile_max);
      // A row with no valid key so far keeps max -inf; its weights are 0 and its scale 1.
      const bool any = new_max != -INFINITY;
      const float alpha = any ? __builtin_amdgcn_exp2f(row_max - new_max) : 1.0f;
      const float shift = any ? new_max : 0.0f;
      row_max = new_max;
      float tile_den = 0.0f;
      f16x8_t pf[4];   // P^T fragments: slice (16 keys) sl = 2 st + (e / 8), slot j = e % 8
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float p = __builtin_amdgcn_exp2f(s[st][e] - shift);
          tile_den += p;
          pf[st * 2 + (e >> 3)][e & 7] = static_cast<_Float16>(p);
        }
      row_den = row_den * alpha + tile_den;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[mt][e] *= alpha;
      // O^T += V^T P^T: A = V^T rows dv = 32 mt + (lane & 31), keys of slice sl in slot order.
#pragma unroll
      for (int sl = 0; sl < 4; ++sl)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          const int dv = mt * 32 + frag_row;
          const f16x8_t vf = __builtin_bit_cast(f16x8_t, sv_tile[dv * 8 + ((sl * 2 + half) ^ frag_swz)]);
          acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[sl], acc[mt], 0, 0, 0);
        }
    }
    if (more) store((kt + 1) & 1);
    __syncthreads();
  }

  // Normalise and store: acc[mt][4 gq + e] is dv = 32 mt + 8 gq + 4 half + e of query lane_q.
  if (lane_q >= sq) return;
  const float den = row_den + __shfl_xor(row_den, 32);
  const bool valid = row_max != -INFINITY;
  const float inv = valid ? __builtin_amdgcn_rcpf(den) : 0.0f;
  uint16_t *orow = obase + static_cast<int64_t>(lane_q) * g.os[2];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      uint32_t w0 = static_cast<uint32_t>(from_f32<f16_t>(acc[mt][4 * gq] * inv).bits) |
                    (static_cast<uint32_t>(from_f32<f16_t>(acc[mt][4 * gq + 1] * inv).bits) << 16);
      uint32_t w1 = static_cast<uint32_t>(from_f32<f16_t>(acc[mt][4 * gq + 2] * inv).bits) |
                    (static_cast<uint32_t>(from_f32<f16_t>(acc[mt][4 * gq + 3] * inv).bits) << 16);
      *reinterpret_cast<uint2 *>(orow + mt * 32 + 8 * gq + 4 * half) = make_uint2(w0, w1);
    }
}

}  // namespace

int attention_resources(int64_t sq, int64_t d, IntentHipKernelResources *out) {
  (void)sq;
  (void)d;
  return describe_kernel(reinterpret_cast<const void *>(&attention_fwd_d128), "attention_fwd_d128", kThreads, out);
}

}  // namespace intent_hip

using namespace intent_hip;

extern "C" int intent_hip_attention_fwd_f16(const void *q, const void *k, const void *v, void *o, int64_t batch,
                                            int64_t heads, int64_t sq, int64_t sk, int64_t d, int64_t dv,
                                            const int64_t *strides, float scale, int causal, void *stream) {
  if (batch < 0 || heads < 0 || sq < 0 || sk < 0 || d < 0 || dv < 0)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (batch == 0 || heads == 0 || sq == 0 || dv == 0) return INTENT_HIP_OK;
  if (d != kD || dv != kD)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "attention kernel supports head dimension 128 (got d=%lld, dv=%lld)",
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
  const int64_t blocks = batch * heads * q_blocks;
  if (blocks > INT32_MAX) return fail(INTENT_HIP_ERR_UNSUPPORTED, "too many attention workgroups");
  attention_fwd_d128<<<dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, as_stream(stream)>>>(
      static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k), static_cast<const uint16_t *>(v),
      static_cast<uint16_t *>(o), static_cast<int>(heads), static_cast<int>(sq), static_cast<int>(sk), g, scale,
      causal ? 1 : 0, q_blocks);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("attention_fwd_d128");
  return INTENT_HIP_OK;
}
