// bf16 GEMM, C = bf16(A @ B) with f32 accumulation, for gfx950 (CDNA4).
//
// Semantics: bf16_gemm (python/intent/examples/kernels/contraction/gemm.py:76-92):
// accumulator = matmul(a, b, acc_dtype=f32); c = cast(accumulator, bf16) (round to
// nearest even). A [M,K], B [K,N], C [M,N], row-major with row strides lda/ldb/ldc.
//
// Design (fast path):
//   * workgroup tile 256 x 256, 8 waves in 2 x 4, each wave 128 x 64 = 4 x 2 tiles of
//     v_mfma_f32_32x32x16_bf16 (128 accumulator registers per lane, so two waves share
//     each SIMD);
//   * interior tiles with K % 32 == 0 (gemm_tile_dma) stream A and B into LDS with
//     global_load_lds (five 32 KB stages) and read B fragments with transposing LDS reads;
//     the two waves of a SIMD alternate between their MFMA cluster and their LDS reads
//     (ping-pong), so the matrix pipe is fed while the other wave waits on LDS;
//   * other tiles (gemm_tile) use K step 64 and two register-staged LDS stages
//     (2 x 64 KB): the next K step's global loads are in flight while the current one is
//     consumed;
//   * MFMA operands need 8 consecutive k per lane. A rows are k-contiguous already;
//     in gemm_tile B is [K,N], so each thread of waves 4-7 loads an 8 (k) x 8 (n) block,
//     transposes it in registers and stores n-rows of 8 k into LDS ("Bt", k-contiguous);
//     waves 0-3 copy A;
//   * gemm_tile's LDS tiles are rows of 8 16-byte chunks; chunk c of row r is stored at
//     c ^ ((r & 7) ^ ((r >> 3) & 1)), so the 16-byte fragment reads of 16 consecutive
//     rows (one LDS cycle) hit distinct banks;
//   * the MFMA is issued as D = Bt_frag x A_frag, i.e. the transposed product, so each
//     lane ends with 4 consecutive output columns of one output row per register
//     quad and writes them as one 8-byte store;
//   * tiles are walked in groups of 2 tile rows, column by column, in dispatch order: the
//     tiles resident at one time share A row panels and B column panels, across XCDs
//     through the MALL and within each XCD through its L2.
// Shapes the fast path cannot take (K or N not a multiple of 8, unaligned rows) use a
// simple LDS-tiled f32 FMA kernel.
#include "common.hpp"

namespace intent_hip {
namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// Operand element type: __bf16 (bf16_gemm) or _Float16 (gemm). Fragments of 8 elements feed
// v_mfma_f32_32x32x16_{bf16,f16}; results are stored 4 at a time.
template <typename E> struct Elem;
template <> struct Elem<__bf16> {
  typedef __bf16 x8 __attribute__((ext_vector_type(8)));
  typedef __bf16 x4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ f32x16_t mma(x8 a, x8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Elem<_Float16> {
  typedef _Float16 x8 __attribute__((ext_vector_type(8)));
  typedef _Float16 x4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ f32x16_t mma(x8 a, x8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// Epilogue activation on the f32 accumulator: 0 = none, 1 = ReLU as I.maximum(acc, 0.0)
// (NaN propagates; -0 and +0 give +0).
template <int kAct>
__device__ __forceinline__ float activate(float v) {
  if constexpr (kAct == 1) return v != v ? v : (v > 0.0f ? v : 0.0f);
  return v;
}

template <typename E, int kAct>
__device__ __forceinline__ typename Elem<E>::x4 pack4(float a, float b, float c, float d) {
  typename Elem<E>::x4 r;
  r[0] = static_cast<E>(activate<kAct>(a));
  r[1] = static_cast<E>(activate<kAct>(b));
  r[2] = static_cast<E>(activate<kAct>(c));
  r[3] = static_cast<E>(activate<kAct>(d));
  return r;
}

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kThreads = 512;
constexpr int kChunksA = kBM * kBK / 8;          // 16-byte chunks of one A stage
constexpr int kStageChunks = (kBM + kBN) * kBK / 8;
constexpr int kGroupM = 2;

__device__ __forceinline__ int swizzle(int row) { return (row & 7) ^ ((row >> 3) & 1); }

template <typename E>
__device__ __forceinline__ float element_to_f32(uint16_t bits) { return static_cast<float>(__builtin_bit_cast(E, bits)); }
template <typename E>
__device__ __forceinline__ uint16_t f32_to_element(float v) { return __builtin_bit_cast(uint16_t, static_cast<E>(v)); }

__device__ __forceinline__ uint32_t word(const uint4 &v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// Component-wise select (a whole-struct select is lowered through scratch memory).
__device__ __forceinline__ uint4 select(bool keep, uint4 v) {
  return make_uint4(keep ? v.x : 0u, keep ? v.y : 0u, keep ? v.z : 0u, keep ? v.w : 0u);
}

// Epilogues: quad(i, n, a, b, c, d) receives the f32 accumulators of output row i, columns n .. n+3
// (n a multiple of 4); one(i, n, a) a single element (the general-shape kernel).
// gemm / bf16_gemm: act(acc) rounded to E.
template <typename E, int kAct>
struct CastStore {
  uint16_t *C;
  int64_t ldc;
  __device__ __forceinline__ void quad(int i, int n, float a, float b, float c, float d) const {
    *reinterpret_cast<typename Elem<E>::x4 *>(C + static_cast<int64_t>(i) * ldc + n) = pack4<E, kAct>(a, b, c, d);
  }
  __device__ __forceinline__ void one(int i, int n, float a) const {
    C[static_cast<int64_t>(i) * ldc + n] = f32_to_element<E>(activate<kAct>(a));
  }
};

// quantized_gemm (contraction/gemm.py:95-121), each step an f32 operation as written there:
// v = maximum(acc + bias[n], 0) (NaN propagates), v = v + residual[i][n], v = v / scale[n] (IEEE
// division), v = minimum(maximum(v, -128), 127), then the cast to i8, which truncates toward
// zero. NaN is an illegal cast input; it gives 0 here.
struct QuantizeStore {
  const float *bias;
  const uint16_t *residual;   // f16 [M, N]
  int64_t ldr;
  const float *scale;
  int8_t *out;
  int64_t ldo;
  __device__ __forceinline__ static int32_t quantize(float acc, float bias, float residual, float scale) {
    float v = acc + bias;
    v = v != v ? v : (v > 0.0f ? v : 0.0f);
    v = v + residual;
    v = __fdiv_rn(v, scale);
    v = v != v ? v : (v < -128.0f ? -128.0f : (v > 127.0f ? 127.0f : v));
    return v != v ? 0 : static_cast<int32_t>(v);
  }
  __device__ __forceinline__ float residual_at(int i, int n) const {
    return element_to_f32<_Float16>(residual[static_cast<int64_t>(i) * ldr + n]);
  }
  __device__ __forceinline__ void quad(int i, int n, float a, float b, float c, float d) const {
    const uint2 r = *reinterpret_cast<const uint2 *>(residual + static_cast<int64_t>(i) * ldr + n);
    const float r0 = element_to_f32<_Float16>(static_cast<uint16_t>(r.x)), r1 = element_to_f32<_Float16>(static_cast<uint16_t>(r.x >> 16));
    const float r2 = element_to_f32<_Float16>(static_cast<uint16_t>(r.y)), r3 = element_to_f32<_Float16>(static_cast<uint16_t>(r.y >> 16));
    const uint32_t q = (static_cast<uint32_t>(quantize(a, bias[n], r0, scale[n])) & 0xffu) |
                       ((static_cast<uint32_t>(quantize(b, bias[n + 1], r1, scale[n + 1])) & 0xffu) << 8) |
                       ((static_cast<uint32_t>(quantize(c, bias[n + 2], r2, scale[n + 2])) & 0xffu) << 16) |
                       (static_cast<uint32_t>(quantize(d, bias[n + 3], r3, scale[n + 3])) << 24);
    *reinterpret_cast<uint32_t *>(out + static_cast<int64_t>(i) * ldo + n) = q;
  }
  __device__ __forceinline__ void one(int i, int n, float a) const {
    out[static_cast<int64_t>(i) * ldo + n] = static_cast<int8_t>(quantize(a, bias[n], residual_at(i, n), scale[n]));
  }
};

// Tile order: groups of kGroupM tile rows walked column by column, in dispatch order (the 8 XCDs
// take consecutive workgroups round-robin). At 8192^3 the 256 resident tiles then span 8 tile
// rows and all columns: each XCD holds 4 rows x 8 columns of them, and every A and B panel is
// read by several XCDs at nearly the same time, which the MALL serves once. Measured against
// other orders (interleaved, 8192^3 bf16): 0.899 ms here; 0.943 ms with XCD-contiguous runs of
// 8-row groups; 1.06 / 1.37 ms with 16 / 32-row groups.
__device__ __forceinline__ void tile_of_block(int block, int tiles_m, int tiles_n, int &tm, int &tn) {
  const int t = block;
  const int per_group = kGroupM * tiles_n;
  const int group = t / per_group;
  const int first_m = group * kGroupM;
  const int rows_in_group = min(tiles_m - first_m, kGroupM);
  const int in_group = t - group * per_group;
  tm = first_m + in_group % rows_in_group;
  tn = in_group / rows_in_group;
}

template <typename E, typename Epi, bool kEdge>
__device__ __forceinline__ void gemm_tile(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
                                          const Epi &ep, int M, int N, int K, int64_t lda, int64_t ldb, int m0,
                                          int n0, uint4 *lds) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;   // wave tile: rows wm*128..+128, cols wn*64..+64

  // Loader roles (wave-uniform). Waves 0-3 copy the A tile: rows a_row + 32 i, 16-byte
  // chunk a_chunk (8 k). Waves 4-7 copy the B tile: k rows b_kg * 8 + j, n chunk b_nc
  // (8 n), transposed in registers into Bt rows b_nc * 8 + m (8 k each).
  const bool loads_a = wave < 4;
  const int lt = tid & 255;
  const int a_chunk = lt & 7, a_row = lt >> 3;
  const int b_kg = lt & 7, b_nc = lt >> 3;
  uint4 r[8];

  auto load = [&](int k0) {
    if (loads_a) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int row = m0 + a_row + 32 * i;
        const int col = k0 + a_chunk * 8;
        if (!kEdge) {
          r[i] = *reinterpret_cast<const uint4 *>(A + static_cast<int64_t>(row) * lda + col);
        } else {
          const bool ok = row < M && col < K;
          const uint16_t *p = A + static_cast<int64_t>(ok ? row : 0) * lda + (ok ? col : 0);
          r[i] = select(ok, *reinterpret_cast<const uint4 *>(p));
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int krow = k0 + b_kg * 8 + j;
        const int col = n0 + b_nc * 8;
        if (!kEdge) {
          r[j] = *reinterpret_cast<const uint4 *>(B + static_cast<int64_t>(krow) * ldb + col);
        } else {
          const bool ok = krow < K && col < N;
          const uint16_t *p = B + static_cast<int64_t>(ok ? krow : 0) * ldb + (ok ? col : 0);
          r[j] = select(ok, *reinterpret_cast<const uint4 *>(p));
        }
      }
    }
  };

  auto store = [&](int stage) {
    uint4 *sa = lds + stage * kStageChunks;
    uint4 *sb = sa + kChunksA;
    if (loads_a) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int row = a_row + 32 * i;
        sa[row * 8 + (a_chunk ^ swizzle(row))] = r[i];
      }
    } else {
      // r[j] word p holds (n = 2p, n = 2p + 1) at k = j: gather the 8 k of each n.
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        uint32_t even[4], odd[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t k_lo = word(r[2 * q], p), k_hi = word(r[2 * q + 1], p);
          even[q] = (k_lo & 0xffffu) | (k_hi << 16);
          odd[q] = (k_lo >> 16) | (k_hi & 0xffff0000u);
        }
        const int n_even = b_nc * 8 + 2 * p, n_odd = n_even + 1;
        sb[n_even * 8 + (b_kg ^ swizzle(n_even))] = make_uint4(even[0], even[1], even[2], even[3]);
        sb[n_odd * 8 + (b_kg ^ swizzle(n_odd))] = make_uint4(odd[0], odd[1], odd[2], odd[3]);
      }
    }
  };

  f32x16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // Fragment rows of this lane: the swizzle depends only on the lane (rows differ by 32s).
  const int frag_row = lane & 31;
  const int frag_swz = swizzle(frag_row);
  const int frag_half = lane >> 5;

  auto compute = [&](int stage) {
    const uint4 *sa = lds + stage * kStageChunks;
    const uint4 *sb = sa + kChunksA;
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      const int chunk = (kk * 2 + frag_half) ^ frag_swz;
      typedef typename Elem<E>::x8 x8;
      x8 af[4], bf[2];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        af[t] = __builtin_bit_cast(x8, sa[(wm * 128 + t * 32 + frag_row) * 8 + chunk]);
#pragma unroll
      for (int t = 0; t < 2; ++t)
        bf[t] = __builtin_bit_cast(x8, sb[(wn * 64 + t * 32 + frag_row) * 8 + chunk]);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          acc[mt][nt] = Elem<E>::mma(bf[nt], af[mt], acc[mt][nt]);
    }
  };

  const int k_tiles = (K + kBK - 1) / kBK;
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < k_tiles; ++kt) {
    const bool more = kt + 1 < k_tiles;
    if (more) load((kt + 1) * kBK);
    compute(kt & 1);
    if (more) store((kt + 1) & 1);
    __syncthreads();
  }

  // Epilogue: acc[mt][nt][4g + e] is C[i][n] with i = the A fragment's row (lane & 31) and
  // n = 8g + 4 * (lane >> 5) + e within the 32-column tile; 4 consecutive n -> one 8-byte store.
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int i = m0 + wm * 128 + mt * 32 + frag_row;
    if (kEdge && i >= M) continue;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn * 64 + nt * 32 + 8 * g + 4 * frag_half;
        if (kEdge && n >= N) continue;
        const f32x16_t &v = acc[mt][nt];
        ep.quad(i, n, v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]);
      }
    }
  }
}

// ---------------------------------------------------------------- interior tiles: LDS-DMA pipeline
// K step 32, five LDS stages of 32 KB (160 KB): up to three later tiles are in flight
// (global_load_lds_dwordx4 writes them straight into LDS, no registers) while tile kt is multiplied. A stage holds A [256 m][32 k]
// (rows of 4 16-byte chunks, chunk c of row r at c ^ ((r >> 2) & 3), which spreads the fragment
// reads of 16 consecutive rows over the 64 LDS banks) and B in its natural
// [32 k][256 n] layout (rows of 32 chunks, chunk c of row k at c ^ 4 (k & 3), so the transposing
// reads of 4 consecutive k rows land on 4 disjoint groups of 4 chunks). B fragments are read
// with ds_read_b64_tr_b16: in each 16-lane group, lane i, slot j receives element i % 4 of the
// 8-byte segment addressed by lane 4 j + i / 4, so lane i addressing B[k0 + i/4][n0 + 4 (i % 4)]
// yields B[k0 .. k0+3][n0 + i], the 4 consecutive k of one n the MFMA operand needs.
constexpr int kDmaBK = 32;
constexpr int kDmaStages = 5;
constexpr int kDmaChunksA = kBM * kDmaBK / 8;            // 1024
constexpr int kDmaStageChunks = (kBM + kBN) * kDmaBK / 8; // 2048 (32 KB)

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
typedef __attribute__((address_space(3))) void lds_void_t;

// s_waitcnt with only the vector-memory counter constrained (vmcnt <= n), and with only the LDS
// counter constrained (lgkmcnt == 0).
#define INTENT_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt((((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8)))
#define INTENT_WAIT_LGKMCNT0() __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4))

// Workgroup barrier of the DMA loop: s_barrier with an acquire fence (later LDS reads stay below
// it) and no release fence. A release fence would wait for every DMA in flight (they are LDS
// writes); DMA completion is awaited explicitly with vmcnt before the barrier instead. The
// scheduling barriers keep each MFMA cluster on its side of the s_barrier.
__device__ __forceinline__ void dma_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  __builtin_amdgcn_sched_barrier(0);
}

template <typename E, typename Epi>
__device__ __forceinline__ void gemm_tile_dma(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
                                              const Epi &ep, int K, int64_t lda, int64_t ldb, int m0, int n0,
                                              uint4 *lds) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;

  // Each wave issues 2 A and 2 B DMA instructions (1 KB each) per K tile. The global chunk a lane
  // fetches is the one its LDS slot (base + 16 * lane) must hold under the swizzle.
  const uint16_t *a_src[2];
  const uint16_t *b_src[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int pa = (wave * 2 + i) * 64 + lane;      // A chunk slot: row pa / 4, physical chunk pa % 4
    const int ra = pa >> 2, ca = (pa & 3) ^ ((ra >> 2) & 3);
    a_src[i] = A + static_cast<int64_t>(m0 + ra) * lda + ca * 8;
    const int pb = (wave * 2 + i) * 64 + lane;      // B chunk slot: row pb / 32, physical chunk pb % 32
    const int kb = pb >> 5, cb = (pb & 31) ^ (4 * (kb & 3));
    b_src[i] = B + static_cast<int64_t>(kb) * ldb + n0 + cb * 8;
  }
  auto issue = [&](int kt) {
    uint4 *stage = lds + (kt % kDmaStages) * kDmaStageChunks;
    const int k0 = kt * kDmaBK;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      __builtin_amdgcn_global_load_lds(a_src[i] + k0, (lds_void_t *)(stage + (wave * 2 + i) * 64), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(b_src[i] + static_cast<int64_t>(k0) * ldb,
                                       (lds_void_t *)(stage + kDmaChunksA + (wave * 2 + i) * 64), 16, 0, 0);
    }
  };

  f32x16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int frag_row = lane & 31;
  const int half = lane >> 5;
  const int a_swz = (frag_row >> 2) & 3;
  // B transposed-read address of this lane within a 32 x 32 (k x n) block: group g = lane / 16,
  // source role i = lane % 16 -> k = 8 (g / 2) + i / 4 (+4 for the second read), n = 16 (g % 2) + 4 (i % 4).
  const int g16 = lane >> 4, i16 = lane & 15;
  const int b_k = 8 * (g16 >> 1) + (i16 >> 2);
  const int b_n = 16 * (g16 & 1) + 4 * (i16 & 3);

  // Ping-pong schedule. Waves 0-3 and 4-7 share the four SIMDs (one of each per SIMD). Waves 4-7
  // run one barrier behind, so between two barriers one wave of each SIMD issues its MFMA cluster
  // (M) while the other reads its fragments from LDS and issues its DMA (R):
  //   waves 0-3: b0 |   R0 b M0 b R1 b M1 b ... M(last) b | b
  //   waves 4-7: b0 | b R0 b M0 b R1 b ... M(last) b
  // Every wave executes 2 + 2 * k_tiles barriers. Before the barrier that opens the interval in
  // which waves 0-3 read tile t, every wave has waited for its own DMA of tile t. The DMA of tile
  // t + S - 1 overwrites stage (t - 1) % S, whose reads every wave completed (lgkmcnt 0) before an
  // earlier barrier.
  const bool lag = wave >= 4;
  const int k_tiles = K / kDmaBK;
#pragma unroll
  for (int kt = 0; kt < kDmaStages - 1; ++kt)
    if (kt < k_tiles) issue(kt);
  auto wait_tile = [&](int t) {   // this wave's DMA of tile t complete; later tiles may stay in flight
    const int later = min(k_tiles - 1 - t, kDmaStages - 2);
    if (later >= 3) INTENT_WAIT_VMCNT(12);
    else if (later == 2) INTENT_WAIT_VMCNT(8);
    else if (later == 1) INTENT_WAIT_VMCNT(4);
    else INTENT_WAIT_VMCNT(0);
  };
  wait_tile(0);
  dma_barrier();
  if (lag) dma_barrier();
  typedef typename Elem<E>::x8 x8;
  x8 af[2][4], bf[2][2];
  for (int kt = 0; kt < k_tiles; ++kt) {
    const uint4 *sa = lds + (kt % kDmaStages) * kDmaStageChunks;
    const uint16_t *sb = reinterpret_cast<const uint16_t *>(sa + kDmaChunksA);
#pragma unroll
    for (int kk = 0; kk < kDmaBK / 16; ++kk) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        af[kk][t] = __builtin_bit_cast(x8, sa[(wm * 128 + t * 32 + frag_row) * 4 + ((kk * 2 + half) ^ a_swz)]);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        i16x4_t parts[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int k = kk * 16 + b_k + 4 * r;
          const int n = wn * 64 + t * 32 + b_n;
          const int chunk = (n >> 3) ^ (4 * (k & 3));
          parts[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(sb + k * kBN + chunk * 8 + (n & 7)));
        }
        bf[kk][t] = __builtin_bit_cast(x8, parts);
      }
    }
    if (kt + kDmaStages - 1 < k_tiles) issue(kt + kDmaStages - 1);
    if (lag) wait_tile(kt + 1);
    INTENT_WAIT_LGKMCNT0();
    dma_barrier();
#pragma unroll
    for (int kk = 0; kk < kDmaBK / 16; ++kk)
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          acc[mt][nt] = Elem<E>::mma(bf[kk][nt], af[kk][mt], acc[mt][nt]);
    if (!lag) wait_tile(kt + 1);
    dma_barrier();
  }
  if (!lag) dma_barrier();

#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int i = m0 + wm * 128 + mt * 32 + frag_row;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn * 64 + nt * 32 + 8 * g + 4 * half;
        const f32x16_t &v = acc[mt][nt];
        ep.quad(i, n, v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]);
      }
  }
}

template <typename E, typename Epi>
__global__ __launch_bounds__(kThreads, 1) void gemm_mfma(const uint16_t *__restrict__ A,
                                                              const uint16_t *__restrict__ B, Epi ep, int M,
                                                              int N, int K, int64_t lda, int64_t ldb, int tiles_m,
                                                              int tiles_n) {
  __shared__ uint4 lds[2 * kStageChunks > kDmaStages * kDmaStageChunks ? 2 * kStageChunks : kDmaStages * kDmaStageChunks];
  int tm, tn;
  tile_of_block(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * kBM, n0 = tn * kBN;
  const bool interior = m0 + kBM <= M && n0 + kBN <= N;
  if (interior && (K % kDmaBK) == 0)
    gemm_tile_dma<E, Epi>(A, B, ep, K, lda, ldb, m0, n0, lds);
  else if (interior && (K % kBK) == 0)
    gemm_tile<E, Epi, false>(A, B, ep, M, N, K, lda, ldb, m0, n0, lds);
  else
    gemm_tile<E, Epi, true>(A, B, ep, M, N, K, lda, ldb, m0, n0, lds);
}

// ---------------------------------------------------------------- general-shape fallback
// 64 x 64 output tile per 256 threads (4 x 4 per thread), K in steps of 16 through LDS,
// f32 fused multiply-add in increasing k.
constexpr int kFT = 64, kFK = 16;

template <typename E, typename Epi>
__global__ __launch_bounds__(256) void gemm_simple(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
                                                        Epi ep, int M, int N, int K, int64_t lda, int64_t ldb) {
  __shared__ float sa[kFK][kFT + 1];
  __shared__ float sb[kFK][kFT + 1];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int m0 = blockIdx.y * kFT, n0 = blockIdx.x * kFT;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += kFK) {
    for (int e = threadIdx.x; e < kFT * kFK; e += 256) {
      const int r = e / kFK, kc = e % kFK;
      const int gm = m0 + r, gk = k0 + kc;
      sa[kc][r] = (gm < M && gk < K) ? element_to_f32<E>(A[static_cast<int64_t>(gm) * lda + gk]) : 0.0f;
      const int kr = e / kFT, nc = e % kFT;
      const int gk2 = k0 + kr, gn = n0 + nc;
      sb[kr][nc] = (gk2 < K && gn < N) ? element_to_f32<E>(B[static_cast<int64_t>(gk2) * ldb + gn]) : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kc = 0; kc < kFK; ++kc)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(sa[kc][ty * 4 + i], sb[kc][tx * 4 + j], acc[i][j]);
    __syncthreads();
  }
  for (int i = 0; i < 4; ++i) {
    const int gm = m0 + ty * 4 + i;
    if (gm >= M) continue;
    for (int j = 0; j < 4; ++j) {
      const int gn = n0 + tx * 4 + j;
      if (gn < N) ep.one(gm, gn, acc[i][j]);
    }
  }
}

bool fast_path(const void *a, const void *b, const void *c, int64_t n, int64_t k, int64_t lda, int64_t ldb,
               int64_t ldc) {
  return k % 8 == 0 && n % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 && ldc % 4 == 0 && aligned(a, 16) &&
         aligned(b, 16) && aligned(c, 8);
}

}  // namespace

int quantized_gemm_resources(IntentHipKernelResources *out) {
  return describe_kernel(reinterpret_cast<const void *>(&gemm_mfma<_Float16, QuantizeStore>), "gemm_mfma<f16,quantize>",
                         kThreads, out);
}

int gemm_resources(int dtype, int64_t m, int64_t n, IntentHipKernelResources *out) {
  (void)m;
  (void)n;
  if (dtype == INTENT_HIP_F16)
    return describe_kernel(reinterpret_cast<const void *>(&gemm_mfma<_Float16, CastStore<_Float16, 0>>), "gemm_mfma<f16>",
                           kThreads, out);
  return describe_kernel(reinterpret_cast<const void *>(&gemm_mfma<__bf16, CastStore<__bf16, 0>>), "gemm_mfma<bf16>",
                         kThreads, out);
}

namespace {

// The MFMA kernel when `fast` (the operand shape and layout it takes), else the general one.
template <typename E, typename Epi>
int launch_epilogue(const uint16_t *A, const uint16_t *B, const Epi &ep, int64_t m, int64_t n, int64_t k, int64_t lda,
                    int64_t ldb, bool fast, hipStream_t s) {
  if (k > 0 && fast) {
    const int tiles_m = static_cast<int>((m + kBM - 1) / kBM), tiles_n = static_cast<int>((n + kBN - 1) / kBN);
    gemm_mfma<E, Epi><<<dim3(tiles_m * tiles_n), dim3(kThreads), 0, s>>>(
        A, B, ep, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k), lda, ldb, tiles_m, tiles_n);
    if (hipPeekAtLastError() != hipSuccess) return launch_status("gemm_mfma");
    return INTENT_HIP_OK;
  }
  const dim3 grid(static_cast<unsigned>((n + kFT - 1) / kFT), static_cast<unsigned>((m + kFT - 1) / kFT));
  gemm_simple<E, Epi><<<grid, dim3(256), 0, s>>>(A, B, ep, static_cast<int>(m), static_cast<int>(n),
                                                 static_cast<int>(k), lda, ldb);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("gemm_simple");
  return INTENT_HIP_OK;
}

template <typename E, int kAct>
int launch_gemm(const void *a, const void *b, void *c, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb,
                int64_t ldc, void *stream) {
  if (m < 0 || n < 0 || k < 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (m > INT32_MAX / 2 || n > INT32_MAX / 2 || k > INT32_MAX / 2)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "GEMM extents must stay below 2^30");
  if (m == 0 || n == 0) return INTENT_HIP_OK;
  if (a == nullptr || b == nullptr || c == nullptr) {
    if (k > 0 || c == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null tensor pointer");
  }
  if (lda < (m > 1 ? k : 0) || ldb < (k > 1 ? n : 0) || ldc < (m > 1 ? n : 0))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "row stride smaller than the row length");
  const hipStream_t s = as_stream(stream);
  const auto *A = static_cast<const uint16_t *>(a);
  const auto *B = static_cast<const uint16_t *>(b);
  const CastStore<E, kAct> ep{static_cast<uint16_t *>(c), ldc};
  return launch_epilogue<E>(A, B, ep, m, n, k, lda, ldb, fast_path(a, b, c, n, k, lda, ldb, ldc), s);
}

}  // namespace
}  // namespace intent_hip

using namespace intent_hip;

extern "C" int intent_hip_gemm_bf16(const void *a, const void *b, void *c, int64_t m, int64_t n, int64_t k,
                                    int64_t lda, int64_t ldb, int64_t ldc, void *stream) {
  return launch_gemm<__bf16, 0>(a, b, c, m, n, k, lda, ldb, ldc, stream);
}

extern "C" int intent_hip_gemm(int dtype, int activation, const void *a, const void *b, void *c, int64_t m, int64_t n,
                               int64_t k, int64_t lda, int64_t ldb, int64_t ldc, void *stream) {
  if (activation != 0 && activation != 1)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "activation code %d (0 = none, 1 = relu)", activation);
  if (dtype == INTENT_HIP_F16)
    return activation ? launch_gemm<_Float16, 1>(a, b, c, m, n, k, lda, ldb, ldc, stream)
                      : launch_gemm<_Float16, 0>(a, b, c, m, n, k, lda, ldb, ldc, stream);
  if (dtype == INTENT_HIP_BF16)
    return activation ? launch_gemm<__bf16, 1>(a, b, c, m, n, k, lda, ldb, ldc, stream)
                      : launch_gemm<__bf16, 0>(a, b, c, m, n, k, lda, ldb, ldc, stream);
  return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "16-bit GEMM dtype code %d (1 = f16, 2 = bf16)", dtype);
}

extern "C" int intent_hip_quantized_gemm(const void *a, const void *b, const float *bias, const void *residual,
                                         const float *output_scale, void *out, int64_t m, int64_t n, int64_t k,
                                         int64_t lda, int64_t ldb, int64_t ldr, int64_t ldo, void *stream) {
  if (m < 0 || n < 0 || k < 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (m > INT32_MAX / 2 || n > INT32_MAX / 2 || k > INT32_MAX / 2)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "GEMM extents must stay below 2^30");
  if (m == 0 || n == 0) return INTENT_HIP_OK;
  if (out == nullptr || bias == nullptr || residual == nullptr || output_scale == nullptr ||
      (k > 0 && (a == nullptr || b == nullptr)))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null tensor pointer");
  if (lda < (m > 1 ? k : 0) || ldb < (k > 1 ? n : 0) || ldr < (m > 1 ? n : 0) || ldo < (m > 1 ? n : 0))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "row stride smaller than the row length");
  const QuantizeStore ep{bias, static_cast<const uint16_t *>(residual), ldr, output_scale, static_cast<int8_t *>(out),
                         ldo};
  // The MFMA kernel's epilogue reads 4 residuals as 8 bytes and stores 4 outputs as 4 bytes.
  const bool fast = k % 8 == 0 && n % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 && aligned(a, 16) && aligned(b, 16) &&
                    ldr % 4 == 0 && aligned(residual, 8) && ldo % 4 == 0 && aligned(out, 4);
  return launch_epilogue<_Float16>(static_cast<const uint16_t *>(a), static_cast<const uint16_t *>(b), ep, m, n, k, lda,
                                   ldb, fast, as_stream(stream));
}
