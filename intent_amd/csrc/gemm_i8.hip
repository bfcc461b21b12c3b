// int8 GEMM with int32 accumulation and an int32 bias, C = A @ B + bias, for gfx950 (CDNA4).
//
// Semantics: gemm_i8 (python/intent/examples/kernels/contraction/gemm.py:41-51):
// c[m, n] = matmul(a[m, k], b[k, n], acc_dtype=i32) + bias[n]. A [M,K] and B [K,N] are int8,
// row-major with row strides lda / ldb (bytes = elements); bias [N] and C [M,N] are int32, C with
// row stride ldc. int32 sums wrap on overflow and are exact in any order, so every path below
// gives the same bits.
//
// Design (interior tiles: K % 64 == 0, N % 16 == 0, 16-byte aligned A and B rows):
//   * the structure of the bf16 kernel: workgroup tile 256 x 256, 8 waves in 2 x 4, each wave
//     128 x 64 = 4 x 2 tiles of v_mfma_i32_32x32x32_i8 (128 accumulator registers per lane). A
//     64-byte K step makes a stage A [256 m][64 k] plus B [64 k][256 n], 32 KB, the byte geometry
//     of the bf16 kernel's 32-deep stages. Five stages arrive by global_load_lds_dwordx4, and the
//     two waves of each SIMD alternate between their MFMA cluster and their fragment reads and DMA
//     (ping-pong, one barrier apart);
//   * A fragments: one ds_read_b128 gives a lane 16 consecutive k of its row (lanes 32-63 the next
//     16), the MFMA operand as it is;
//   * B fragments: ds_read_b64_tr_b8. In each 16-lane group, lane i slot j receives byte i % 8 of
//     the 8-byte segment addressed by lane 2 j + i / 8 (probed on the GPU). Lane m of a group
//     addresses row k0 + m / 2 at bytes n0 + 8 (m & 1) .. + 7, so lane i receives
//     B[k0 .. k0 + 7][n0 + i], 8 consecutive k of one column; two reads give the operand's 16 k.
//     A and B lanes hold the same k, so the products pair correctly whatever order the MFMA sums
//     them in;
//   * B rows are 256 bytes, one row of the 64 LDS banks. Chunk c (16 bytes) of row k is stored at
//     c ^ ((k & 7) | 8 ((k >> 4) & 1)): a transposing read of the wave touches 16 rows in two
//     chunk columns, and with this layout every bank exactly twice (two cycles for 512 bytes);
//   * the MFMA computes the transposed product, so each lane ends with 4 consecutive output
//     columns of one row and stores them, bias added, as one 16-byte store.
// Other shapes use gemm_i8_simple: 64 x 64 tiles through LDS, four products per v_dot4_i32_i8.
#include "common.hpp"

namespace intent_hip {
namespace {

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int kBM = 256, kBN = 256;
constexpr int kBK = 64;                                // bytes of k per stage
constexpr int kThreads = 512;
constexpr int kStages = 5;
constexpr int kChunksA = kBM * kBK / 16;               // 1024 16-byte chunks
constexpr int kStageChunks = (kBM + kBN) * kBK / 16;   // 2048 (32 KB)
constexpr int kGroupM = 2;

#define INTENT_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt((((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8)))
#define INTENT_WAIT_LGKMCNT0() __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4))

// int32 addition that wraps (two's complement), as the reference's int32 arithmetic does.
__device__ __forceinline__ int32_t wrap_add(int32_t a, int32_t b) {
  return static_cast<int32_t>(static_cast<uint32_t>(a) + static_cast<uint32_t>(b));
}

typedef __attribute__((address_space(3))) i32x2_t lds_i32x2_t;

// ds_read_b64_tr_b8 of the LDS byte at `p`, through the compiler builtin, so the compiler tracks
// the read's completion itself. `p` must be derived from the kernel's __shared__ array by pointer
// arithmetic (not through an integer): the compiler then knows which LDS object the read touches,
// and adds no wait for the DMA writes in flight before it.
__device__ __forceinline__ i32x2_t ds_read_tr8(const int8_t *p) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2_t *)(p));
}

// Physical chunk of B's logical chunk c in row k (16 chunks per row).
__device__ __forceinline__ int b_chunk(int c, int k) { return c ^ ((k & 7) | (((k >> 4) & 1) << 3)); }

// Barrier of the DMA loop: s_barrier with an acquire fence and no release fence (a release
// fence would wait for every DMA in flight; their completion is awaited with vmcnt instead).
__device__ __forceinline__ void dma_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  __builtin_amdgcn_sched_barrier(0);
}

// Tile order: groups of kGroupM tile rows walked column by column, in dispatch order (the tiles
// resident at one time share A row panels and B column panels, across XCDs through the MALL).
__device__ __forceinline__ void tile_of_block(int t, int tiles_m, int tiles_n, int &tm, int &tn) {
  const int per_group = kGroupM * tiles_n;
  const int group = t / per_group;
  const int first_m = group * kGroupM;
  const int rows_in_group = min(tiles_m - first_m, kGroupM);
  const int in_group = t - group * per_group;
  tm = first_m + in_group % rows_in_group;
  tn = in_group / rows_in_group;
}

// One interior tile (rows beyond M read row M - 1 and are not stored). A separate function with
// __restrict__ operands, inlined into the kernel: the compiler then carries alias scopes on the
// DMA and on the LDS reads, and adds no wait for the DMA in flight before the transposing reads
// (the kernel's own vmcnt waits and barriers order them).
__device__ __forceinline__ void gemm_i8_tile(const int8_t *__restrict__ A, const int8_t *__restrict__ B,
                                             const int32_t *__restrict__ bias, int32_t *__restrict__ C, int M,
                                             int K, int64_t lda, int64_t ldb, int64_t ldc, int m0, int n0,
                                             uint4 *lds) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;

  // DMA: each wave moves 2 A and 2 B chunks of 1 KB per stage. The global chunk a lane fetches is
  // the one its LDS slot (base + 16 lane) holds under the layouts above.
  const int8_t *a_src[2];
  const int8_t *b_src[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = (wave * 2 + i) * 64 + lane;
    const int ra = p >> 2, ca = (p & 3) ^ ((ra >> 2) & 3);
    a_src[i] = A + static_cast<int64_t>(min(m0 + ra, M - 1)) * lda + ca * 16;
    const int kb = p >> 4, cb = b_chunk(p & 15, kb);
    b_src[i] = B + static_cast<int64_t>(kb) * ldb + n0 + cb * 16;
  }
  const int k_tiles = K / kBK;
  auto issue = [&](int kt) {
    uint4 *stage = lds + (kt % kStages) * kStageChunks;
    const int64_t k0 = static_cast<int64_t>(kt) * kBK;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      __builtin_amdgcn_global_load_lds(a_src[i] + k0, (lds_void_t *)(stage + (wave * 2 + i) * 64), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(b_src[i] + k0 * ldb, (lds_void_t *)(stage + kChunksA + (wave * 2 + i) * 64),
                                       16, 0, 0);
    }
  };

  i32x16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

  const int frag_row = lane & 31, half = lane >> 5;
  const int a_swz = (frag_row >> 2) & 3;
  // B transposing-read address of this lane: group g = lane / 16, index i = lane % 16.
  const int g16 = lane >> 4, i16 = lane & 15;
  const int b_k = 16 * (g16 >> 1) + (i16 >> 1);        // + 32 kk + 8 r
  const int b_n = 16 * (g16 & 1) + 8 * (i16 & 1);      // + 64 wn + 32 nt

  // Ping-pong as in the bf16 kernel: waves 4-7 run one barrier behind waves 0-3, so between two
  // barriers one wave of each SIMD issues its MFMAs while the other reads its fragments and
  // issues its DMA. Before the barrier that opens the interval in which waves 0-3 read tile t,
  // every wave has waited for its own DMA of tile t; the DMA of tile t + S - 1 overwrites the
  // stage of tile t - 1, whose reads every wave completed (lgkmcnt 0) before an earlier barrier.
  const bool lag = wave >= 4;
#pragma unroll
  for (int kt = 0; kt < kStages - 1; ++kt)
    if (kt < k_tiles) issue(kt);
  auto wait_tile = [&](int t) {   // this wave's DMA of tile t complete; later tiles may stay in flight
    const int later = min(k_tiles - 1 - t, kStages - 2);
    if (later >= 3) INTENT_WAIT_VMCNT(12);
    else if (later == 2) INTENT_WAIT_VMCNT(8);
    else if (later == 1) INTENT_WAIT_VMCNT(4);
    else INTENT_WAIT_VMCNT(0);
  };
  wait_tile(0);
  dma_barrier();
  if (lag) dma_barrier();
  i32x4_t af[2][4], bf[2][2];
  for (int kt = 0; kt < k_tiles; ++kt) {
    const uint4 *sa = lds + (kt % kStages) * kStageChunks;
    const int8_t *sb = reinterpret_cast<const int8_t *>(sa + kChunksA);
#pragma unroll
    for (int kk = 0; kk < kBK / 32; ++kk) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        af[kk][t] = __builtin_bit_cast(i32x4_t, sa[(wm * 128 + t * 32 + frag_row) * 4 + ((kk * 2 + half) ^ a_swz)]);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        i32x2_t parts[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int k = kk * 32 + b_k + 8 * r;
          const int n = wn * 64 + t * 32 + b_n;
          parts[r] = ds_read_tr8(sb + k * kBN + b_chunk(n >> 4, k) * 16 + (n & 15));
        }
        bf[kk][t] = i32x4_t{parts[0][0], parts[0][1], parts[1][0], parts[1][1]};
      }
    }
    if (kt + kStages - 1 < k_tiles) issue(kt + kStages - 1);
    if (lag) wait_tile(kt + 1);
    INTENT_WAIT_LGKMCNT0();
    dma_barrier();
#pragma unroll
    for (int kk = 0; kk < kBK / 32; ++kk)
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[kk][nt], af[kk][mt], acc[mt][nt], 0, 0, 0);
    if (!lag) wait_tile(kt + 1);
    dma_barrier();
  }
  if (!lag) dma_barrier();

  // Epilogue: acc[mt][nt][4g + e] is C[i][n] with i = the A fragment's row (lane & 31) and
  // n = 8g + 4 (lane >> 5) + e within the 32-column tile.
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int i = m0 + wm * 128 + mt * 32 + frag_row;
    if (i >= M) continue;
    int32_t *crow = C + static_cast<int64_t>(i) * ldc;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn * 64 + nt * 32 + 8 * g + 4 * half;
        const i32x16_t &v = acc[mt][nt];
        *reinterpret_cast<i32x4_t *>(crow + n) =
            i32x4_t{wrap_add(v[4 * g], bias[n]), wrap_add(v[4 * g + 1], bias[n + 1]),
                    wrap_add(v[4 * g + 2], bias[n + 2]), wrap_add(v[4 * g + 3], bias[n + 3])};
      }
  }
}

__global__ __launch_bounds__(kThreads, 1) void gemm_i8_mfma(const int8_t *__restrict__ A,
                                                            const int8_t *__restrict__ B,
                                                            const int32_t *__restrict__ bias,
                                                            int32_t *__restrict__ C, int M, int K, int64_t lda,
                                                            int64_t ldb, int64_t ldc, int tiles_m, int tiles_n) {
  __shared__ uint4 lds[kStages * kStageChunks];
  int tm, tn;
  tile_of_block(blockIdx.x, tiles_m, tiles_n, tm, tn);
  gemm_i8_tile(A, B, bias, C, M, K, lda, ldb, ldc, tm * kBM, tn * kBN, lds);
}

// ---------------------------------------------------------------- general shapes
// 64 x 64 output tile per 256 threads (4 x 4 per thread), K in steps of 64 through LDS. A is kept
// [m][k] and B transposed to [n][k], so 4 consecutive k of either are one dword for v_dot4_i32_i8.
constexpr int kST = 64, kSK = 64;

__global__ __launch_bounds__(256) void gemm_i8_simple(const int8_t *__restrict__ A, const int8_t *__restrict__ B,
                                                      const int32_t *__restrict__ bias, int32_t *__restrict__ C,
                                                      int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc) {
  __shared__ int32_t sa[kST][kSK / 4 + 1];
  __shared__ int32_t sb[kST][kSK / 4 + 1];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int m0 = blockIdx.y * kST, n0 = blockIdx.x * kST;
  int acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += kSK) {
    // 64 x 16 dwords of each tile, 4 per thread; bytes past M, N or K are zero.
    for (int e = threadIdx.x; e < kST * (kSK / 4); e += 256) {
      const int r = e / (kSK / 4), q = e % (kSK / 4);
      uint32_t wa = 0, wb = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int k = k0 + 4 * q + b;
        const uint8_t va = (m0 + r < M && k < K) ? static_cast<uint8_t>(A[static_cast<int64_t>(m0 + r) * lda + k]) : 0;
        const uint8_t vb = (n0 + r < N && k < K) ? static_cast<uint8_t>(B[static_cast<int64_t>(k) * ldb + n0 + r]) : 0;
        wa |= static_cast<uint32_t>(va) << (8 * b);
        wb |= static_cast<uint32_t>(vb) << (8 * b);
      }
      sa[r][q] = static_cast<int32_t>(wa);
      sb[r][q] = static_cast<int32_t>(wb);
    }
    __syncthreads();
#pragma unroll 4
    for (int q = 0; q < kSK / 4; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_sdot4(sa[ty * 4 + i][q], sb[tx * 4 + j][q], acc[i][j], false);
    __syncthreads();
  }
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + ty * 4 + i;
    if (m >= M) continue;
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tx * 4 + j;
      if (n < N) C[static_cast<int64_t>(m) * ldc + n] = wrap_add(acc[i][j], bias[n]);
    }
  }
}

bool fast_path(const void *a, const void *b, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc,
               const void *c, const void *bias) {
  return k % kBK == 0 && n % 16 == 0 && lda % 16 == 0 && ldb % 16 == 0 && ldc % 4 == 0 && aligned(a, 16) &&
         aligned(b, 16) && aligned(c, 16) && aligned(bias, 4);
}

}  // namespace

int gemm_i8_resources(int64_t m, int64_t n, IntentHipKernelResources *out) {
  (void)m;
  (void)n;
  return describe_kernel(reinterpret_cast<const void *>(&gemm_i8_mfma), "gemm_i8_mfma", kThreads, out);
}

}  // namespace intent_hip

using namespace intent_hip;

extern "C" int intent_hip_gemm_i8(const void *a, const void *b, const int32_t *bias, int32_t *c, int64_t m, int64_t n,
                                  int64_t k, int64_t lda, int64_t ldb, int64_t ldc, void *stream) {
  if (m < 0 || n < 0 || k < 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (m > INT32_MAX / 2 || n > INT32_MAX / 2 || k > INT32_MAX / 2)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "GEMM extents must stay below 2^30");
  if (m == 0 || n == 0) return INTENT_HIP_OK;
  if (c == nullptr || bias == nullptr || (k > 0 && (a == nullptr || b == nullptr)))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null tensor pointer");
  if (lda < (m > 1 ? k : 0) || ldb < (k > 1 ? n : 0) || ldc < (m > 1 ? n : 0))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "row stride smaller than the row length");
  const hipStream_t s = as_stream(stream);
  const auto *A = static_cast<const int8_t *>(a);
  const auto *B = static_cast<const int8_t *>(b);
  if (k > 0 && fast_path(a, b, n, k, lda, ldb, ldc, c, bias) && n % kBN == 0) {
    const int tiles_m = static_cast<int>((m + kBM - 1) / kBM), tiles_n = static_cast<int>(n / kBN);
    gemm_i8_mfma<<<dim3(tiles_m * tiles_n), dim3(kThreads), 0, s>>>(A, B, bias, c, static_cast<int>(m),
                                                                    static_cast<int>(k), lda, ldb, ldc, tiles_m,
                                                                    tiles_n);
    if (hipPeekAtLastError() != hipSuccess) return launch_status("gemm_i8_mfma");
    return INTENT_HIP_OK;
  }
  const dim3 grid(static_cast<unsigned>((n + kST - 1) / kST), static_cast<unsigned>((m + kST - 1) / kST));
  gemm_i8_simple<<<grid, dim3(256), 0, s>>>(A, B, bias, c, static_cast<int>(m), static_cast<int>(n),
                                            static_cast<int>(k), lda, ldb, ldc);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("gemm_i8_simple");
  return INTENT_HIP_OK;
}
