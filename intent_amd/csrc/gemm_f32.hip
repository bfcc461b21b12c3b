// f32 GEMM for gfx950: C = A @ B (gemm_f32) or C = X @ W^T (linear_f32), f32 operands and
// f32 accumulation.
//
// Semantics: gemm_f32 (python/intent/examples/kernels/contraction/gemm.py:15-27) and
// linear_f32 (:30-38): matmul(acc_dtype=f32) with no TF32 and no scaling; A [M,K] row-major,
// B [K,N] row-major (gemm_f32) or W [N,K] row-major (linear_f32, transpose_rhs). The sum over k
// is reassociated (a reduction whose order the DSL leaves free).
//
// Design:
//   * v_mfma_f32_32x32x2f32 (full f32 products and sums); workgroup tile 128 x 128, 4 waves in
//     2 x 2, each wave 64 x 64 = 2 x 2 MFMA tiles (64 accumulator registers per lane);
//   * K step 16 through double-buffered LDS, next step's global loads held in registers while
//     the current step is multiplied;
//   * within a K step, lanes 0-31 take k = 0..7 and lanes 32-63 take k = 8..15 (instruction i
//     uses k = 8 half + i), so each lane reads 8 consecutive k of its A row with two 16-byte LDS
//     reads; both operands use the same assignment, so every product pairs A[m][k] with B[k][n];
//   * B is kept in its natural [k][n] layout in LDS (rows padded by 4 floats so the two lane
//     halves, 8 rows apart, use different banks); W (linear_f32) is stored like A;
//   * the MFMA computes the transposed tile (B fragment first), so each lane holds 4
//     consecutive output columns of one row per register quad and stores them as one float4.
// Rows need 16-byte alignment and row strides that are multiples of 4 for the vector loads;
// other layouts take the same kernel with scalar loads.
#include "common.hpp"

namespace intent_hip {
namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBN = 128, kBK = 16;
constexpr int kThreads = 256;
constexpr int kRowA = kBK + 4;                 // A / W tile row: 16 k + 4 pad floats (80 bytes)
constexpr int kRowB = kBN + 4;                 // natural B tile row: 128 n + 4 pad floats
constexpr int kStageA = kBM * kRowA;
constexpr int kStageB = (kBN * kRowA > kBK * kRowB) ? kBN * kRowA : kBK * kRowB;
constexpr int kStage = kStageA + kStageB;

template <bool kTransB, bool kVec>
__global__ __launch_bounds__(kThreads) void gemm_f32_mfma(const float *__restrict__ A, const float *__restrict__ B,
                                                          float *__restrict__ C, int M, int N, int K, int64_t lda,
                                                          int64_t ldb, int64_t ldc) {
  __shared__ float lds[2 * kStage];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;

  // Global -> register roles. A (and W): 128 rows x 4 float4 per K step, two per thread: row
  // c / 4, quarter c % 4 for c = tid + 256 i. Natural B: 16 k-rows x 32 float4: k c / 32,
  // quarter c % 32.
  float4 ra[2], rb[2];
  auto load_rows = [&](const float *base, int64_t ld, int rows_total, int row0, int k0, float4 *r) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + kThreads * i;
      const int row = row0 + (c >> 2), kq = k0 + 4 * (c & 3);
      if (kVec) {
        const bool ok = row < rows_total && kq < K;
        r[i] = ok ? *reinterpret_cast<const float4 *>(base + static_cast<int64_t>(row) * ld + kq)
                  : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        const float *p = base + static_cast<int64_t>(row) * ld;
        const bool okr = row < rows_total;
        r[i].x = okr && kq < K ? p[kq] : 0.f;
        r[i].y = okr && kq + 1 < K ? p[kq + 1] : 0.f;
        r[i].z = okr && kq + 2 < K ? p[kq + 2] : 0.f;
        r[i].w = okr && kq + 3 < K ? p[kq + 3] : 0.f;
      }
    }
  };
  auto load_b_natural = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + kThreads * i;
      const int k = k0 + (c >> 5), nq = n0 + 4 * (c & 31);
      if (kVec) {
        const bool ok = k < K && nq < N;
        rb[i] = ok ? *reinterpret_cast<const float4 *>(B + static_cast<int64_t>(k) * ldb + nq)
                   : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        const float *p = B + static_cast<int64_t>(k) * ldb;
        const bool okk = k < K;
        rb[i].x = okk && nq < N ? p[nq] : 0.f;
        rb[i].y = okk && nq + 1 < N ? p[nq + 1] : 0.f;
        rb[i].z = okk && nq + 2 < N ? p[nq + 2] : 0.f;
        rb[i].w = okk && nq + 3 < N ? p[nq + 3] : 0.f;
      }
    }
  };
  auto load = [&](int k0) {
    load_rows(A, lda, M, m0, k0, ra);
    if (kTransB) load_rows(B, ldb, N, n0, k0, rb);
    else load_b_natural(k0);
  };
  auto store = [&](int stage) {
    float *sa = lds + stage * kStage;
    float *sb = sa + kStageA;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + kThreads * i;
      *reinterpret_cast<float4 *>(sa + (c >> 2) * kRowA + 4 * (c & 3)) = ra[i];
      if (kTransB) *reinterpret_cast<float4 *>(sb + (c >> 2) * kRowA + 4 * (c & 3)) = rb[i];
      else *reinterpret_cast<float4 *>(sb + (c >> 5) * kRowB + 4 * (c & 31)) = rb[i];
    }
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int frag = lane & 31, half = lane >> 5;
  auto compute = [&](int stage) {
    const float *sa = lds + stage * kStage;
    const float *sb = sa + kStageA;
    float af[2][8], bf[2][8];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const float *row = sa + (wm * 64 + t * 32 + frag) * kRowA + 8 * half;
      const float4 lo = *reinterpret_cast<const float4 *>(row), hi = *reinterpret_cast<const float4 *>(row + 4);
      af[t][0] = lo.x; af[t][1] = lo.y; af[t][2] = lo.z; af[t][3] = lo.w;
      af[t][4] = hi.x; af[t][5] = hi.y; af[t][6] = hi.z; af[t][7] = hi.w;
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int n = wn * 64 + t * 32 + frag;
      if (kTransB) {
        const float *row = sb + n * kRowA + 8 * half;
        const float4 lo = *reinterpret_cast<const float4 *>(row), hi = *reinterpret_cast<const float4 *>(row + 4);
        bf[t][0] = lo.x; bf[t][1] = lo.y; bf[t][2] = lo.z; bf[t][3] = lo.w;
        bf[t][4] = hi.x; bf[t][5] = hi.y; bf[t][6] = hi.z; bf[t][7] = hi.w;
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) bf[t][i] = sb[(8 * half + i) * kRowB + n];
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(bf[nt][i], af[mt][i], acc[mt][nt], 0, 0, 0);
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

  // acc[mt][nt][4 g + e] is C[m][n], m = this lane's A row (lane & 31 of tile mt),
  // n = 8 g + 4 half + e of tile nt.
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const int m = m0 + wm * 64 + mt * 32 + frag;
    if (m >= M) continue;
    float *crow = C + static_cast<int64_t>(m) * ldc;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn * 64 + nt * 32 + 8 * g + 4 * half;
        const f32x16_t &v = acc[mt][nt];
        if (kVec && n + 3 < N) {
          *reinterpret_cast<float4 *>(crow + n) = make_float4(v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < N) crow[n + e] = v[4 * g + e];
        }
      }
  }
}

}  // namespace

int gemm_f32_resources(int64_t m, int64_t n, IntentHipKernelResources *out) {
  (void)m;
  (void)n;
  return describe_kernel(reinterpret_cast<const void *>(&gemm_f32_mfma<false, true>), "gemm_f32_mfma", kThreads, out);
}

}  // namespace intent_hip

using namespace intent_hip;

extern "C" int intent_hip_gemm_f32(const float *a, const float *b, float *c, int64_t m, int64_t n, int64_t k,
                                   int64_t lda, int64_t ldb, int64_t ldc, int transpose_b, void *stream) {
  if (m < 0 || n < 0 || k < 0) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "negative extent");
  if (transpose_b != 0 && transpose_b != 1)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "transpose_b must be 0 or 1 (got %d)", transpose_b);
  if (m > INT32_MAX / 2 || n > INT32_MAX / 2 || k > INT32_MAX / 2)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "GEMM extents must stay below 2^30");
  if (m == 0 || n == 0) return INTENT_HIP_OK;
  if (c == nullptr || (k > 0 && (a == nullptr || b == nullptr)))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null tensor pointer");
  const int64_t b_row = transpose_b ? k : n;
  const int64_t b_rows = transpose_b ? n : k;
  if (lda < (m > 1 ? k : 0) || ldb < (b_rows > 1 ? b_row : 0) || ldc < (m > 1 ? n : 0))
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "row stride smaller than the row length");
  const bool vec = k % 4 == 0 && (transpose_b || n % 4 == 0) && lda % 4 == 0 && ldb % 4 == 0 && ldc % 4 == 0 &&
                   aligned(a, 16) && aligned(b, 16) && aligned(c, 16);
  const dim3 grid(static_cast<unsigned>((n + kBN - 1) / kBN), static_cast<unsigned>((m + kBM - 1) / kBM));
  const hipStream_t s = as_stream(stream);
  const int M = static_cast<int>(m), N = static_cast<int>(n), K = static_cast<int>(k);
  if (transpose_b) {
    if (vec) gemm_f32_mfma<true, true><<<grid, dim3(kThreads), 0, s>>>(a, b, c, M, N, K, lda, ldb, ldc);
    else gemm_f32_mfma<true, false><<<grid, dim3(kThreads), 0, s>>>(a, b, c, M, N, K, lda, ldb, ldc);
  } else {
    if (vec) gemm_f32_mfma<false, true><<<grid, dim3(kThreads), 0, s>>>(a, b, c, M, N, K, lda, ldb, ldc);
    else gemm_f32_mfma<false, false><<<grid, dim3(kThreads), 0, s>>>(a, b, c, M, N, K, lda, ldb, ldc);
  }
  if (hipPeekAtLastError() != hipSuccess) return launch_status("gemm_f32_mfma");
  return INTENT_HIP_OK;
}
