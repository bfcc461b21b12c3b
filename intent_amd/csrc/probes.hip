// Measurement probe: the box's own MFMA ceiling, timed beside the operators so that the roofline
// fractions of the matrix kernels can also be read against what this GPU sustains, not only
// against the published peak. Every wave issues `iterations` rounds of kChains independent
// v_mfma_f32_32x32x16_{bf16,f16} on register operands (no memory traffic in the loop), two waves
// per SIMD as the GEMM and attention kernels run, so it gives the sustained dense MFMA rate at the
// clock the matrix pipes hold under full load. (The box's copy rate is torch's own device copy.)
#include "common.hpp"

namespace intent_hip {
namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int kChains = 8;          // independent accumulators per wave (8 x 16 VGPRs)
constexpr int kProbeThreads = 256;  // 4 waves: two workgroups per CU give two waves per SIMD

template <bool kBf16>
__global__ __launch_bounds__(kProbeThreads) void mfma_probe(int64_t iterations, float *out) {
  const int lane = threadIdx.x & 63;
  // Operands depend on the lane so the compiler cannot fold the products; small values keep the
  // sums finite for any iteration count.
  f16x8_t ah, bh;
  bf16x8_t ab, bb;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float va = 1e-3f * static_cast<float>((lane + i) & 7), vb = 1e-3f * static_cast<float>((lane * 3 + i) & 7);
    ah[i] = static_cast<_Float16>(va);
    bh[i] = static_cast<_Float16>(vb);
    ab[i] = static_cast<__bf16>(va);
    bb[i] = static_cast<__bf16>(vb);
  }
  f32x16_t acc[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[c][e] = 0.0f;
  for (int64_t it = 0; it < iterations; ++it) {
#pragma unroll
    for (int c = 0; c < kChains; ++c) {
      if constexpr (kBf16)
        acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ab, bb, acc[c], 0, 0, 0);
      else
        acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, acc[c], 0, 0, 0);
    }
  }
  float sum = 0.0f;
#pragma unroll
  for (int c = 0; c < kChains; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) sum += acc[c][e];
  sum = wave_sum(sum);
  if (lane == 0) out[static_cast<int64_t>(blockIdx.x) * (kProbeThreads / 64) + (threadIdx.x >> 6)] = sum;
}

}  // namespace
}  // namespace intent_hip

using namespace intent_hip;

extern "C" int intent_hip_mfma_probe(int dtype, int64_t blocks, int64_t iterations, float *out, void *stream) {
  if (dtype != INTENT_HIP_F16 && dtype != INTENT_HIP_BF16)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "mfma_probe: dtype %d (F16 or BF16 only)", dtype);
  if (blocks <= 0 || blocks > (1 << 20) || iterations < 0)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "mfma_probe: blocks in [1, 2^20] and iterations >= 0");
  if (out == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null output");
  const dim3 grid(static_cast<unsigned>(blocks));
  if (dtype == INTENT_HIP_BF16)
    mfma_probe<true><<<grid, dim3(kProbeThreads), 0, as_stream(stream)>>>(iterations, out);
  else
    mfma_probe<false><<<grid, dim3(kProbeThreads), 0, as_stream(stream)>>>(iterations, out);
  if (hipPeekAtLastError() != hipSuccess) return launch_status("mfma_probe");
  return INTENT_HIP_OK;
}
