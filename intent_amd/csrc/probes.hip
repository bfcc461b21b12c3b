// Measurement probe: the box's own MFMA ceiling, timed beside the operators so that the roofline
// fractions of the matrix kernels can also be read against what this GPU sustains, not only
// against the published peak. Every wave issues `iterations` rounds of kChains independent
// v_mfma_f32_32x32x16_{bf16,f16} on register operands (no memory traffic in the loop), two waves
// per SIMD as the GEMM and attention kernels run, so it gives the sustained dense MFMA rate at the
// clock the matrix pipes hold under full load: with the same operands in every MFMA, and with
// varied operands, whose switching activity (power) is that of real data. (The box's copy rate is
// torch's own device copy.)
#include "common.hpp"

namespace intent_hip {
namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int kChains = 8;          // independent accumulators per wave (8 x 16 VGPRs)
constexpr int kProbeThreads = 256;  // 4 waves: two workgroups per CU give two waves per SIMD

// Operand values in [0.5, 1): all positive, so the sums never cancel and grow linearly with the
// rounds. kVaried gives every chain its own operands with pseudo-random mantissas (a hash of lane,
// element and chain), so consecutive MFMAs switch as many multiplier bits as real data does;
// otherwise every chain multiplies the same two operands.
__device__ __forceinline__ float probe_value(uint32_t lane, uint32_t i, uint32_t c, bool varied) {
  uint32_t h = varied ? (lane * 2654435761u) ^ (i * 40503u + 1u) ^ (c * 2246822519u) : (lane + i) & 7u;
  h ^= h >> 15;
  h *= 2246822519u;
  h ^= h >> 13;
  return 0.5f + static_cast<float>(h & 0xffffu) * (0.5f / 65536.0f);
}

// Two waves per SIMD: without the attribute hipcc places the accumulators in AGPRs beside 130
// VGPRs, 258 registers, which leaves one wave per SIMD.
template <bool kBf16, bool kVaried>
__global__ __launch_bounds__(kProbeThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void mfma_probe(
    int64_t iterations, float *out) {
  const int lane = threadIdx.x & 63;
  constexpr int kSets = kVaried ? kChains : 1;
  f16x8_t ah[kSets], bh[kSets];
  bf16x8_t ab[kSets], bb[kSets];
#pragma unroll
  for (int c = 0; c < kSets; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float va = probe_value(lane, i, 2 * c, kVaried), vb = probe_value(lane, i + 8, 2 * c + 1, kVaried);
      ah[c][i] = static_cast<_Float16>(va);
      bh[c][i] = static_cast<_Float16>(vb);
      ab[c][i] = static_cast<__bf16>(va);
      bb[c][i] = static_cast<__bf16>(vb);
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
        acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ab[c % kSets], bb[c % kSets], acc[c], 0, 0, 0);
      else
        acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[c % kSets], bh[c % kSets], acc[c], 0, 0, 0);
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

extern "C" int intent_hip_mfma_probe(int dtype, int varied, int64_t blocks, int64_t iterations, float *out,
                                     void *stream) {
  if (dtype != INTENT_HIP_F16 && dtype != INTENT_HIP_BF16)
    return fail(INTENT_HIP_ERR_UNSUPPORTED, "mfma_probe: dtype %d (F16 or BF16 only)", dtype);
  if (blocks <= 0 || blocks > (1 << 20) || iterations < 0)
    return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "mfma_probe: blocks in [1, 2^20] and iterations >= 0");
  if (out == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null output");
  const dim3 grid(static_cast<unsigned>(blocks)), block(kProbeThreads);
  const hipStream_t s = as_stream(stream);
  if (dtype == INTENT_HIP_BF16) {
    if (varied) mfma_probe<true, true><<<grid, block, 0, s>>>(iterations, out);
    else mfma_probe<true, false><<<grid, block, 0, s>>>(iterations, out);
  } else {
    if (varied) mfma_probe<false, true><<<grid, block, 0, s>>>(iterations, out);
    else mfma_probe<false, false><<<grid, block, 0, s>>>(iterations, out);
  }
  if (hipPeekAtLastError() != hipSuccess) return launch_status("mfma_probe");
  return INTENT_HIP_OK;
}
