// Shared helpers of libintent_hip.so (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "intent_hip.h"

namespace intent_hip {

// ---------------------------------------------------------------- host-side status handling
// Records `message` as the calling thread's last error and returns `status`.
int fail(int status, const char *format, ...) __attribute__((format(printf, 2, 3)));
// Turns the HIP runtime's launch status into an ABI status.
int launch_status(const char *kernel);

inline hipStream_t as_stream(void *stream) { return reinterpret_cast<hipStream_t>(stream); }

inline bool aligned(const void *p, unsigned bytes) {
  return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0;
}

// Workgroups of `kernel` (with `block` threads) the current device holds at once: CUs x resident
// workgroups per CU, queried once per device and kernel.
int resident_blocks(const void *kernel, int block);

// Compute units of the current device, queried once per device.
int device_cus();

// Fills `out` from hipFuncGetAttributes of `kernel`.
int describe_kernel(const void *kernel, const char *name, int block_threads,
                    IntentHipKernelResources *out);

// Kernel selection facts exported by each operator file for intent_hip_kernel_resources().
int softmax_fwd_resources(int dtype, int64_t rows, int64_t cols, IntentHipKernelResources *out);
int softmax_bwd_resources(int dtype, int64_t rows, int64_t cols, IntentHipKernelResources *out);
int gemm_resources(int dtype, int64_t m, int64_t n, IntentHipKernelResources *out);
int gemm_f32_resources(int64_t m, int64_t n, IntentHipKernelResources *out);
int gemm_i8_resources(int64_t m, int64_t n, IntentHipKernelResources *out);
int quantized_gemm_resources(IntentHipKernelResources *out);
int attention_resources(int dtype, int64_t sq, int64_t d, int64_t dv, int mode, IntentHipKernelResources *out);
int spmv_resources(int64_t rows, int64_t nnz, IntentHipKernelResources *out);
int attention_bwd_resources(int64_t which, int64_t rows, int64_t d, IntentHipKernelResources *out);
int decode_resources(int64_t which, int64_t d, int64_t group, IntentHipKernelResources *out);
int spmm_resources(int64_t features, IntentHipKernelResources *out);

constexpr int kWave = 64;

// ---------------------------------------------------------------- wave-wide reductions
// Cross-lane moves use DPP within each 16-lane row (quad permutes, half-row and
// row mirrors), then v_readlane of the four row results: no LDS traffic and no
// barrier. Every lane of the wave must be active.
template <int kCtrl>
__device__ __forceinline__ float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}

__device__ __forceinline__ float lane_value(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// maximum_num semantics: fmaxf returns the non-NaN operand when one side is NaN.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_move<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_move<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_move<0x140>(v));  // row_mirror
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_move<0xB1>(v);
  v += dpp_move<0x4E>(v);
  v += dpp_move<0x141>(v);
  v += dpp_move<0x140>(v);
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

// ---------------------------------------------------------------- 16-bit float conversions
// Storage types are raw 16-bit patterns; arithmetic is f32.
struct f16_t {
  uint16_t bits;
};
struct bf16_t {
  uint16_t bits;
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(f16_t v) {
  return static_cast<float>(__builtin_bit_cast(_Float16, v.bits));
}
__device__ __forceinline__ float to_f32(bf16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}

// f32 -> _Float16 or __bf16, rounded to nearest even. The empty asm makes v opaque, so
// instruction selection cannot fuse the conversion with the f32 product or FMA that produced v:
// v_fma_mixlo_f16 would round once, straight to 16 bits, where the definitions round the f32
// result and then cast. It emits no instruction.
template <typename E>
__device__ __forceinline__ E round_to(float v) {
  asm("" : "+v"(v));
  return static_cast<E>(v);
}

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ f16_t from_f32<f16_t>(float v) {
  // v_cvt_f16_f32 rounds to nearest even; finite overflow gives infinity.
  return f16_t{__builtin_bit_cast(uint16_t, round_to<_Float16>(v))};
}
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) {
  // Round to nearest even on the bit pattern; NaN stays a (quiet) NaN.
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return bf16_t{static_cast<uint16_t>((u >> 16) | 0x40u)};
  u += 0x7fffu + ((u >> 16) & 1u);
  return bf16_t{static_cast<uint16_t>(u >> 16)};
}

}  // namespace intent_hip
