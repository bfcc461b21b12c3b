// Library-level entry points of libintent_hip.so: ABI version, status strings,
// device facts and kernel resource facts.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "common.hpp"

namespace intent_hip {
namespace {
thread_local char g_last_error[512] = "";
}

int fail(int status, const char *format, ...) {
  va_list args;
  va_start(args, format);
  vsnprintf(g_last_error, sizeof(g_last_error), format, args);
  va_end(args);
  return status;
}

int launch_status(const char *kernel) {
  const hipError_t error = hipGetLastError();
  return fail(INTENT_HIP_ERR_LAUNCH, "launch of %s failed: %s", kernel, hipGetErrorString(error));
}

int describe_kernel(const void *kernel, const char *name, int block_threads, IntentHipKernelResources *out) {
  if (out == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null output");
  memset(out, 0, sizeof(*out));
  snprintf(out->kernel, sizeof(out->kernel), "%s", name);
  hipFuncAttributes attributes;
  if (hipFuncGetAttributes(&attributes, kernel) != hipSuccess)
    return fail(INTENT_HIP_ERR_DEVICE, "hipFuncGetAttributes(%s): %s", name, hipGetErrorString(hipGetLastError()));
  out->vgprs = attributes.numRegs;
  out->lds_bytes = static_cast<int32_t>(attributes.sharedSizeBytes);
  out->scratch_bytes = static_cast<int32_t>(attributes.localSizeBytes);
  out->max_threads_per_block = attributes.maxThreadsPerBlock;
  out->block_threads = block_threads;
  return INTENT_HIP_OK;
}

// Workgroups of `kernel` the current device holds at once (CUs x resident workgroups per CU),
// queried once per device and kernel.
int resident_blocks(const void *kernel, int block) {
  static std::mutex lock;
  static struct { const void *kernel; int device; int blocks; } cache[16];
  static int used = 0;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return 1024;
  std::lock_guard<std::mutex> guard(lock);
  for (int i = 0; i < used; ++i)
    if (cache[i].kernel == kernel && cache[i].device == device) return cache[i].blocks;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0) cus = 256;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, 0) != hipSuccess || per_cu <= 0) per_cu = 1;
  const int blocks = cus * per_cu;
  if (used < 16) cache[used++] = {kernel, device, blocks};
  return blocks;
}

int device_cus() {
  static std::mutex lock;
  static int cus[64] = {};
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return 256;
  std::lock_guard<std::mutex> guard(lock);
  if (cus[device] <= 0 &&
      (hipDeviceGetAttribute(&cus[device], hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
       cus[device] <= 0))
    cus[device] = 256;
  return cus[device];
}

}  // namespace intent_hip

using namespace intent_hip;

extern "C" int intent_hip_abi_version(void) { return INTENT_HIP_ABI_VERSION; }

extern "C" const char *intent_hip_status_string(int status) {
  switch (status) {
    case INTENT_HIP_OK: return "ok";
    case INTENT_HIP_ERR_INVALID_ARGUMENT: return "invalid argument";
    case INTENT_HIP_ERR_UNSUPPORTED: return "unsupported";
    case INTENT_HIP_ERR_LAUNCH: return "launch failed";
    case INTENT_HIP_ERR_DEVICE: return "device query failed";
    case INTENT_HIP_ERR_WORKSPACE: return "workspace missing or too small";
  }
  return "unknown status";
}

extern "C" const char *intent_hip_last_error(void) { return g_last_error; }

extern "C" int intent_hip_device_count(int *count) {
  if (count == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null output");
  if (hipGetDeviceCount(count) != hipSuccess) {
    *count = 0;
    return fail(INTENT_HIP_ERR_DEVICE, "hipGetDeviceCount: %s", hipGetErrorString(hipGetLastError()));
  }
  return INTENT_HIP_OK;
}

extern "C" int intent_hip_device_info(int device, IntentHipDeviceInfo *out) {
  if (out == nullptr) return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "null output");
  memset(out, 0, sizeof(*out));
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess)
    return fail(INTENT_HIP_ERR_DEVICE, "hipGetDeviceProperties(%d): %s", device,
                hipGetErrorString(hipGetLastError()));
  snprintf(out->arch, sizeof(out->arch), "%s", prop.gcnArchName);
  out->compute_units = prop.multiProcessorCount;
  out->wavefront_size = prop.warpSize;
  out->lds_per_workgroup = static_cast<int64_t>(prop.sharedMemPerBlock);
  out->global_memory_bytes = static_cast<int64_t>(prop.totalGlobalMem);
  out->clock_khz = prop.clockRate;
  out->memory_clock_khz = prop.memoryClockRate;
  out->memory_bus_width = prop.memoryBusWidth;
  out->l2_bytes = prop.l2CacheSize;
  return INTENT_HIP_OK;
}

extern "C" int intent_hip_kernel_resources(int op, int dtype, int64_t rows, int64_t cols,
                                           IntentHipKernelResources *out) {
  switch (op) {
    case INTENT_HIP_OP_SOFTMAX_FWD: return softmax_fwd_resources(dtype, rows, cols, out);
    case INTENT_HIP_OP_SOFTMAX_BWD: return softmax_bwd_resources(dtype, rows, cols, out);
    case INTENT_HIP_OP_GEMM_BF16: return gemm_resources(INTENT_HIP_BF16, rows, cols, out);
    case INTENT_HIP_OP_GEMM: return gemm_resources(dtype, rows, cols, out);
    case INTENT_HIP_OP_GEMM_F32: return gemm_f32_resources(rows, cols, out);
    // cols = d, or d | dv << 16 when dv differs from d.
    case INTENT_HIP_OP_ATTENTION_FWD_F16:
      return attention_resources(INTENT_HIP_F16, rows, cols & 0xFFFF, (cols >> 16) ? (cols >> 16) : (cols & 0xFFFF),
                                 0, out);
    case INTENT_HIP_OP_ATTENTION_FWD:
      return attention_resources(dtype, rows, cols & 0xFFFF, (cols >> 16) ? (cols >> 16) : (cols & 0xFFFF), 0,
                                 out);
    case INTENT_HIP_OP_ATTENTION_VARLEN:
      return attention_resources(dtype, rows, cols & 0xFFFF, (cols >> 16) ? (cols >> 16) : (cols & 0xFFFF), 1,
                                 out);
    case INTENT_HIP_OP_CSR_SPMV_F32: return spmv_resources(rows, cols, out);
    case INTENT_HIP_OP_ATTENTION_BWD_DELTA: return attention_bwd_resources(0, rows, cols, out);
    case INTENT_HIP_OP_ATTENTION_BWD_DQ: return attention_bwd_resources(1, rows, cols, out);
    case INTENT_HIP_OP_ATTENTION_BWD_DKDV: return attention_bwd_resources(2, rows, cols, out);
    case INTENT_HIP_OP_PAGED_DECODE_PARTIALS: return decode_resources(0, cols, rows, out);
    case INTENT_HIP_OP_SPLITK_REDUCE: return decode_resources(1, cols, rows, out);
    case INTENT_HIP_OP_GROUPED_DECODE_PARTIALS: return decode_resources(2, cols, rows, out);
    case INTENT_HIP_OP_CONTINUOUS_DECODE: return decode_resources(3, cols, rows, out);
    case INTENT_HIP_OP_VARLEN_DECODE: return decode_resources(4, cols, rows, out);
    case INTENT_HIP_OP_DECODE_MERGE: return decode_resources(5, cols, rows, out);
    case INTENT_HIP_OP_MLA_PREFILL:
      return attention_resources(INTENT_HIP_F16, rows, cols & 0xFFFF, cols >> 16, 3, out);
    case INTENT_HIP_OP_CSR_SPMM_F32: return spmm_resources(cols, out);
    case INTENT_HIP_OP_GEMM_I8: return gemm_i8_resources(rows, cols, out);
    case INTENT_HIP_OP_QUANTIZED_GEMM: return quantized_gemm_resources(out);
    case INTENT_HIP_OP_ATTENTION_BIAS:
      return attention_resources(INTENT_HIP_F16, rows, cols & 0xFFFF, (cols >> 16) ? (cols >> 16) : (cols & 0xFFFF), 2,
                                 out);
  }
  return fail(INTENT_HIP_ERR_INVALID_ARGUMENT, "unknown operator code %d", op);
}
