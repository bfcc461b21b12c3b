"""ctypes binding of libintent_hip.so (declared in include/intent_hip.h).

The library is loaded after torch so that both share torch's HIP runtime
(same soname `libamdhip64.so.7`). A missing or mismatched library raises
`CompilationStageError("native_loading", ...)`: there is no fallback path."""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

from ...diagnostics import CompilationStageError

ABI_VERSION = 17
# INTENT_HIP_STATIC_SCRATCH_BYTES: the static scratch of intent_hip_csr_spmv_f32_static.
STATIC_SCRATCH_BYTES = 32 << 20
LIBRARY_NAME = "libintent_hip.so"
LIBRARY_PATH = Path(__file__).resolve().parents[2] / LIBRARY_NAME

F32, F16, BF16 = 0, 1, 2
(OP_SOFTMAX_FWD, OP_SOFTMAX_BWD, OP_GEMM_BF16, OP_ATTENTION_FWD_F16, OP_CSR_SPMV_F32, OP_GEMM, OP_GEMM_F32,
 OP_ATTENTION_FWD, OP_ATTENTION_BWD_DELTA, OP_ATTENTION_BWD_DQ, OP_ATTENTION_BWD_DKDV, OP_PAGED_DECODE_PARTIALS,
 OP_SPLITK_REDUCE, OP_CSR_SPMM_F32, OP_ATTENTION_VARLEN, OP_GEMM_I8, OP_QUANTIZED_GEMM,
 OP_ATTENTION_BIAS, OP_GROUPED_DECODE_PARTIALS, OP_CONTINUOUS_DECODE, OP_VARLEN_DECODE, OP_DECODE_MERGE,
 OP_MLA_PREFILL) = range(23)
ACT_NONE, ACT_RELU = 0, 1

_i64, _int, _p, _f32, _sz = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_float, ctypes.c_size_t


class DeviceInfo(ctypes.Structure):
    _fields_ = [("arch", ctypes.c_char * 64), ("compute_units", ctypes.c_int32),
                ("wavefront_size", ctypes.c_int32), ("lds_per_workgroup", ctypes.c_int64),
                ("global_memory_bytes", ctypes.c_int64), ("clock_khz", ctypes.c_int32),
                ("memory_clock_khz", ctypes.c_int32), ("memory_bus_width", ctypes.c_int32),
                ("l2_bytes", ctypes.c_int32)]


class KernelResources(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_char * 128), ("vgprs", ctypes.c_int32), ("lds_bytes", ctypes.c_int32),
                ("scratch_bytes", ctypes.c_int32), ("max_threads_per_block", ctypes.c_int32),
                ("block_threads", ctypes.c_int32)]


# Exported entry points: name -> (restype, argtypes). Mirrors include/intent_hip.h.
SIGNATURES = {
    "intent_hip_abi_version": (_int, ()),
    "intent_hip_status_string": (ctypes.c_char_p, (_int,)),
    "intent_hip_last_error": (ctypes.c_char_p, ()),
    "intent_hip_device_count": (_int, (ctypes.POINTER(_int),)),
    "intent_hip_device_info": (_int, (_int, ctypes.POINTER(DeviceInfo))),
    "intent_hip_kernel_resources": (_int, (_int, _int, _i64, _i64, ctypes.POINTER(KernelResources))),
    "intent_hip_softmax_fwd": (_int, (_int, _p, _p, _i64, _i64, _i64, _i64, _p)),
    "intent_hip_softmax_bwd": (_int, (_int, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p)),
    "intent_hip_gemm_bf16": (_int, (_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p)),
    "intent_hip_gemm": (_int, (_int, _int, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p)),
    "intent_hip_gemm_f32": (_int, (_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _int, _p)),
    "intent_hip_gemm_i8": (_int, (_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p)),
    "intent_hip_quantized_gemm": (_int, (_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p)),
    "intent_hip_attention_fwd_f16": (_int, (_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                            ctypes.POINTER(_i64), _f32, _int, _p)),
    "intent_hip_attention_fwd": (_int, (_int, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                        ctypes.POINTER(_i64), _f32, _int, _p)),
    "intent_hip_attention_fwd_workspace_bytes": (_int, (_i64, _i64, _i64, _i64, _i64, ctypes.POINTER(_sz))),
    "intent_hip_attention_fwd_ws": (_int, (_int, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                           ctypes.POINTER(_i64), _f32, _int, _p, _sz, _p)),
    "intent_hip_mla_prefill_workspace_bytes": (_int, (_i64, _i64, _i64, _i64, _i64, ctypes.POINTER(_sz))),
    "intent_hip_mla_prefill": (_int, (_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                      ctypes.POINTER(_i64), _f32, _p, _sz, _p)),
    "intent_hip_attention_bias_fwd": (_int, (_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                             ctypes.POINTER(_i64), ctypes.POINTER(_i64), _f32, _p)),
    "intent_hip_attention_varlen_workspace_bytes": (_int, (_i64, _i64, ctypes.POINTER(_sz))),
    "intent_hip_attention_varlen_fwd": (_int, (_int, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                               ctypes.POINTER(_i64), _f32, _int, _p, _sz, _p)),
    "intent_hip_attention_bwd_delta": (_int, (_p, _p, _p, _i64, _i64, _i64, _i64, ctypes.POINTER(_i64), _p)),
    "intent_hip_attention_bwd_dq": (_int, (_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                           ctypes.POINTER(_i64), _f32, _int, _p)),
    "intent_hip_attention_bwd_dkdv": (_int, (_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                             ctypes.POINTER(_i64), _f32, _int, _p)),
    "intent_hip_paged_decode_partials": (_int, (_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                                _i64, _i64, _i64, _i64, _i64, _i64, ctypes.POINTER(_i64), _f32,
                                                _p)),
    "intent_hip_splitk_reduce_f32_to_f16": (_int, (_p, _p, _p, _i64, _i64, _i64, _i64, ctypes.POINTER(_i64), _p)),
    "intent_hip_grouped_decode_partials": (_int, (_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                                  _i64, ctypes.POINTER(_i64), _f32, _p)),
    "intent_hip_dense_decode_workspace_bytes": (_int, (_i64, _i64, _i64, _i64, _i64, ctypes.POINTER(_sz))),
    "intent_hip_continuous_gqa_decode": (_int, (_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                                ctypes.POINTER(_i64), _f32, _p, _sz, _p)),
    "intent_hip_varlen_decode_workspace_bytes": (_int, (_i64, _i64, _i64, _i64, _i64, ctypes.POINTER(_sz))),
    "intent_hip_varlen_decode_sink": (_int, (_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                             _i64, ctypes.POINTER(_i64), _f32, _p, _sz, _p)),
    "intent_hip_attention_bwd_dkdv_workspace_bytes": (_int, (_i64, _i64, _i64, _i64, _i64, _i64,
                                                              ctypes.POINTER(_sz))),
    "intent_hip_attention_bwd_dq_workspace_bytes": (_int, (_i64, _i64, _i64, _i64, _i64, _i64,
                                                            ctypes.POINTER(_sz))),
    "intent_hip_attention_bwd_dq_ws": (_int, (_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                              ctypes.POINTER(_i64), _f32, _int, _p, _sz, _p)),
    "intent_hip_attention_bwd_dkdv_ws": (_int, (_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                                ctypes.POINTER(_i64), _f32, _int, _p, _sz, _p)),
    "intent_hip_csr_spmv_workspace_bytes": (_int, (_i64, _i64, ctypes.POINTER(_sz))),
    "intent_hip_csr_spmv_f32": (_int, (_p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _sz, _p)),
    "intent_hip_csr_spmv_f32_static": (_int, (_p, _p, _p, _p, _p, _i64, _i64, _i64, _p)),
    "intent_hip_csr_spmm_f32": (_int, (_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p)),
    "intent_hip_mfma_probe": (_int, (_int, _int, _i64, _i64, _p, _p)),
}


class HipLibrary:
    """Loaded library: raw entry points in `fn[name]` (without the `intent_hip_` prefix)."""

    def __init__(self, path: Path):
        import torch  # noqa: F401  (loads the HIP runtime this library must share)

        if not path.exists():
            raise CompilationStageError(
                "native_loading", f"{path} is not built; run `python -m intent_amd.build`")
        try:
            self.handle = ctypes.CDLL(str(path))
        except OSError as error:
            raise CompilationStageError("native_loading", f"cannot load {path}: {error}") from error
        self.path = path
        self.fn = {}
        for name, (restype, argtypes) in SIGNATURES.items():
            function = getattr(self.handle, name)
            function.restype, function.argtypes = restype, list(argtypes)
            self.fn[name[len("intent_hip_"):]] = function
        self.abi_version = self.fn["abi_version"]()
        if self.abi_version != ABI_VERSION:
            raise CompilationStageError("native_loading",
                                        f"{path} has ABI {self.abi_version}, expected {ABI_VERSION}")

    def error(self, status: int) -> str:
        return f"{self.fn['status_string'](status).decode()}: {self.fn['last_error']().decode()}"

    def check(self, status: int, stage: str = "provider_invocation") -> None:
        if status != 0:
            raise CompilationStageError(stage, self.error(status))

    def device_count(self) -> int:
        count = _int(0)
        self.check(self.fn["device_count"](ctypes.byref(count)), "target_resolution")
        return count.value

    def device_info(self, device: int) -> dict:
        info = DeviceInfo()
        self.check(self.fn["device_info"](device, ctypes.byref(info)), "target_resolution")
        return {"arch": info.arch.decode(), "compute_units": info.compute_units,
                "wavefront_size": info.wavefront_size, "lds_per_workgroup": info.lds_per_workgroup,
                "global_memory_bytes": info.global_memory_bytes, "clock_khz": info.clock_khz,
                "memory_clock_khz": info.memory_clock_khz, "memory_bus_width": info.memory_bus_width,
                "l2_bytes": info.l2_bytes}

    def kernel_resources(self, op: int, dtype: int, rows: int, cols: int) -> dict | None:
        out = KernelResources()
        if self.fn["kernel_resources"](op, dtype, rows, cols, ctypes.byref(out)) != 0:
            return None
        return {"kernel": out.kernel.decode(), "vgprs": out.vgprs, "lds_bytes": out.lds_bytes,
                "scratch_bytes": out.scratch_bytes, "block_threads": out.block_threads}


_LOCK = threading.Lock()
_LIBRARY: HipLibrary | None = None


def library() -> HipLibrary:
    """The process-wide library image (loaded once, under a lock)."""
    global _LIBRARY
    with _LOCK:
        if _LIBRARY is None:
            _LIBRARY = HipLibrary(LIBRARY_PATH)
        return _LIBRARY
