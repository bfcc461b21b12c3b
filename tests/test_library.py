"""The C-ABI library loads without a GPU and exports exactly what include/intent_hip.h declares."""
import ctypes
import re
from pathlib import Path

import pytest

from intent_amd.runtime.hip import library as hiplib

HEADER = Path(__file__).resolve().parents[1] / "include" / "intent_hip.h"


def declared_entry_points():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(intent_hip_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_entry_points() == sorted(hiplib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    if not hiplib.LIBRARY_PATH.exists():
        pytest.fail(f"{hiplib.LIBRARY_PATH} is not built")
    handle = ctypes.CDLL(str(hiplib.LIBRARY_PATH))
    for name in declared_entry_points():
        assert hasattr(handle, name), name


def test_library_loads_and_reports_abi():
    lib = hiplib.library()
    assert lib.abi_version == hiplib.ABI_VERSION
    assert lib.fn["status_string"](0) == b"ok"
    assert lib.fn["status_string"](5).startswith(b"workspace")


def test_argument_validation_without_gpu():
    """Extent checks run on the host before any HIP call."""
    lib = hiplib.library()
    status = lib.fn["softmax_fwd"](0, None, None, -1, 4, 4, 4, None)
    assert status == 1 and b"negative" in lib.fn["last_error"]()
    status = lib.fn["softmax_fwd"](9, 1, 1, 4, 4, 4, 4, None)
    assert status == 1 and b"dtype" in lib.fn["last_error"]()
    # zero-size work is a successful no-op
    assert lib.fn["softmax_fwd"](0, None, None, 0, 4, 4, 4, None) == 0
    size = ctypes.c_size_t(0)
    assert lib.fn["csr_spmv_workspace_bytes"](4_194_304, 67_108_855, ctypes.byref(size)) == 0
    # worst case (every nonzero in rows of 128 or in large rows): about 1.13 bytes per nonzero
    assert 0 < size.value <= 1.13 * 67_108_855 + 4096
    small = ctypes.c_size_t(0)
    assert lib.fn["csr_spmv_workspace_bytes"](1000, 127, ctypes.byref(small)) == 0
    assert small.value <= 4096                      # no row can be medium or large
    assert lib.fn["csr_spmv_f32"](1, 1, 1, 1, 1, 10, 10, 10, None, 0, None) == 5
    assert lib.fn["csr_spmv_f32"](1, 1, 1, 1, 1, 2**31 - 5, 10, 10, 1, 1 << 30, None) == 2


def test_attention_bias_validation_without_gpu():
    """The key-bias entry refuses a non-unit key stride, a negative stride and a null bias before
    any HIP call; empty work is a successful no-op."""
    lib = hiplib.library()
    fn = lib.fn["attention_bias_fwd"]
    strides = (ctypes.c_int64 * 16)(*([1 << 20, 1 << 16, 128, 1] * 4))

    def call(bias, bias_strides, sq=4, sk=4):
        return fn(16, 16, 16, bias, 16, 1, 1, sq, sk, 128, 128, strides, (ctypes.c_int64 * 3)(*bias_strides),
                  0.1, None)

    assert call(16, (64, 64, 2)) == 1 and b"unit key stride" in lib.fn["last_error"]()
    assert call(16, (-64, 64, 1)) == 1 and b"negative" in lib.fn["last_error"]()
    assert call(None, (64, 64, 1)) == 1 and b"null" in lib.fn["last_error"]()
    assert call(18, (64, 64, 1)) == 2 and b"aligned" in lib.fn["last_error"]()
    assert call(None, (64, 64, 1), sq=0) == 0


def test_decode_and_latent_validation_without_gpu():
    """The decode variants and latent attention refuse bad requests on the host: head counts that
    the group does not divide, unsupported head dimensions, a missing or short workspace, a null
    mask; empty work is a successful no-op. Workspace sizes follow the split rule."""
    lib = hiplib.library()
    err = lambda: lib.fn["last_error"]()  # noqa: E731
    s19, s17, s15, s24 = ((ctypes.c_int64 * n)(*([1 << 20] * (n - 1) + [1])) for n in (19, 17, 15, 24))
    grouped = lib.fn["grouped_decode_partials"]
    assert grouped(16, 16, 16, 16, 16, 1, 8, 2, 3, 64, 128, 128, 4, 16, s19, 0.1, None) == 1 and b"HEAD_GROUP" in err()
    assert grouped(16, 16, 16, 16, 16, 1, 8, 2, 4, 64, 96, 96, 4, 16, s19, 0.1, None) == 2 and b"D = DV" in err()
    assert grouped(16, 16, 16, 16, 16, 1, 8, 2, 4, 64, 128, 128, 4, 0, s19, 0.1, None) == 1
    assert grouped(16, 16, 16, 16, 16, 0, 8, 2, 4, 64, 128, 128, 4, 16, s19, 0.1, None) == 0
    size = ctypes.c_size_t(0)
    assert lib.fn["dense_decode_workspace_bytes"](32, 32, 8, 8192, 128, ctypes.byref(size)) == 0
    # 8 splits of 1024 keys: maxima and denominators, each from a 256-byte boundary, then 128 sums per split
    n = 32 * 32 * 8
    assert size.value == 2 * ((4 * n + 255) // 256 * 256) + 4 * n * 128
    cont = lib.fn["continuous_gqa_decode"]
    assert cont(16, 16, 16, 16, 16, 2, 8, 2, 4, 100, 128, 128, s17, 0.1, None, 0, None) == 5 and b"workspace" in err()
    assert cont(16, 16, 16, None, 16, 2, 8, 2, 4, 100, 128, 128, s17, 0.1, 256, 1 << 20, None) == 1
    assert lib.fn["varlen_decode_workspace_bytes"](8, 32, 8, 64, 64, ctypes.byref(size)) == 0
    n = 8 * 32 * 16                                  # 16 splits of 256 keys over the 4096-key cap
    assert size.value == 2 * ((4 * n + 255) // 256 * 256) + 4 * n * 64
    varlen = lib.fn["varlen_decode_sink"]
    assert varlen(16, 16, 16, 16, None, 16, 16, 8, 100, 32, 8, 4, 64, 64, 64, s15, 0.1, 256, 1 << 20, None) == 1
    assert varlen(16, 16, 16, 16, 16, 16, 16, 8, 100, 32, 8, 4, 64, 64, 64, s15, 0.1, 256, 16, None) == 5
    mla = lib.fn["mla_prefill"]
    assert mla(16, 16, 16, 16, 16, 16, 1, 8, 4, 64, 64, 128, 32, s24, 0.1, None, 0, None) == 2 and b"P = 64" in err()
    assert mla(16, 16, 16, 16, 16, 16, 1, 8, 3, 64, 64, 128, 64, s24, 0.1, None, 0, None) == 1
    assert mla(16, 16, 16, 16, 16, 16, 0, 8, 4, 64, 64, 128, 64, s24, 0.1, None, 0, None) == 0


def test_probe_validation_without_gpu():
    """The measurement probe checks its arguments on the host before any HIP call."""
    lib = hiplib.library()
    assert lib.fn["mfma_probe"](hiplib.F32, 1, 4, 1, 1, None) == 2              # F16 or BF16 only
    assert lib.fn["mfma_probe"](hiplib.BF16, 1, 0, 1, 1, None) == 1             # at least one workgroup
    assert lib.fn["mfma_probe"](hiplib.F16, 0, 4, 1, None, None) == 1           # null output
