"""The no-allocation SpMV entry point (intent_hip_csr_spmv_f32_static, a static device scratch)
against the workspace entry point (intent_hip_csr_spmv_f32) through the C-ABI, on two calls in a
row, the second with a smaller input: the same kernels run on the same inputs, so the outputs are
bit-identical; both are also held to the SpMV parity bar against the oracle (rows of up to 4
nonzeros bit-exact, all rows within the backward-error bound)."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from intent_amd.examples import inputs
from intent_amd.runtime.hip.library import library
from tests.gpu_util import announce

pytestmark = pytest.mark.gpu

STATIC_BYTES = 32 << 20


def matrix(seed, rows, cols, long_rows):
    """Rows of every length class: lane (<= 4), 16-lane (5..127), medium windows and large slices."""
    rng = np.random.default_rng(seed)
    lengths = np.concatenate((rng.integers(0, 5, rows // 2), rng.integers(5, 128, rows // 4),
                              rng.integers(128, 300, rows // 8), rng.integers(300, 6000, long_rows)))
    lengths = lengths[rng.permutation(lengths.shape[0])]
    offsets, columns = inputs.csr_matrix(rng, lengths, cols)
    values = inputs.uniform(rng, int(offsets[-1]), -1, 1)
    x = inputs.uniform(rng, cols, -1, 1)
    return offsets, columns, values, x


def spmv(lib, device, offsets, columns, values, x, static):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    off, col, val, vec = t(offsets), t(columns), t(values), t(x)
    rows, nnz = offsets.shape[0] - 1, columns.shape[0]
    y = torch.full((rows,), float("nan"), dtype=torch.float32, device=device)
    stream = torch.cuda.current_stream().cuda_stream
    if static:
        rc = lib.fn["csr_spmv_f32_static"](off.data_ptr(), col.data_ptr(), val.data_ptr(), vec.data_ptr(),
                                            y.data_ptr(), rows, x.shape[0], nnz, stream)
    else:
        size = ctypes.c_size_t(0)
        assert lib.fn["csr_spmv_workspace_bytes"](rows, nnz, ctypes.byref(size)) == 0
        assert size.value <= STATIC_BYTES
        workspace = torch.empty(size.value, dtype=torch.uint8, device=device)
        rc = lib.fn["csr_spmv_f32"](off.data_ptr(), col.data_ptr(), val.data_ptr(), vec.data_ptr(), y.data_ptr(),
                                     rows, x.shape[0], nnz, workspace.data_ptr(), size.value, stream)
    assert rc == 0, lib.fn["last_error"]()
    torch.cuda.synchronize()
    return y.cpu().numpy()


def test_static_scratch_matches_workspace_entry(device):
    lib = library()
    cases = [matrix(41, 40_000, 300_000, 400), matrix(42, 3_000, 20_000, 30)]   # the second is smaller
    for n, (offsets, columns, values, x) in enumerate(cases):
        announce("spmv static scratch, call", n, "rows", offsets.shape[0] - 1, "nnz", columns.shape[0])
        got = spmv(lib, device, offsets, columns, values, x, static=True)
        want = spmv(lib, device, offsets, columns, values, x, static=False)
        assert np.array_equal(got, want), "static-scratch and workspace entries differ"
        ref = oracle.csr_spmv(offsets, columns, values, x)
        lengths = np.diff(offsets.astype(np.int64))
        products = np.abs(values.astype(np.float64) * x[columns].astype(np.float64))
        magnitude = np.zeros(lengths.shape[0])
        np.add.at(magnitude, np.repeat(np.arange(lengths.shape[0]), lengths), products)
        bound = (1e-5 + 2 * np.maximum(lengths - 1, 0) * 2.0 ** -24) * magnitude + 1e-38
        assert np.all(np.abs(got.astype(np.float64) - ref) <= bound)
        assert (got[lengths <= 4] == ref[lengths <= 4]).all()


def test_static_scratch_rejects_sizes_beyond_its_maximum(device):
    lib = library()
    size = ctypes.c_size_t(0)
    assert lib.fn["csr_spmv_workspace_bytes"](4_194_304, 67_108_855, ctypes.byref(size)) == 0
    assert size.value > STATIC_BYTES
    # The size check comes before any pointer is read or any kernel is launched.
    rc = lib.fn["csr_spmv_f32_static"](1, 1, 1, 1, 1, 4_194_304, 4_194_304, 67_108_855, None)
    assert rc == 5 and b"static scratch" in lib.fn["last_error"]()
