"""GPU parity of the CSR SpMM kernel (csr_spmm) against the C oracle.

Bar: bit-exact. Kernel and oracle fold each output element over the row's nonzeros in the
definition's order with the product rounded before the add, so the results are identical; the
float64 backward-error bound |out - out64| <= L 2^-24 sum|a_i d_i| is checked beside it."""
import numpy as np
import pytest
import torch

import intent_amd as intent
import oracle
from intent_amd.examples import inputs
from intent_amd.examples.kernels.sparse.csr_spmm import csr_spmm
from tests.gpu_util import announce

pytestmark = pytest.mark.gpu


def t(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def spmm(device, offsets, columns, values, dense_t, outputs=None):
    kernel = intent.jit(csr_spmm, backend="hip")
    args = (t(offsets, device), t(columns, device), t(values, device), dense_t)
    if outputs is None:
        return kernel.run(*args).cpu().numpy()
    kernel.prepare(*args, outputs=outputs).launch()
    return outputs[0].cpu().numpy()


def check_float64(offsets, columns, values, dense, got):
    import scipy.sparse

    rows = offsets.shape[0] - 1
    a = scipy.sparse.csr_matrix((values.astype(np.float64), columns, offsets), shape=(rows, dense.shape[0]))
    want = a @ dense.astype(np.float64)
    mag = abs(a) @ np.abs(dense.astype(np.float64))
    longest = max(int(np.diff(offsets).max()) if rows else 0, 1)
    assert np.all(np.abs(got - want) <= longest * 2.0 ** -24 * mag + 1e-38)


def test_spmm_reference_shape_bit_exact(device):
    announce("csr_spmm reference shape 8192x8192, 32 per row, 128 features")
    offsets, columns, values, dense = inputs.csr_spmm(seed=1)
    got = spmm(device, offsets, columns, values, t(dense, device))
    want = oracle.csr_spmm(offsets, columns, values, dense)
    assert np.array_equal(got, want)
    check_float64(offsets, columns, values, dense, got)


@pytest.mark.parametrize("features", [1, 13, 64, 128, 200, 256])
def test_spmm_ragged_rows_and_feature_widths(device, features):
    announce("csr_spmm ragged", features)
    rng = np.random.default_rng(features)
    lengths = rng.integers(0, 40, 777)
    lengths[::9] = 0
    offsets, columns = inputs.csr_matrix(rng, lengths, 301)
    values = inputs.uniform(rng, offsets[-1], -1, 1)
    dense = inputs.uniform(rng, (301, features), -1, 1)
    got = spmm(device, offsets, columns, values, t(dense, device))
    assert np.array_equal(got, oracle.csr_spmm(offsets, columns, values, dense))
    assert (got[lengths == 0] == 0).all()


def test_spmm_strided_and_unaligned_operands(device):
    """dense as a column slice of a wider matrix (row stride > features), an explicit output view
    with a padded row stride, and a dense view starting one element in (4-byte aligned only)."""
    announce("csr_spmm strided")
    offsets, columns, values, dense = inputs.csr_spmm(seed=3, rows=500, cols=260, per_row=11, features=96)
    want = oracle.csr_spmm(offsets, columns, values, dense)
    wide = torch.zeros((260, 130), dtype=torch.float32, device=device)
    wide[:, 3:99] = t(dense, device)
    out_wide = torch.full((500, 100), 7.0, dtype=torch.float32, device=device)
    got = spmm(device, offsets, columns, values, wide[:, 3:99], outputs=(out_wide[:, :96],))
    assert np.array_equal(got, want)
    assert (out_wide[:, 96:] == 7.0).all()
    flat = torch.zeros(260 * 96 + 1, dtype=torch.float32, device=device)
    flat[1:] = t(dense, device).reshape(-1)
    assert np.array_equal(spmm(device, offsets, columns, values, flat[1:].view(260, 96)), want)


def test_spmm_probes(device):
    """Identity dense gives the matrix itself; ones count the nonzeros; empty matrix gives zeros."""
    announce("csr_spmm probes")
    rng = np.random.default_rng(9)
    lengths = np.array([0, 3, 1, 0, 5, 64, 2], np.int64)
    offsets, columns = inputs.csr_matrix(rng, lengths, 70)
    values = inputs.uniform(rng, offsets[-1], -1, 1)
    got = spmm(device, offsets, columns, values, t(np.eye(70, dtype=np.float32), device))
    expect = np.zeros((7, 70), np.float32)
    for r in range(7):
        expect[r, columns[offsets[r]:offsets[r + 1]]] = values[offsets[r]:offsets[r + 1]]
    assert np.array_equal(got, expect)
    ones = spmm(device, offsets, columns, np.ones_like(values), t(np.ones((70, 4), np.float32), device))
    assert (ones == lengths[:, None]).all()
    empty = np.zeros(5, np.int32)
    none = spmm(device, empty, np.zeros(0, np.int32), np.zeros(0, np.float32),
                t(np.ones((3, 8), np.float32), device))
    assert none.shape == (4, 8) and (none == 0).all()


def test_spmm_shape_errors(device):
    offsets, columns, values, dense = inputs.csr_spmm(seed=4, rows=10, cols=12, per_row=3, features=8)
    kernel = intent.jit(csr_spmm, backend="hip")
    with pytest.raises(ValueError):
        kernel.run(t(offsets, device), t(columns, device), t(values[:-1], device), t(dense, device))
    out = torch.empty((10, 9), dtype=torch.float32, device=device)
    with pytest.raises(ValueError):
        kernel.prepare(t(offsets, device), t(columns, device), t(values, device), t(dense, device),
                       outputs=(out,)).launch()
