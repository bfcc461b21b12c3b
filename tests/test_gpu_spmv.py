"""GPU parity of the CSR SpMV kernels.

Bars: index traversal bit-exact (probes with ones, one-hot x and small integers give
exact results in any summation order); rows folded by one lane (up to 4 nonzeros) equal the
oracle's strict left fold bit for bit; all rows within the backward-error bound
|y - y64| <= 1e-5 * sum|a_i x_i| against float64, and within (1e-5 + 2 (L-1) 2^-24) *
sum|a_i x_i| against the oracle. The cases reach every row class: one lane, 16-lane groups,
medium rows cut at 8 column windows, and large rows cut at 16384-column slices (x in LDS)."""
import numpy as np
import pytest
import torch

import intent_amd as intent
import oracle
from intent_amd.examples import inputs
from intent_amd.examples.kernels.sparse.csr_spmv import csr_spmv
from tests.gpu_util import announce

pytestmark = pytest.mark.gpu


def run(device, offsets, columns, values, x):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    return intent.jit(csr_spmv, backend="hip").run(t(offsets), t(columns), t(values), t(x)).cpu().numpy()


def reference64(offsets, columns, values, x):
    """float64 row sums and magnitudes over each row's absolute range [off[r], off[r+1])."""
    rows = offsets.shape[0] - 1
    starts, ends = offsets[:-1].astype(np.int64), offsets[1:].astype(np.int64)
    lengths = ends - starts
    products = values.astype(np.float64) * x[columns].astype(np.float64)
    y64, mag = np.zeros(rows), np.zeros(rows)
    nonempty = lengths > 0
    if nonempty.any():
        padded = np.concatenate((products, [0.0]))      # an end index may equal the array length
        cuts = np.stack((starts[nonempty], ends[nonempty]), axis=1).ravel()
        y64[nonempty] = np.add.reduceat(padded, cuts)[::2]
        mag[nonempty] = np.add.reduceat(np.abs(padded), cuts)[::2]
    return y64, mag, lengths


def check(device, offsets, columns, values, x):
    y = run(device, offsets, columns, values, x)
    want = oracle.csr_spmv(offsets, columns, values, x)
    y64, mag, lengths = reference64(offsets, columns, values, x)
    assert np.all(np.abs(y - y64) <= 1e-5 * mag + 1e-38), "backward error vs float64"
    bound = (1e-5 + 2 * np.maximum(lengths - 1, 0) * 2.0 ** -24) * mag + 1e-38
    assert np.all(np.abs(y.astype(np.float64) - want) <= bound), "vs oracle"
    lane_rows = lengths <= 4
    assert (y[lane_rows] == want[lane_rows]).all(), "rows of up to 4 nonzeros must be bit-exact"
    assert (y[lengths == 0] == 0).all()
    return y, want


def test_spmv_golden_and_probes(device, golden):
    announce("spmv golden")
    g = golden("spmv")
    off, col, val, x = g["spmv_offsets"], g["spmv_columns"], g["spmv_values"], g["spmv_x"]
    y, _ = check(device, off, col, val, x)
    assert np.all(np.abs(y - g["spmv_y64"]) <= 1e-5 * g["spmv_abs"] + 1e-38)
    ones = run(device, off, col, np.ones_like(val), np.ones(off.shape[0] - 1, np.float32))
    assert (ones == g["spmv_lengths"]).all()
    assert (run(device, off, col, val, g["spmv_onehot_x"]) == g["spmv_onehot_y"]).all()


@pytest.mark.parametrize("seed,rows,max_len", [(1, 5000, 40), (2, 3000, 5000), (3, 20000, 3), (4, 257, 70000)])
def test_spmv_random_lengths(device, seed, rows, max_len):
    announce("spmv random", seed, rows, max_len)
    rng = np.random.default_rng(seed)
    lengths = rng.integers(0, max_len + 1, rows)
    lengths[rng.integers(0, rows, rows // 10)] = 0
    cols = max(rows, 4 * max_len + 1)     # room for distinct columns: redraws of duplicates stay few
    offsets, columns = inputs.csr_matrix(rng, lengths, cols)
    values = inputs.uniform(rng, int(offsets[-1]), -1, 1)
    x = inputs.uniform(rng, cols, -1, 1)
    check(device, offsets, columns, values, x)
    ival = rng.integers(-3, 4, values.shape).astype(np.float32)
    ix = rng.integers(-3, 4, x.shape).astype(np.float32)
    assert (run(device, offsets, columns, ival, ix) == oracle.csr_spmv(offsets, columns, ival, ix)).all()


def test_spmv_reference_example_unsorted_columns(device):
    """The reference's irregular example (examples/programs/irregular.py:27-33): 32 nonzeros per row
    at the definition's constants (csr_spmv.py:5-8), columns drawn with replacement, so unsorted
    within a row and repeated. A few rows of 5000 nonzeros spread over every column exercise the
    single-row placement with unsorted columns. Placement only chooses which workgroup runs a
    block, so the bars are those of sorted matrices; small integers make every sum exact."""
    from intent_amd.examples.kernels.sparse.csr_spmv import COLUMNS, NONZEROS_PER_ROW, ROWS

    announce("spmv reference example, unsorted columns")
    rng = np.random.default_rng(33)
    lengths = np.full(ROWS, NONZEROS_PER_ROW, np.int64)
    lengths[rng.integers(0, ROWS, 5)] = 5000
    offsets = np.concatenate(([0], np.cumsum(lengths))).astype(np.int32)
    columns = rng.integers(0, COLUMNS, int(offsets[-1])).astype(np.int32)
    assert (np.diff(columns[:NONZEROS_PER_ROW]) < 0).any()            # unsorted in the first row
    values = inputs.uniform(rng, int(offsets[-1]), -1, 1)
    x = inputs.uniform(rng, COLUMNS, -1, 1)
    check(device, offsets, columns, values, x)
    ival = rng.integers(-3, 4, values.shape).astype(np.float32)
    ix = rng.integers(-3, 4, x.shape).astype(np.float32)
    assert (run(device, offsets, columns, ival, ix) == oracle.csr_spmv(offsets, columns, ival, ix)).all()


def test_spmv_special_values_stay_in_their_rows(device):
    """inf, -inf and NaN in x reach only the rows that reference them. They sit at every column a
    lane past a piece's end can stand in with (column 0, the last column, each 32768-column slice
    start, each column-window start), and every row class runs beside them: masked lanes must not
    multiply those entries by zero. A few rows do reference them; their inf or NaN follows IEEE
    addition in any order."""
    announce("spmv special values in x")
    rng = np.random.default_rng(41)
    cols = 300_000
    lengths = np.concatenate((rng.integers(1, 5, 2000), rng.integers(5, 128, 2000), rng.integers(128, 304, 1500),
                              rng.integers(304, 20000, 150)))
    rng.shuffle(lengths)
    offsets, columns = inputs.csr_matrix(rng, lengths, cols)
    window = -(-cols // 8)
    poison = np.unique(np.concatenate(([0, cols - 1], np.arange(0, cols, 32768), np.arange(0, cols, window))))
    hit = np.isin(columns, poison)
    columns[hit] = np.where(columns[hit] == cols - 1, cols - 2, columns[hit] + 1)   # no row references them
    chosen = rng.choice(np.nonzero(lengths > 0)[0], 60, replace=False)
    columns[offsets[chosen] + rng.integers(0, lengths[chosen])] = rng.choice(poison, 60)
    values = inputs.uniform(rng, int(offsets[-1]), -1, 1)
    x = inputs.uniform(rng, cols, -1, 1)
    x[poison] = np.resize(np.array([np.inf, -np.inf, np.nan], np.float32), poison.size)
    y = run(device, offsets, columns, values, x)
    want = oracle.csr_spmv(offsets, columns, values, x)
    assert (np.isnan(y) == np.isnan(want)).all()
    special = ~np.isfinite(want)
    assert special.sum() >= 40 and (y[special & ~np.isnan(want)] == want[special & ~np.isnan(want)]).all()
    clean_x = np.where(np.isfinite(x), x, 0).astype(np.float32)
    y64, mag, rows_len = reference64(offsets, columns, values, clean_x)
    finite = ~special
    assert np.isfinite(y[finite]).all()
    assert np.all(np.abs(y[finite] - y64[finite]) <= 1e-5 * mag[finite] + 1e-38)


def test_spmv_block_boundaries(device):
    """Rows whose ends fall exactly on, just before and just after workgroup boundaries."""
    announce("spmv block boundaries")
    lengths = np.array([2047, 0, 1, 2046, 1, 2048, 0, 0, 4095, 1, 1, 2047, 4096, 3, 0], np.int64)
    rng = np.random.default_rng(7)
    offsets, columns = inputs.csr_matrix(rng, lengths, 5000)
    values = inputs.uniform(rng, int(offsets[-1]), -1, 1)
    x = inputs.uniform(rng, 5000, -1, 1)
    check(device, offsets, columns, values, x)


def test_spmv_degenerate(device):
    announce("spmv degenerate")
    empty = run(device, np.zeros(6, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32),
                np.zeros(4, np.float32))
    assert (empty == 0).all() and empty.shape == (5,)
    one = run(device, np.array([0, 3], np.int32), np.array([0, 1, 2], np.int32),
              np.array([1.0, 1e-8, 1e-8], np.float32), np.ones(3, np.float32))
    assert one[0] == np.float32(1.0)                       # the ordered fold, bit for bit
    zero_rows = run(device, np.zeros(1, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32),
                    np.zeros(3, np.float32))
    assert zero_rows.shape == (0,)


def test_spmv_config5_full(device):
    announce("spmv config 5 (4194304 rows, recipe A)")
    offsets, columns, values, x = inputs.spmv_f32()
    y, want = check(device, offsets, columns, values, x)
    assert int(offsets[-1]) == 67_108_855
    # Beside the backward-error bound (every row, asserted in check), the plain relative bar
    # |y - y64| <= 1e-5 |y64|: rows whose sum cancels can miss it without any error in the kernel
    # (the bound is relative to a near-zero result), so its share is reported and held to a floor.
    y64, mag, _ = reference64(offsets, columns, values, x)
    plain = np.abs(y.astype(np.float64) - y64) <= 1e-5 * np.abs(y64)
    announce(f"spmv config 5: {plain.mean():.6f} of rows within plain rel 1e-5 "
             f"({int((~plain).sum())} outside, all within the backward-error bound)")
    assert plain.mean() > 0.999


def test_spmv_shape_errors(device):
    announce("spmv shape errors")
    t = lambda a: torch.from_numpy(np.asarray(a)).to(device)  # noqa: E731
    kernel = intent.jit(csr_spmv, backend="hip")
    with pytest.raises(ValueError):
        kernel.run(t(np.array([0, 1], np.int32)), t(np.array([0, 0], np.int32)), t(np.zeros(1, np.float32)),
                   t(np.zeros(2, np.float32)))
    with pytest.raises(ValueError):
        out = torch.empty(3, device=device)
        kernel(t(np.array([0, 1], np.int32)), t(np.array([0], np.int32)), t(np.zeros(1, np.float32)),
               t(np.zeros(2, np.float32)), out)


def test_spmv_offsets_inside_larger_arrays(device):
    """Row offsets that start above 0 and end below the length of the column and value arrays (a
    row slice of a larger CSR): rows read their absolute ranges, nothing outside is touched."""
    announce("spmv offsets inside larger arrays")
    rng = np.random.default_rng(11)
    for first, lengths in ((3000, [1, 1]), (0, [1, 0, 0]), (777, [5, 0, 300, 9, 2000, 1, 40])):
        nnz = first + int(np.sum(lengths)) + 1234
        offsets = (first + np.concatenate(([0], np.cumsum(lengths)))).astype(np.int32)
        columns = rng.integers(0, 6000, nnz).astype(np.int32)
        values = inputs.uniform(rng, nnz, -1, 1)
        x = inputs.uniform(rng, 6000, -1, 1)
        check(device, offsets, columns, values, x)


@pytest.mark.parametrize("sort", [True, False])
def test_spmv_medium_and_large_rows(device, sort):
    """300000 columns give 19 slices, so rows of 128..303 nonzeros are medium (cut at 8 column
    windows) and longer rows large (cut at slices); with unsorted columns the cuts still partition
    each row and entries outside their window or slice read x from global memory."""
    announce("spmv medium and large rows", sort)
    rng = np.random.default_rng(21 + sort)
    cols = 300_000
    lengths = np.concatenate((rng.integers(128, 304, 3000), rng.integers(304, 20000, 300), rng.integers(0, 128, 3000),
                              [127, 128, 303, 304, 0, 1, 8, 9]))
    rng.shuffle(lengths)
    offsets, columns = inputs.csr_matrix(rng, lengths, cols)
    if not sort:
        for r in np.nonzero(lengths >= 128)[0]:
            rng.shuffle(columns[offsets[r]:offsets[r + 1]])
    values = inputs.uniform(rng, int(offsets[-1]), -1, 1)
    x = inputs.uniform(rng, cols, -1, 1)
    check(device, offsets, columns, values, x)
    ival = rng.integers(-3, 4, values.shape).astype(np.float32)
    ix = rng.integers(-3, 4, x.shape).astype(np.float32)
    assert (run(device, offsets, columns, ival, ix) == oracle.csr_spmv(offsets, columns, ival, ix)).all()


def test_spmv_large_rows_over_several_batches(device):
    """More than 1024 large rows per slice workgroup (16.8M columns give 1025 slices, one workgroup
    per slice): the slice kernel walks its rows in several LDS batches."""
    announce("spmv large rows over several batches")
    rng = np.random.default_rng(31)
    cols = 1025 * 16384
    lengths = np.full(1300, 16400, np.int64)
    lengths[::13] = 0                                   # 1200 large rows, and empty ones among them
    offsets, columns = inputs.csr_matrix(rng, lengths, cols)
    values = inputs.uniform(rng, int(offsets[-1]), -1, 1)
    x = inputs.uniform(rng, cols, -1, 1)
    check(device, offsets, columns, values, x)


def test_static_workspace_option(device):
    """backend_options={"workspace": "static"} runs csr_spmv through the no-allocation entry point
    (static per-GPU scratch): bit-identical to the default path; problems beyond the scratch are
    refused at prepare."""
    announce("spmv workspace=static")
    rng = np.random.default_rng(77)
    lengths = np.concatenate((rng.integers(0, 5, 20000), rng.integers(5, 300, 3000), rng.integers(300, 9000, 40)))
    offsets, columns = inputs.csr_matrix(rng, lengths[rng.permutation(lengths.shape[0])], 60000)
    values = inputs.uniform(rng, int(offsets[-1]), -1, 1)
    x = inputs.uniform(rng, 60000, -1, 1)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    args = (t(offsets), t(columns), t(values), t(x))
    static = intent.jit(csr_spmv, backend="hip", backend_options={"workspace": "static"})
    call = static.prepare(*args)
    call.launch()
    assert call.observation.entry == "intent_hip_csr_spmv_f32_static"
    want = intent.jit(csr_spmv, backend="hip").run(*args)
    assert torch.equal(call.result(), want)
    big_rows, big_nnz = 1_000_000, 30_000_000
    huge = (torch.zeros(big_rows + 1, dtype=torch.int32, device=device),
            torch.zeros(big_nnz, dtype=torch.int32, device=device),
            torch.zeros(big_nnz, dtype=torch.float32, device=device), torch.zeros(16, device=device))
    with pytest.raises(intent.CompilationStageError) as error:
        static.prepare(*huge)
    assert error.value.stage == "provider_preparation"
