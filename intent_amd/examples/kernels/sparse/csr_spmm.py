"""CSR SpMM definition with symbolic extents.

The reference declares `csr_spmm` with static extents (ROWS = COLUMNS = 8192, 32 nonzeros per
row, FEATURES = 128; `python/intent/examples/kernels/sparse/csr_spmm.py:5-33`). This definition
keeps its body and parameter order but names the extents, so one artifact serves any matrix;
R1 = R + 1 is checked (and R derived from it) by the hip binder. Per row, the accumulation runs
over the row's nonzeros in order: acc = acc + values[nz] * dense[column, :]."""
import intent_amd as intent
import intent_amd.language as I

ROWS = 8192
COLUMNS = 8192
NONZEROS_PER_ROW = 32
NONZEROS = ROWS * NONZEROS_PER_ROW
FEATURES = 128


@intent.kernel
def csr_spmm(
    row_offsets: I.In[I.i32, ("R1",)],
    column_indices: I.In[I.i32, ("NNZ",)],
    values: I.In[I.f32, ("NNZ",)],
    dense: I.In[I.f32, ("C", "F")],
    output: I.Out[I.f32, ("R", "F")],
):
    features = I.domain(0, dense.shape[1])
    for row in I.parallel(I.domain(0, output.shape[0])):
        accumulation = I.zeros((dense.shape[1],), dtype=I.f32)
        for nonzero in range(row_offsets[row], row_offsets[row + 1]):
            I.assume_in_bounds(nonzero, column_indices, axis=0)
            I.assume_in_bounds(nonzero, values, axis=0)
            column = column_indices[nonzero]
            I.assume_in_bounds(column, dense, axis=0)
            accumulation = accumulation + values[nonzero] * dense[column, features]
        output[row, features] = accumulation
