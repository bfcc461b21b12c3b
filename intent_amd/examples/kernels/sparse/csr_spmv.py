"""CSR SpMV definition with symbolic extents.

The reference declares `csr_spmv` with static extents (R = C = 32768, 32 nonzeros per
row; `python/intent/examples/kernels/sparse/csr_spmv.py:5-29`). This definition keeps
its body and parameter order but names the extents, so one artifact serves any
matrix; R1 = R + 1 is checked (and R derived from it) by the hip binder."""
import intent_amd as intent
import intent_amd.language as I

# The reference's static extents (csr_spmv.py:5-8), kept as module constants for callers that
# import them (examples/programs/irregular.py:14-33); the definition below takes any extents.
ROWS = 32768
COLUMNS = 32768
NONZEROS_PER_ROW = 32
NONZEROS = ROWS * NONZEROS_PER_ROW


@intent.kernel
def csr_spmv(
    row_offsets: I.In[I.i32, ("R1",)],
    column_indices: I.In[I.i32, ("NNZ",)],
    values: I.In[I.f32, ("NNZ",)],
    vector: I.In[I.f32, ("C",)],
    output: I.Out[I.f32, ("R",)],
):
    for row in I.parallel(I.domain(0, output.shape[0])):
        acc = I.cast(0.0, I.f32)
        for nz in range(row_offsets[row], row_offsets[row + 1]):
            I.assume_in_bounds(nz, column_indices, axis=0)
            I.assume_in_bounds(nz, values, axis=0)
            column = column_indices[nz]
            I.assume_in_bounds(column, vector, axis=0)
            acc = acc + values[nz] * vector[column]
        output[row] = acc
