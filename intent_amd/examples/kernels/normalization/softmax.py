"""Row softmax definitions (interface and semantics of the reference's
`python/intent/examples/kernels/normalization/softmax.py:6-66`).

The bodies state the algorithm in the kernel language; the hip provider runs a
hand-written kernel for each definition and never executes a body."""
import intent_amd as intent
import intent_amd.language as I

# The reference's example extents (normalization/softmax.py:4-5), kept as module constants for
# callers that import them; the definitions below take any extents.
ROWS = 8192
COLUMNS = 8192

ROW_MAJOR_NOALIAS = I.constraints(strides=(None, 1), noalias=True)


@intent.fn
def maximum_number(lhs, rhs):
    return I.maximum_num(lhs, rhs)


@intent.fn
def softmax_maximum(values):
    # maximum_num skips a one-sided NaN here, but a NaN still reaches every output
    # through the exponential sum.
    return I.reduce(values, axis=0, identity=-I.inf, combine=maximum_number)


@intent.kernel
def stable_softmax(
    x: I.In[I.f32, ("M", "N"), ROW_MAJOR_NOALIAS],
    y: I.Out[I.f32, ("M", "N"), ROW_MAJOR_NOALIAS],
):
    M, N = x.shape
    columns = I.domain(0, N)
    for row in I.parallel(I.domain(0, M)):
        values = x[row, columns]
        shifted = I.exp(values - softmax_maximum(values))
        y[row, columns] = shifted * (1.0 / I.reduce.sum(shifted, axis=0))


@intent.kernel
def stable_softmax_f16(
    x: I.In[I.f16, ("M", "N")],
    y: I.Out[I.f16, ("M", "N")],
):
    M, N = x.shape
    columns = I.domain(0, N)
    for row in I.parallel(I.domain(0, M)):
        values = I.cast(x[row, columns], I.f32)
        shifted = I.exp(values - softmax_maximum(values))
        y[row, columns] = I.cast(shifted / I.reduce.sum(shifted, axis=0), I.f16)


@intent.kernel
def chunked_softmax_bf16(
    x: I.In[I.bf16, ("M", "N")],
    y: I.Out[I.bf16, ("M", "N")],
):
    M, N = x.shape
    columns = I.domain(0, N)
    for row in I.parallel(I.domain(0, M)):
        values = I.cast(x[row, columns], I.f32)
        shifted = I.exp(values - softmax_maximum(values))
        y[row, columns] = I.cast(shifted / I.reduce.sum(shifted, axis=0), I.bf16)
