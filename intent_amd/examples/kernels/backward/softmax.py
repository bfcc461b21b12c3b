"""Softmax backward definitions.

`softmax_backward` keeps the reference's static f32 contract
(`python/intent/examples/kernels/backward/softmax.py:5-25`, 4096 x 4097).
`softmax_backward_f16` is the f16-storage / f32-accumulation variant of the same
body with symbolic extents, derived the way `stable_softmax_f16` derives from
`stable_softmax` (cast in, f32 reduce, cast out); the reference has no f16 backward."""
import intent_amd as intent
import intent_amd.language as I

ROWS = 4096
COLUMNS = 4097


@intent.kernel
def softmax_backward(
    probabilities: I.In[I.f32, (ROWS, COLUMNS)],
    upstream: I.In[I.f32, (ROWS, COLUMNS)],
    gradient: I.Out[I.f32, (ROWS, COLUMNS)],
):
    columns = I.domain(0, COLUMNS)
    for row in I.parallel(I.domain(0, ROWS)):
        p = probabilities[row, columns]
        g = upstream[row, columns]
        gradient[row, columns] = p * (g - I.reduce.sum(p * g, axis=0))


@intent.kernel
def softmax_backward_f16(
    probabilities: I.In[I.f16, ("M", "N")],
    upstream: I.In[I.f16, ("M", "N")],
    gradient: I.Out[I.f16, ("M", "N")],
):
    M, N = probabilities.shape
    columns = I.domain(0, N)
    for row in I.parallel(I.domain(0, M)):
        p = I.cast(probabilities[row, columns], I.f32)
        g = I.cast(upstream[row, columns], I.f32)
        gradient[row, columns] = I.cast(p * (g - I.reduce.sum(p * g, axis=0)), I.f16)
