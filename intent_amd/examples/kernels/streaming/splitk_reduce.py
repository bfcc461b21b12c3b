"""Split-K attention merge, splitk_attention_f32_to_f16_reduce. Name, signature and example
extents are the reference's (`python/intent/examples/kernels/streaming/splitk_reduce.py:129-155`).

Per (batch, head), the S partial rows are combined with weights w_s = exp(lse_s - max_s lse_s).
The maximum ignores NaN and the exponential is natural. The output is
f16((sum_s w_s partial_s) * approx_recip(sum_s w_s)), with the sums in f32.
"""
import intent_amd as intent
import intent_amd.language as I

BATCH = 8
HEADS = 32
SPLITS = 16
HEAD_DIMENSION = 128


@intent.kernel
def splitk_attention_f32_to_f16_reduce(
    partial: I.In[I.f32, ("B", "H", "S", "D")],
    partial_lse: I.In[I.f32, ("B", "H", "S")],
    output: I.Out[I.f16, ("B", "H", "D")],
):
    B, H = partial.shape[0], partial.shape[1]
    for b in I.parallel(I.domain(0, B)):
        for h in I.parallel(I.domain(0, H)):
            lse = partial_lse[b, h, :]
            w = I.exp(lse - I.reduce(lse, axis=0, identity=-I.inf, combine=I.maximum_num))
            merged = I.vecmat(w, partial[b, h, :, :], acc_dtype=I.f32)
            output[b, h, :] = I.cast(merged * I.fdiv(1.0, I.reduce.sum(w, axis=0), approximate=True,
                                                     flush_to_zero=True), I.f16)
