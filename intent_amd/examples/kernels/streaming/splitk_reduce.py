"""Split-K attention merge (interface and semantics of the reference's
`python/intent/examples/kernels/streaming/splitk_reduce.py:129-155`, splitk_attention_f32_to_f16_reduce):
per (batch, head): m = maximum_num over splits of partial_lse; w = exp(partial_lse - m) (natural
exponential, as written); output = f16((sum w * partial) * approximate_reciprocal(sum w)).
"""
import intent_amd as intent
import intent_amd.language as I

from intent_amd.examples.kernels.streaming.attention import reduce_score_maximum

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
    B, H, S, D = partial.shape
    splits, dims = I.domain(0, S), I.domain(0, D)
    for batch in I.parallel(I.domain(0, B)):
        for head in I.parallel(I.domain(0, H)):
            lse = partial_lse[batch, head, splits]
            weights = I.exp(lse - reduce_score_maximum(lse, axis=0))
            numerator = I.vecmat(weights, partial[batch, head, splits, dims], acc_dtype=I.f32)
            output[batch, head, dims] = I.cast(
                numerator * I.fdiv(1.0, I.reduce.sum(weights, axis=0), approximate=True, flush_to_zero=True), I.f16)
