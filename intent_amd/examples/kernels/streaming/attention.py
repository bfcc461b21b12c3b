"""Fused attention forward definitions (interface and semantics of the reference's
`python/intent/examples/kernels/streaming/attention.py:47-237, 417-553`): flash_attention_fwd,
flash_gqa_attention_fwd (grouped key/value heads) and flash_attention_bf16_fwd.

A region fold over key chunks keeps, per query row, a summary record
(valid, maximum, denominator, accumulator) in the exp2 domain:
  chunk:   s = (q . k^T) * scale * log2(e); causal validity q_idx >= k_idx; masked -inf;
           m = maximum_num of valid scores (0 when none valid); p = exp2(s - m) (approximate,
           flush-to-zero) on valid keys; den = sum p; acc = cast(p, f16) @ v (f32 accumulate)
  merge:   m = maximum_num of the valid maxima; each side scaled by exp2(m_side - m)
  output:  acc * approx_reciprocal(den) for valid rows, 0 otherwise; cast to f16
"""
import math

import intent_amd as intent
import intent_amd.language as I

# The reference's example extents (streaming/attention.py:7-11), kept as module constants for
# callers that import them; the definitions below take any extents.
BATCH = 4
HEADS = 32
SEQUENCE = 4096
HEAD_DIMENSION = 128
SCALE = 1.0 / math.sqrt(HEAD_DIMENSION)


@intent.fn
def maximum_score(lhs, rhs):
    return I.maximum_num(lhs, rhs)


@intent.fn
def reduce_score_maximum(scores, axis):
    return I.reduce(scores, axis=axis, identity=-I.inf, combine=maximum_score)


@intent.fn
def empty_attention_summary(query_count, value_width):
    return I.record(
        valid=I.full((query_count,), fill=False, dtype=I.bool),
        maximum=I.full((query_count,), fill=0.0, dtype=I.f32),
        denominator=I.zeros((query_count,), dtype=I.f32),
        accumulator=I.zeros((query_count, value_width), dtype=I.f32),
    )


@intent.fn
def merge_attention_summaries(lhs, rhs):
    merged_max = I.select(lhs.valid, lhs.maximum, rhs.maximum)
    merged_max = I.select(rhs.valid, I.maximum_num(merged_max, rhs.maximum), merged_max)
    left = I.select(lhs.valid, I.exp2(I.select(lhs.valid, lhs.maximum, merged_max) - merged_max,
                                      approximate=True, flush_to_zero=True), 0.0)
    right = I.select(rhs.valid, I.exp2(I.select(rhs.valid, rhs.maximum, merged_max) - merged_max,
                                       approximate=True, flush_to_zero=True), 0.0)
    return I.record(
        valid=lhs.valid | rhs.valid,
        maximum=merged_max,
        denominator=left * lhs.denominator + right * rhs.denominator,
        accumulator=left[:, None] * lhs.accumulator + right[:, None] * rhs.accumulator,
    )


@intent.fn
def summarize_attention_chunk_f16(key_chunk, value_chunk, key_coordinates, queries, query_coordinates,
                                  scale, causal):
    scores = I.matmul(queries, key_chunk, transpose_rhs=True, acc_dtype=I.f32) * (scale * I.LOG2E)
    valid = I.full(scores.shape, fill=True, dtype=I.bool)
    if causal:
        valid = query_coordinates[:, None] >= key_coordinates[None, :]
    masked = I.select(valid, scores, -I.inf)
    any_valid = I.reduce.any(valid, axis=1)
    chunk_max = I.select(any_valid, reduce_score_maximum(masked, axis=1), 0.0)
    weights = I.select(valid, I.exp2(masked - chunk_max[:, None], approximate=True, flush_to_zero=True), 0.0)
    return I.record(
        valid=any_valid,
        maximum=chunk_max,
        denominator=I.reduce.sum(weights, axis=1),
        accumulator=I.select(any_valid[:, None],
                             I.matmul(I.cast(weights, I.f16), value_chunk, acc_dtype=I.f32), 0.0),
    )


@intent.fn
def summarize_attention_chunk_bf16(key_chunk, value_chunk, key_coordinates, queries, query_coordinates,
                                   scale, causal, active):
    scores = I.matmul(queries, key_chunk, transpose_rhs=True, acc_dtype=I.f32) * (scale * I.LOG2E)
    valid = I.full(scores.shape, fill=True, dtype=I.bool) & active
    if causal:
        valid = valid & (query_coordinates[:, None] >= key_coordinates[None, :])
    masked = I.select(valid, scores, -I.inf)
    any_valid = I.reduce.any(valid, axis=1)
    chunk_max = I.select(any_valid, reduce_score_maximum(masked, axis=1), 0.0)
    weights = I.select(valid, I.exp2(masked - chunk_max[:, None], approximate=True, flush_to_zero=True), 0.0)
    return I.record(
        valid=any_valid,
        maximum=chunk_max,
        denominator=I.reduce.sum(weights, axis=1),
        accumulator=I.select(any_valid[:, None],
                             I.matmul(I.cast(weights, I.bf16), value_chunk, acc_dtype=I.f32), 0.0),
    )


@intent.fn
def summarize_masked_attention_chunk(key_chunk, value_chunk, key_coordinates, active, queries, query_coordinates,
                                     scale):
    """Decode chunk summary: every pair of an active key is valid (attention.py:250-290)."""
    scores = I.matmul(queries, key_chunk, transpose_rhs=True, acc_dtype=I.f32) * (scale * I.LOG2E)
    valid = I.full(scores.shape, fill=True, dtype=I.bool) & active[None, :]
    masked = I.select(valid, scores, -I.inf)
    any_valid = I.reduce.any(valid, axis=1)
    chunk_max = I.select(any_valid, reduce_score_maximum(masked, axis=1), 0.0)
    weights = I.select(valid, I.exp2(masked - chunk_max[:, None], approximate=True, flush_to_zero=True), 0.0)
    return I.record(valid=any_valid, maximum=chunk_max, denominator=I.reduce.sum(weights, axis=1),
                    accumulator=I.matmul(I.cast(weights, I.f16), value_chunk, acc_dtype=I.f32))


@intent.fn
def normalize_attention_summary(summary):
    denominator = I.select(summary.valid, summary.denominator, 1.0)
    reciprocal = I.fdiv(1.0, denominator, approximate=True, flush_to_zero=True)
    return I.select(summary.valid[:, None], summary.accumulator * reciprocal[:, None], 0.0)


@intent.kernel
def flash_attention_fwd(
    q: I.In[I.f16, ("B", "H", "Q", "D")],
    k: I.In[I.f16, ("B", "H", "K", "D")],
    v: I.In[I.f16, ("B", "H", "K", "DV")],
    output: I.Out[I.f16, ("B", "H", "Q", "DV")],
    scale: I.f32,
    CAUSAL: I.Constexpr[bool],
):
    B, H, Q, _ = q.shape
    K = k.shape[2]
    DV = v.shape[3]
    q_axis, k_axis = I.domain(0, Q), I.domain(0, K)
    for batch in I.parallel(I.domain(0, B)):
        for head in I.parallel(I.domain(0, H)):
            summary = I.region_fold(
                source=(k[batch, head, k_axis, :], v[batch, head, k_axis, :], I.indices(k_axis)),
                axis=0,
                summarize=summarize_attention_chunk_f16,
                combine=merge_attention_summaries,
                identity=empty_attention_summary(Q, DV),
                operands=(q[batch, head, q_axis, :], I.indices(q_axis), scale, CAUSAL),
            )
            output[batch, head, q_axis, :] = I.cast(normalize_attention_summary(summary), I.f16)


@intent.kernel
def flash_gqa_attention_fwd(
    q: I.In[I.f16, ("B", "HQ", "Q", "D")],
    k: I.In[I.f16, ("B", "HK", "K", "D")],
    v: I.In[I.f16, ("B", "HK", "K", "DV")],
    output: I.Out[I.f16, ("B", "HQ", "Q", "DV")],
    scale: I.f32,
    HEAD_GROUP: I.Constexpr[int],
    CAUSAL: I.Constexpr[bool],
):
    B, HQ, Q, _ = q.shape
    K = k.shape[2]
    DV = v.shape[3]
    q_axis, k_axis = I.domain(0, Q), I.domain(0, K)
    for batch in I.parallel(I.domain(0, B)):
        for query_head in I.parallel(I.domain(0, HQ)):
            key_head = query_head // HEAD_GROUP
            summary = I.region_fold(
                source=(k[batch, key_head, k_axis, :], v[batch, key_head, k_axis, :], I.indices(k_axis)),
                axis=0,
                summarize=summarize_attention_chunk_f16,
                combine=merge_attention_summaries,
                identity=empty_attention_summary(Q, DV),
                operands=(q[batch, query_head, q_axis, :], I.indices(q_axis), scale, CAUSAL),
            )
            output[batch, query_head, q_axis, :] = I.cast(normalize_attention_summary(summary), I.f16)


@intent.kernel
def flash_attention_bf16_fwd(
    q: I.In[I.bf16, ("B", "HQ", "Q", "D")],
    k: I.In[I.bf16, ("B", "HK", "K", "D")],
    v: I.In[I.bf16, ("B", "HK", "K", "DV")],
    output: I.Out[I.bf16, ("B", "HQ", "Q", "DV")],
    scale: I.f32,
    HEAD_GROUP: I.Constexpr[int],
    CAUSAL: I.Constexpr[bool],
):
    B, HQ, Q, _ = q.shape
    K = k.shape[2]
    DV = v.shape[3]
    q_axis, k_axis = I.domain(0, Q), I.domain(0, K)
    for batch in I.parallel(I.domain(0, B)):
        for query_head in I.parallel(I.domain(0, HQ)):
            key_head = query_head // HEAD_GROUP
            summary = I.region_fold(
                source=(k[batch, key_head, k_axis, :], v[batch, key_head, k_axis, :], I.indices(k_axis)),
                axis=0,
                summarize=summarize_attention_chunk_bf16,
                combine=merge_attention_summaries,
                identity=empty_attention_summary(Q, DV),
                operands=(q[batch, query_head, q_axis, :], I.indices(q_axis), scale, CAUSAL, True),
            )
            output[batch, query_head, q_axis, :] = I.cast(normalize_attention_summary(summary), I.bf16)
