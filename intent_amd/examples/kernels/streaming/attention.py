"""Attention forward definitions: flash_attention_fwd, flash_gqa_attention_fwd (key/value heads
shared by HEAD_GROUP query heads), flash_attention_bf16_fwd, flash_attention_bias_fwd and the
packed-sequence forms. Names, signatures and extents are the reference's
(`python/intent/examples/kernels/streaming/attention.py:428-553, 800-924`).

What each computes, per (batch, query head) and query row i:

  logit[i, j] = (q_i . k_j) * scale * log2(e)          f32 accumulation of the storage type
  admitted    = every key, or with CAUSAL the keys j <= i
  peak_i      = largest admitted logit (NaN-ignoring maximum)
  w[i, j]     = exp2(logit - peak_i) on admitted pairs (approximate, subnormals flushed), else 0
  out_i       = (sum_j round(w[i, j]) v_j) * approx_recip(sum_j w[i, j]), stored in the storage type;
                round() is the storage type (f16 or bf16), the sums are f32; a row that admits
                no key is 0.

The bodies below state this densely, one (batch, head) at a time. They are never traced by the hip
provider, which recognises a definition by name and signature. The hand-written kernel streams
the keys in tiles with a running maximum, so its sums are ordered differently; the tests hold it to
the oracle within the tolerance stated there.
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
def causal_pairs(query_positions, key_positions, causal):
    """Which (query, key) pairs take part: all of them, or with `causal` those with key <= query."""
    if causal:
        return query_positions[:, None] >= key_positions[None, :]
    return I.full((query_positions.shape[0], key_positions.shape[0]), fill=True, dtype=I.bool)


@intent.fn
def admitted_attention(logits, admitted, values, element):
    """The unnormalised softmax of each row of base-2 `logits` over its admitted entries, applied
    to `values` with the weights rounded to `element`: `live` (the row admits a key), `peak`,
    `total` (the f32 sum of the weights; 1 where the row is not live) and `mixed` (the weighted
    sum of value rows, f32)."""
    live = I.reduce.any(admitted, axis=1)
    peak = I.select(live, I.reduce(I.select(admitted, logits, -I.inf), axis=1, identity=-I.inf,
                                   combine=I.maximum_num), 0.0)
    weights = I.select(admitted, I.exp2(logits - peak[:, None], approximate=True, flush_to_zero=True), 0.0)
    return I.record(live=live, peak=peak, total=I.select(live, I.reduce.sum(weights, axis=1), 1.0),
                    mixed=I.matmul(I.cast(weights, element), values, acc_dtype=I.f32))


@intent.fn
def attend_head(q_rows, k_rows, v_rows, scale, causal, element):
    logits = I.matmul(q_rows, k_rows, transpose_rhs=True, acc_dtype=I.f32) * (scale * I.LOG2E)
    admitted = causal_pairs(I.indices(I.domain(0, q_rows.shape[0])), I.indices(I.domain(0, k_rows.shape[0])),
                            causal)
    summary = admitted_attention(logits, admitted, v_rows, element)
    share = I.fdiv(1.0, summary.total, approximate=True, flush_to_zero=True)
    return I.cast(I.select(summary.live[:, None], summary.mixed * share[:, None], 0.0), element)


@intent.kernel
def flash_attention_fwd(
    q: I.In[I.f16, ("B", "H", "Q", "D")],
    k: I.In[I.f16, ("B", "H", "K", "D")],
    v: I.In[I.f16, ("B", "H", "K", "DV")],
    output: I.Out[I.f16, ("B", "H", "Q", "DV")],
    scale: I.f32,
    CAUSAL: I.Constexpr[bool],
):
    B, H = q.shape[0], q.shape[1]
    for b in I.parallel(I.domain(0, B)):
        for h in I.parallel(I.domain(0, H)):
            output[b, h, :, :] = attend_head(q[b, h, :, :], k[b, h, :, :], v[b, h, :, :], scale, CAUSAL, I.f16)


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
    B, HQ = q.shape[0], q.shape[1]
    for b in I.parallel(I.domain(0, B)):
        for h in I.parallel(I.domain(0, HQ)):
            shared = h // HEAD_GROUP
            output[b, h, :, :] = attend_head(q[b, h, :, :], k[b, shared, :, :], v[b, shared, :, :], scale, CAUSAL,
                                             I.f16)


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
    B, HQ = q.shape[0], q.shape[1]
    for b in I.parallel(I.domain(0, B)):
        for h in I.parallel(I.domain(0, HQ)):
            shared = h // HEAD_GROUP
            output[b, h, :, :] = attend_head(q[b, h, :, :], k[b, shared, :, :], v[b, shared, :, :], scale, CAUSAL,
                                             I.bf16)


# ------------------------------------------------------------------------------ additive key bias
# flash_attention_bias_fwd (streaming/attention.py:800-836): every key is admitted and its logit
# gains bias[b, h, j] before the base-2 scaling, logit[i, j] = ((q_i . k_j) * scale + bias[j]) *
# log2(e) (summarize_biased_attention_chunk, :328-366). The hip kernel forms it as one fused
# multiply-add, (q_i . k_j) * (scale log2 e) + bias[j] log2 e.
@intent.kernel
def flash_attention_bias_fwd(
    q: I.In[I.f16, ("B", "H", "Q", "D")],
    k: I.In[I.f16, ("B", "H", "K", "D")],
    v: I.In[I.f16, ("B", "H", "K", "DV")],
    bias: I.In[I.f32, ("B", "H", "K")],
    output: I.Out[I.f16, ("B", "H", "Q", "DV")],
    scale: I.f32,
):
    B, H = q.shape[0], q.shape[1]
    for b in I.parallel(I.domain(0, B)):
        for h in I.parallel(I.domain(0, H)):
            q_rows, k_rows = q[b, h, :, :], k[b, h, :, :]
            logits = (I.matmul(q_rows, k_rows, transpose_rhs=True, acc_dtype=I.f32) * scale
                      + bias[b, h, :][None, :]) * I.LOG2E
            admitted = causal_pairs(I.indices(I.domain(0, q_rows.shape[0])), I.indices(I.domain(0, k_rows.shape[0])),
                                    False)
            summary = admitted_attention(logits, admitted, v[b, h, :, :], I.f16)
            share = I.fdiv(1.0, summary.total, approximate=True, flush_to_zero=True)
            output[b, h, :, :] = I.cast(I.select(summary.live[:, None], summary.mixed * share[:, None], 0.0), I.f16)


# ------------------------------------------------------------------------------ packed sequences
# Rows cu_seqlens[s] .. cu_seqlens[s + 1] of q, k, v and output form sequence s, and each sequence
# attends only within itself, with row positions relative to its start (the reference's
# I.ragged over cu_seqlens, streaming/attention.py:839-924). `sequence_lengths` gives the sequence
# count and is otherwise unread, as in the reference; rows outside every sequence are not written.
@intent.kernel
def flash_varlen_attention_fwd(
    q: I.In[I.f16, ("U", "D")],
    k: I.In[I.f16, ("U", "D")],
    v: I.In[I.f16, ("U", "DV")],
    sequence_lengths: I.In[I.i32, ("B",)],
    cu_seqlens: I.In[I.i32, ("B_PLUS_1",)],
    output: I.Out[I.f16, ("U", "DV")],
    scale: I.f32,
    CAUSAL: I.Constexpr[bool],
):
    for s in I.parallel(I.domain(0, sequence_lengths.shape[0])):
        rows = I.domain(cu_seqlens[s], cu_seqlens[s + 1])
        output[rows, :] = attend_head(q[rows, :], k[rows, :], v[rows, :], scale, CAUSAL, I.f16)


@intent.kernel
def flash_varlen_gqa_prefill(
    q: I.In[I.f16, ("U", "HQ", "D")],
    k: I.In[I.f16, ("U", "HK", "D")],
    v: I.In[I.f16, ("U", "HK", "DV")],
    sequence_lengths: I.In[I.i32, ("B",)],
    cu_seqlens: I.In[I.i32, ("B_PLUS_1",)],
    output: I.Out[I.f16, ("U", "HQ", "DV")],
    scale: I.f32,
    HEAD_GROUP: I.Constexpr[int],
):
    for s in I.parallel(I.domain(0, sequence_lengths.shape[0])):
        rows = I.domain(cu_seqlens[s], cu_seqlens[s + 1])
        for h in I.parallel(I.domain(0, q.shape[1])):
            shared = h // HEAD_GROUP
            output[rows, h, :] = attend_head(q[rows, h, :], k[rows, shared, :], v[rows, shared, :], scale, True,
                                             I.f16)
