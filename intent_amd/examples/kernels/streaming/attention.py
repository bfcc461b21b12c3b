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
# Decode extents of the reference's examples (streaming/attention.py:18-34).
GQA_DECODE_BATCH, GQA_DECODE_QUERY_HEADS, GQA_DECODE_KV_HEADS = 32, 32, 8
GQA_DECODE_SEQUENCE, GQA_DECODE_HEAD_DIMENSION = 8192, 128
VARLEN_GQA_DECODE_BATCH, VARLEN_GQA_DECODE_QUERY_HEADS, VARLEN_GQA_DECODE_KV_HEADS = 8, 32, 8
VARLEN_GQA_DECODE_HEAD_DIMENSION, VARLEN_GQA_DECODE_BLOCK_SIZE, VARLEN_GQA_DECODE_MAX_BLOCKS = 64, 64, 64


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


# ------------------------------------------------------------------------------ latent attention
# mla_prefill (streaming/attention.py:756-798): each score adds a position product, qpe . kpe, to
# the content product q . k before the base-2 scaling (summarize_mla_chunk, :368-415); kpe has one
# row per key shared by every head; causal, with key heads shared by HEAD_GROUP query heads.
@intent.kernel
def mla_prefill(
    q: I.In[I.f16, ("B", "H", "Q", "D")],
    qpe: I.In[I.f16, ("B", "H", "Q", "P")],
    k: I.In[I.f16, ("B", "HK", "K", "D")],
    kpe: I.In[I.f16, ("B", 1, "K", "P")],
    v: I.In[I.f16, ("B", "HK", "K", "D")],
    output: I.Out[I.f16, ("B", "H", "Q", "D")],
    scale: I.f32,
    HEAD_GROUP: I.Constexpr[int],
):
    B, H = q.shape[0], q.shape[1]
    for b in I.parallel(I.domain(0, B)):
        for h in I.parallel(I.domain(0, H)):
            shared = h // HEAD_GROUP
            logits = (I.matmul(q[b, h, :, :], k[b, shared, :, :], transpose_rhs=True, acc_dtype=I.f32)
                      + I.matmul(qpe[b, h, :, :], kpe[b, 0, :, :], transpose_rhs=True, acc_dtype=I.f32)) * (
                          scale * I.LOG2E)
            admitted = causal_pairs(I.indices(I.domain(0, q.shape[2])), I.indices(I.domain(0, k.shape[2])), True)
            summary = admitted_attention(logits, admitted, v[b, shared, :, :], I.f16)
            share = I.fdiv(1.0, summary.total, approximate=True, flush_to_zero=True)
            output[b, h, :, :] = I.cast(I.select(summary.live[:, None], summary.mixed * share[:, None], 0.0), I.f16)


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


# ------------------------------------------------------------------------------ decode
# One query row per (batch, query head) against a key/value cache (streaming/attention.py:556-754).
# Each definition folds its keys as the forward ones do (exp2-domain logits, weights rounded to the
# storage type before they weigh the values); they differ in where the keys live and what is kept.
@intent.fn
def decode_summary(query_row, k_rows, v_rows, admitted, scale, element):
    logits = I.matmul(query_row, k_rows, transpose_rhs=True, acc_dtype=I.f32) * (scale * I.LOG2E)
    return admitted_attention(logits, admitted, v_rows, element)


@intent.kernel
def grouped_flash_decode_partials(
    q: I.In[I.bf16, ("B", "HQ", 1, "D")],
    k: I.In[I.bf16, ("B", "HK", "K", "D")],
    v: I.In[I.bf16, ("B", "HK", "K", "DV")],
    partial_lse: I.Out[I.f32, ("B", "HQ", "P")],
    partial_output: I.Out[I.bf16, ("B", "HQ", "P", "DV")],
    scale: I.f32,
    HEAD_GROUP: I.Constexpr[int],
    P: I.Constexpr[int],
    SPLIT_SIZE: I.Constexpr[int],
):
    """Part p of every (batch, query head) covers key slots p * SPLIT_SIZE .. + SPLIT_SIZE of its
    key head, those below K taking part. It keeps the part's base-2 log-sum (peak + log2 of the
    weight total; -inf when no slot takes part) and its normalised mix in bf16 (0 when none)."""
    B, HQ, K = q.shape[0], q.shape[1], k.shape[2]
    for b in I.parallel(I.domain(0, B)):
        for h in I.parallel(I.domain(0, HQ)):
            shared = h // HEAD_GROUP
            for part in I.parallel(I.domain(0, P)):
                keys = I.domain(I.minimum(part * SPLIT_SIZE, K), I.minimum((part + 1) * SPLIT_SIZE, K))
                admitted = causal_pairs(I.indices(I.domain(0, 1)), I.indices(keys), False)
                summary = decode_summary(q[b, h, :, :], k[b, shared, keys, :], v[b, shared, keys, :], admitted,
                                         scale, I.bf16)
                share = I.fdiv(1.0, summary.total, approximate=True, flush_to_zero=True)
                partial_lse[b, h, part] = I.select(summary.live[0], summary.peak[0] + I.log(summary.total[0]) * I.LOG2E,
                                                   -I.inf)
                partial_output[b, h, part, :] = I.cast(I.select(summary.live[0], summary.mixed[0] * share[0], 0.0),
                                                       I.bf16)


@intent.kernel
def continuous_gqa_decode(
    q: I.In[I.f16, ("B", "HQ", "D")],
    k: I.In[I.f16, ("B", "K", "HK", "D")],
    v: I.In[I.f16, ("B", "K", "HK", "DV")],
    valid_mask: I.In[I.u8, ("B", "K", "HK")],
    output: I.Out[I.f16, ("B", "HQ", "DV")],
    scale: I.f32,
    HEAD_GROUP: I.Constexpr[int],
):
    """Token-major cache; key j of key head kh takes part where valid_mask[b, j, kh] is nonzero. A
    query with no admitted key gives 0."""
    B, HQ, D = q.shape
    for b in I.parallel(I.domain(0, B)):
        for h in I.parallel(I.domain(0, HQ)):
            shared = h // HEAD_GROUP
            admitted = (valid_mask[b, :, shared] != 0)[None, :]
            summary = decode_summary(I.reshape(q[b, h, :], (1, D)), k[b, :, shared, :], v[b, :, shared, :], admitted,
                                     scale, I.f16)
            share = I.fdiv(1.0, summary.total, approximate=True, flush_to_zero=True)
            output[b, h, :] = I.cast(I.select(summary.live[0], summary.mixed[0] * share[0], 0.0), I.f16)


@intent.kernel
def varlen_gqa_decode_with_sink_logits(
    q: I.In[I.f16, ("B", "HQ", "D")],
    k: I.In[I.f16, ("U", "HK", "D")],
    v: I.In[I.f16, ("U", "HK", "DV")],
    cu_seqlens: I.In[I.i32, ("B_PLUS_1",)],
    sink: I.In[I.f32, ("HQ",)],
    output: I.Out[I.f16, ("B", "HQ", "DV")],
    block_logits: I.Out[I.f32, ("B", "HQ", VARLEN_GQA_DECODE_MAX_BLOCKS)],
    scale: I.f32,
    HEAD_GROUP: I.Constexpr[int],
    MAX_BLOCKS: I.Constexpr[int],
):
    """Sequence s's keys are rows cu_seqlens[s] .. cu_seqlens[s + 1], folded in blocks of
    VARLEN_GQA_DECODE_BLOCK_SIZE; only the first MAX_BLOCKS blocks are read. With `peak` the
    largest block peak and `total` the weight total against it, the sink of the query head joins
    the total: output = mix / (total + sink[h]); block j's logit is exp2(peak_j - peak) / (total +
    sink[h]) for the sequence's blocks, 0 past them. An empty sequence gives 0 everywhere."""
    B, HQ, D = q.shape
    size = VARLEN_GQA_DECODE_BLOCK_SIZE
    for s in I.parallel(I.domain(0, B)):
        begin, end = cu_seqlens[s], cu_seqlens[s + 1]
        blocks = (end - begin + size - 1) // size
        for h in I.parallel(I.domain(0, HQ)):
            shared = h // HEAD_GROUP
            query = I.reshape(q[s, h, :], (1, D))
            rows = I.domain(begin, I.minimum(end, begin + size * MAX_BLOCKS))
            admitted = causal_pairs(I.indices(I.domain(0, 1)), I.indices(rows), False)
            summary = decode_summary(query, k[rows, shared, :], v[rows, shared, :], admitted, scale, I.f16)
            share = I.fdiv(1.0, I.select(summary.live[0], summary.total[0] + sink[h], 1.0), approximate=True,
                           flush_to_zero=True)
            output[s, h, :] = I.cast(I.select(summary.live[0], summary.mixed[0] * share, 0.0), I.f16)
            for j in I.domain(0, MAX_BLOCKS):
                block = I.domain(I.minimum(begin + j * size, end), I.minimum(begin + (j + 1) * size, end))
                peak_j = decode_summary(query, k[block, shared, :], v[block, shared, :],
                                        causal_pairs(I.indices(I.domain(0, 1)), I.indices(block), False), scale,
                                        I.f16).peak[0]
                block_logits[s, h, j] = I.select(j < blocks,
                                                 I.exp2(peak_j - summary.peak[0], approximate=True,
                                                        flush_to_zero=True) * share, 0.0)
