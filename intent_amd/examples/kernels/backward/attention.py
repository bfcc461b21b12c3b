"""Attention backward definitions: attention_backward_delta, attention_backward_dkdv and
attention_backward_dq, for grouped-query attention with f16 storage and f32 arithmetic. Names,
signatures and example extents are the reference's
(`python/intent/examples/kernels/backward/attention.py:17-211`).

For query head h (key head h // HEAD_GROUP), query row i and key row j:

  delta_i  = sum_d f32(out_id) * f32(dout_id)
  taken    = every pair, or with CAUSAL the pairs j <= i
  P_ij     = exp2(s_ij * scale * log2(e) - lse_i * log2(e)) with s_ij = q_i . k_j
             (approximate exp2, subnormals flushed); lse is the natural log of the forward's
             softmax denominator
  dS_ij    = P_ij * (dout_i . v_j - delta_i)
  dQ_i     = scale * sum_j f16(dS_ij) k_j
  dK_j     = scale * sum_(h, i) f16(dS_ij) q_i,   dV_j = sum_(h, i) f16(P_ij) dout_i

The (h, i) sums run over every query row of the HEAD_GROUP query heads that share key j's head.
Every sum includes only the pairs that are taken. A pair that is not taken adds nothing, even when a row it would
touch holds inf or NaN (a zero weight times inf would give NaN). All sums are f32. The kernels add
in their own order, so results match any order of the same sum to f32 rounding.

The bodies state this one head at a time. The hip provider recognises a definition by name and
signature and runs its own kernels.
"""
import math

import intent_amd as intent
import intent_amd.language as I

BATCH = 2
QUERY_HEADS = 8
KV_HEADS = 2
HEAD_GROUP = QUERY_HEADS // KV_HEADS
SEQUENCE = 1024
HEAD_DIMENSION = 64
SCALE = 1.0 / math.sqrt(HEAD_DIMENSION)


@intent.fn
def taken_pairs(query_count, key_count, causal):
    rows, cols = I.indices(I.domain(0, query_count)), I.indices(I.domain(0, key_count))
    if causal:
        return rows[:, None] >= cols[None, :]
    return I.full((query_count, key_count), fill=True, dtype=I.bool)


@intent.fn
def pair_weights(q_rows, k_rows, lse_rows, scale, taken):
    """P of one query head against one key head, 0 on pairs that are not taken."""
    s = I.matmul(q_rows, k_rows, transpose_rhs=True, acc_dtype=I.f32)
    return I.select(taken, I.exp2(s * (scale * I.LOG2E) - lse_rows[:, None] * I.LOG2E, approximate=True,
                                  flush_to_zero=True), 0.0)


@intent.fn
def taken_sum(weights, rows, taken):
    """out[a, :] = sum over b with taken[a, b] of f32(weights[a, b]) * f32(rows[b, :]).
    A pair that is not taken is left out of the sum, not multiplied by zero."""
    terms = I.cast(weights, I.f32)[:, :, None] * I.cast(rows, I.f32)[None, :, :]
    return I.reduce.sum(I.select(taken[:, :, None], terms, 0.0), axis=1)


@intent.kernel
def attention_backward_delta(
    output: I.In[I.f16, ("B", "HQ", "Q", "D")],
    grad_output: I.In[I.f16, ("B", "HQ", "Q", "D")],
    delta: I.Out[I.f32, ("B", "HQ", "Q")],
):
    B, HQ = output.shape[0], output.shape[1]
    for b in I.parallel(I.domain(0, B)):
        for h in I.parallel(I.domain(0, HQ)):
            delta[b, h, :] = I.reduce.sum(I.cast(output[b, h, :, :], I.f32) * I.cast(grad_output[b, h, :, :], I.f32),
                                          axis=1)


@intent.kernel
def attention_backward_dkdv(
    q: I.In[I.f16, ("B", "HQ", "Q", "D")],
    k: I.In[I.f16, ("B", "HK", "K", "D")],
    v: I.In[I.f16, ("B", "HK", "K", "D")],
    grad_output: I.In[I.f16, ("B", "HQ", "Q", "D")],
    lse: I.In[I.f32, ("B", "HQ", "Q")],
    delta: I.In[I.f32, ("B", "HQ", "Q")],
    grad_k: I.Out[I.f16, ("B", "HK", "K", "D")],
    grad_v: I.Out[I.f16, ("B", "HK", "K", "D")],
    scale: I.f32,
    HEAD_GROUP: I.Constexpr[int],
    CAUSAL: I.Constexpr[bool],
):
    B, Q, D = q.shape[0], q.shape[2], q.shape[3]
    HK, K = k.shape[1], k.shape[2]
    taken = taken_pairs(Q, K, CAUSAL)                                     # [Q, K]
    for b in I.parallel(I.domain(0, B)):
        for kv in I.parallel(I.domain(0, HK)):
            keys, values = k[b, kv, :, :], v[b, kv, :, :]
            dk, dv = I.zeros((K, D), dtype=I.f32), I.zeros((K, D), dtype=I.f32)
            for member in range(HEAD_GROUP):
                h = kv * HEAD_GROUP + member
                queries, upstream = q[b, h, :, :], grad_output[b, h, :, :]
                p = pair_weights(queries, keys, lse[b, h, :], scale, taken)                 # [Q, K]
                ds = p * (I.matmul(upstream, values, transpose_rhs=True, acc_dtype=I.f32) - delta[b, h, :][:, None])
                dv = dv + taken_sum(I.transpose(I.cast(p, I.f16)), upstream, I.transpose(taken))
                dk = dk + taken_sum(I.transpose(I.cast(ds, I.f16)), queries, I.transpose(taken))
            grad_k[b, kv, :, :] = I.cast(dk * scale, I.f16)
            grad_v[b, kv, :, :] = I.cast(dv, I.f16)


@intent.kernel
def attention_backward_dq(
    q: I.In[I.f16, ("B", "HQ", "Q", "D")],
    k: I.In[I.f16, ("B", "HK", "K", "D")],
    v: I.In[I.f16, ("B", "HK", "K", "D")],
    grad_output: I.In[I.f16, ("B", "HQ", "Q", "D")],
    lse: I.In[I.f32, ("B", "HQ", "Q")],
    delta: I.In[I.f32, ("B", "HQ", "Q")],
    grad_q: I.Out[I.f16, ("B", "HQ", "Q", "D"), I.constraints(noalias=True)],
    scale: I.f32,
    HEAD_GROUP: I.Constexpr[int],
    CAUSAL: I.Constexpr[bool],
):
    B, HQ, Q = q.shape[0], q.shape[1], q.shape[2]
    K = k.shape[2]
    taken = taken_pairs(Q, K, CAUSAL)                                     # [Q, K]
    for b in I.parallel(I.domain(0, B)):
        for h in I.parallel(I.domain(0, HQ)):
            keys, values = k[b, h // HEAD_GROUP, :, :], v[b, h // HEAD_GROUP, :, :]
            p = pair_weights(q[b, h, :, :], keys, lse[b, h, :], scale, taken)
            dp = I.matmul(grad_output[b, h, :, :], values, transpose_rhs=True, acc_dtype=I.f32)
            ds = p * (dp - delta[b, h, :][:, None])
            grad_q[b, h, :, :] = I.cast(taken_sum(I.cast(ds, I.f16), keys, taken) * scale, I.f16)
