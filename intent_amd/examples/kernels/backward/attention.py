"""Attention backward definitions (interface and semantics of the reference's
`python/intent/examples/kernels/backward/attention.py:17-211`): delta, dK/dV and dQ of a
grouped-query attention with f16 storage and f32 arithmetic.

  delta[b,h,q] = sum_d o * do
  p  = exp2(s * scale * log2(e) - lse * log2(e)), s = q . k  (approximate, flush-to-zero),
       lse the natural log of the forward's softmax denominator; causal pairs need q >= k
  dv = sum_q f16(p) * do;  dp = do . v;  ds = p * (dp - delta)
  dk = scale * sum_q f16(ds) * q;  dq = scale * sum_k f16(ds) * k
Causally excluded pairs contribute nothing, even with non-finite operands; the summed axes are
region folds combined by addition. Key head of query head h: h // HEAD_GROUP.
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


@intent.kernel
def attention_backward_delta(
    output: I.In[I.f16, ("B", "HQ", "Q", "D")],
    grad_output: I.In[I.f16, ("B", "HQ", "Q", "D")],
    delta: I.Out[I.f32, ("B", "HQ", "Q")],
):
    B, HQ, Q, _ = output.shape
    rows = I.domain(0, Q)
    for batch in I.parallel(I.domain(0, B)):
        for head in I.parallel(I.domain(0, HQ)):
            delta[batch, head, rows] = I.reduce.sum(
                I.cast(output[batch, head, rows, :], I.f32) * I.cast(grad_output[batch, head, rows, :], I.f32),
                axis=1)


@intent.fn
def masked_gradient_product(weights, operands, valid):
    products = I.cast(weights, I.f32)[:, :, None] * I.cast(operands, I.f32)[None, :, :]
    return I.reduce.sum(I.mask(products, valid=valid[:, :, None], fill=0.0), axis=1)


@intent.fn
def summarize_key_value_gradients(queries, grad_outputs, lse, delta, query_coordinates,
                                  keys, values, key_coordinates, scale, causal):
    scores = I.matmul(keys, queries, transpose_rhs=True, acc_dtype=I.f32)
    weights = I.exp2(scores * (scale * I.LOG2E) - lse[None, :] * I.LOG2E, approximate=True, flush_to_zero=True)
    if causal:
        valid = key_coordinates[:, None] <= query_coordinates[None, :]
        weights = I.mask(weights, valid=valid, fill=0.0)
        grad_values = masked_gradient_product(I.cast(weights, I.f16), grad_outputs, valid)
    else:
        grad_values = I.matmul(I.cast(weights, I.f16), grad_outputs, acc_dtype=I.f32)
    grad_weights = I.matmul(values, grad_outputs, transpose_rhs=True, acc_dtype=I.f32)
    grad_scores = weights * (grad_weights - delta[None, :])
    if causal:
        grad_keys = masked_gradient_product(I.cast(grad_scores, I.f16), queries, valid)
    else:
        grad_keys = I.matmul(I.cast(grad_scores, I.f16), queries, acc_dtype=I.f32)
    return I.record(grad_k=grad_keys, grad_v=grad_values)


@intent.fn
def merge_key_value_gradients(lhs, rhs):
    return I.record(grad_k=lhs.grad_k + rhs.grad_k, grad_v=lhs.grad_v + rhs.grad_v)


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
    B, HQ, Q, D = q.shape
    _, HK, K, _ = k.shape
    keys = I.domain(0, K)
    group = I.domain(0, HEAD_GROUP * Q)
    for batch in I.parallel(I.domain(0, B)):
        for key_head in I.parallel(I.domain(0, HK)):
            member = I.indices(group)
            heads = key_head * HEAD_GROUP + member // Q
            rows = member % Q
            summary = I.region_fold(
                source=(q[batch, heads, rows, :], grad_output[batch, heads, rows, :], lse[batch, heads, rows],
                        delta[batch, heads, rows], rows),
                axis=0,
                summarize=summarize_key_value_gradients,
                combine=merge_key_value_gradients,
                identity=I.record(grad_k=I.zeros((K, D), dtype=I.f32), grad_v=I.zeros((K, D), dtype=I.f32)),
                operands=(k[batch, key_head, keys, :], v[batch, key_head, keys, :], I.indices(keys), scale, CAUSAL),
            )
            grad_k[batch, key_head, keys, :] = I.cast(summary.grad_k * scale, I.f16)
            grad_v[batch, key_head, keys, :] = I.cast(summary.grad_v, I.f16)


@intent.fn
def summarize_query_gradients(keys, values, key_coordinates, queries, grad_outputs, lse, delta,
                              query_coordinates, scale, causal):
    scores = I.matmul(queries, keys, transpose_rhs=True, acc_dtype=I.f32)
    weights = I.exp2(scores * (scale * I.LOG2E) - lse[:, None] * I.LOG2E, approximate=True, flush_to_zero=True)
    if causal:
        valid = query_coordinates[:, None] >= key_coordinates[None, :]
        weights = I.mask(weights, valid=valid, fill=0.0)
    grad_weights = I.matmul(grad_outputs, values, transpose_rhs=True, acc_dtype=I.f32)
    grad_scores = weights * (grad_weights - delta[:, None])
    if causal:
        return masked_gradient_product(I.cast(grad_scores, I.f16), keys, valid)
    return I.matmul(I.cast(grad_scores, I.f16), keys, acc_dtype=I.f32)


@intent.fn
def merge_query_gradients(lhs, rhs):
    return lhs + rhs


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
    B, HQ, Q, D = q.shape
    K = k.shape[2]
    rows, keys = I.domain(0, Q), I.domain(0, K)
    for batch in I.parallel(I.domain(0, B)):
        for head in I.parallel(I.domain(0, HQ)):
            key_head = head // HEAD_GROUP
            value = I.region_fold(
                source=(k[batch, key_head, keys, :], v[batch, key_head, keys, :], I.indices(keys)),
                axis=0,
                summarize=summarize_query_gradients,
                combine=merge_query_gradients,
                identity=I.zeros((Q, D), dtype=I.f32),
                operands=(q[batch, head, rows, :], grad_output[batch, head, rows, :], lse[batch, head, rows],
                          delta[batch, head, rows], I.indices(rows), scale, CAUSAL),
            )
            grad_q[batch, head, rows, :] = I.cast(value * scale, I.f16)
