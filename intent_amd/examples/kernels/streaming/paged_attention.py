"""Paged grouped-query decode attention, split over page ranges. Names, signature and example
extents are the reference's (`python/intent/examples/kernels/streaming/paged_attention.py:77-165`).

A job is one (batch, split) pair. Its pages are the page-table positions p in
[split_offsets[job], split_offsets[job + 1]); position p holds physical page page_indices[p], and
token t of it is logical token (p - page_offsets[batch]) * PAGE_SIZE + t. A token takes part while
its logical index is below sequence_lengths[batch]. For each key head, the HEAD_GROUP query heads
that share it attend over the job's tokens as the forward attention does (base-2 logits, NaN-ignoring
peak, approximate exp2 weights rounded to f16 before they weight V). The job writes, per query head,
the base-2 log-sum-exp of its weights to partial_lse and its rows divided (exactly) by the sum of
the weights to partial_output, in f32. A job with no live token writes -inf and 0. The split-K
merge (splitk_reduce.py) combines the splits of a batch.

The body states this for one job at a time; the hip provider recognises the definition by name and
signature and runs its own kernel.
"""
import math

import intent_amd as intent
import intent_amd.language as I

from intent_amd.examples.kernels.streaming.attention import admitted_attention

BATCH = 8
QUERY_HEADS = 32
KV_HEADS = 8
HEAD_GROUP = QUERY_HEADS // KV_HEADS
PAGE_SIZE = 64
HEAD_DIMENSION = 128
SEQUENCE_LENGTHS = (8191, 7937, 7683, 7429, 7175, 6921, 6667, 6413)
SCALE = 1.0 / math.sqrt(HEAD_DIMENSION)
SPLITS = 16


@intent.kernel
def paged_gqa_decode_partials(
    q: I.In[I.f16, ("B", "HQ", "D")],
    key_cache: I.In[I.f16, ("P", "PS", "HK", "D")],
    value_cache: I.In[I.f16, ("P", "PS", "HK", "DV")],
    page_offsets: I.In[I.i32, ("B_PLUS_1",)],
    page_indices: I.In[I.i32, ("S",)],
    sequence_lengths: I.In[I.i32, ("B",)],
    split_offsets: I.In[I.i32, ("SP_PLUS_1",)],
    partial_lse: I.Out[I.f32, ("B", "HQ", "SPLITS")],
    partial_output: I.Out[I.f32, ("B", "HQ", "SPLITS", "DV")],
    scale: I.f32,
    PAGE_SIZE: I.Constexpr[int],
    HEAD_GROUP: I.Constexpr[int],
    SPLITS: I.Constexpr[int],
):
    B, HK, PS = q.shape[0], key_cache.shape[2], key_cache.shape[1]
    for job in I.parallel(I.domain(0, B * SPLITS)):
        batch, split = job // SPLITS, job % SPLITS
        first, last = I.cast(split_offsets[job], I.index), I.cast(split_offsets[job + 1], I.index)
        token = I.indices(I.domain(0, (last - first) * PS))
        position, slot = first + token // PS, token % PS
        page = I.cast(page_indices[position], I.index)
        live = (position - I.cast(page_offsets[batch], I.index)) * PAGE_SIZE + slot < I.cast(sequence_lengths[batch],
                                                                                              I.index)
        for kv in I.parallel(I.domain(0, HK)):
            heads = kv * HEAD_GROUP + I.indices(I.domain(0, HEAD_GROUP))
            queries = I.gather(q, index=(batch, heads, slice(None)))
            logits = I.matmul(queries, key_cache[page, slot, kv, :], transpose_rhs=True, acc_dtype=I.f32)
            result = admitted_attention(logits * (scale * I.LOG2E), live[None, :] & I.full(
                (HEAD_GROUP, token.shape[0]), fill=True, dtype=I.bool), value_cache[page, slot, kv, :], I.f16)
            I.scatter_unique(partial_lse, index=(batch, heads, split),
                             value=I.select(result.live, result.peak + I.log(result.total) * I.LOG2E, -I.inf))
            I.scatter_unique(partial_output, index=(batch, heads, split, slice(None)),
                             value=I.select(result.live[:, None], result.mixed * (1.0 / result.total)[:, None], 0.0))
