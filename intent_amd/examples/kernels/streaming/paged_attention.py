"""Paged grouped-query decode attention, split over page ranges (interface and semantics of the
reference's `python/intent/examples/kernels/streaming/paged_attention.py:77-165`).

For each (batch, split) job and key head, the HEAD_GROUP query heads of that key head attend over
the tokens of the job's pages: page position p in [split_offsets[job], split_offsets[job+1]),
physical page page_indices[p], token offset o in [0, PS); logical token
(p - page_offsets[batch]) * PAGE_SIZE + o, active while below sequence_lengths[batch]. The fold
is the f16 attention summary in the exp2 domain (masked chunk summaries merged by rescaling);
outputs: partial_lse = maximum + log(denominator) * log2(e) (-inf for an empty job) and
partial_output = accumulator * (1 / denominator) (0 for an empty job), in f32.
"""
import math

import intent_amd as intent
import intent_amd.language as I

from intent_amd.examples.kernels.streaming.attention import (empty_attention_summary, merge_attention_summaries,
                                                             summarize_masked_attention_chunk)

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
    B, HQ, D = q.shape
    PS, HK = key_cache.shape[1], key_cache.shape[2]
    DV = value_cache.shape[3]
    for job in I.parallel(I.domain(0, B * SPLITS)):
        batch, split = job // SPLITS, job % SPLITS
        page_begin = I.cast(page_offsets[batch], I.index)
        length = I.cast(sequence_lengths[batch], I.index)
        first = I.cast(split_offsets[job], I.index)
        pages = I.cast(split_offsets[job + 1] - split_offsets[job], I.index)
        token = I.indices(I.domain(0, pages * PS))
        position = first + token // PS
        offset = token % PS
        physical = I.cast(page_indices[position], I.index)
        logical = (position - page_begin) * PAGE_SIZE + offset
        for key_head in I.parallel(I.domain(0, HK)):
            heads = key_head * HEAD_GROUP + I.indices(I.domain(0, HEAD_GROUP))
            summary = I.region_fold(
                source=(key_cache[physical, offset, key_head, :], value_cache[physical, offset, key_head, :],
                        logical, logical < length),
                axis=0,
                summarize=summarize_masked_attention_chunk,
                combine=merge_attention_summaries,
                identity=empty_attention_summary(HEAD_GROUP, DV),
                operands=(I.gather(q, index=(batch, heads, slice(None))),
                          I.full((HEAD_GROUP,), fill=0, dtype=I.index), scale),
            )
            denominator = I.select(summary.valid, summary.denominator, 1.0)
            I.scatter_unique(partial_lse, index=(batch, heads, split),
                             value=I.select(summary.valid, summary.maximum + I.log(denominator) * I.LOG2E, -I.inf))
            I.scatter_unique(partial_output, index=(batch, heads, split, slice(None)),
                             value=I.select(summary.valid[:, None],
                                            summary.accumulator * (1.0 / denominator)[:, None], 0.0))
