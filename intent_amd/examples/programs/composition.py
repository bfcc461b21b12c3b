"""Split-K paged decode as one program of two kernels: `PagedDecode`.

Public names and call shapes are the reference's `PagedDecode`
(`python/intent/examples/programs/composition.py:95-122`): `run`, `into`, `prepare` and the
`mutable_inputs` class attribute. `from_jit` is added here so that callers need not name the
constexprs themselves.

The first kernel, `paged_gqa_decode_partials`, writes per split the base-2 log-sum-exp and the
normalised partial rows of every query head. The second, `splitk_attention_f32_to_f16_reduce`,
merges the splits into the f16 output. All three entry points go through one binding step. `run`
lets both kernels allocate. `into` writes the caller's three buffers. `prepare` returns the bound
pair as a PreparedSequence, with the merge bound to the exact partial buffers of the first call,
so each launch replays both kernels on the caller's current stream.
"""
from dataclasses import dataclass
from typing import ClassVar

from intent_amd.examples.kernels.streaming.paged_attention import paged_gqa_decode_partials
from intent_amd.examples.kernels.streaming.splitk_reduce import splitk_attention_f32_to_f16_reduce
from intent_amd.runtime import PreparedSequence


@dataclass(frozen=True)
class PagedDecode:
    mutable_inputs: ClassVar[tuple[int, ...]] = ()     # no input is written
    partials: object                                  # JIT kernel of paged_gqa_decode_partials
    merge: object                                     # JIT kernel of splitk_attention_f32_to_f16_reduce

    @classmethod
    def from_jit(cls, jit, *, page_size, head_group, splits):
        """Jit both kernels through `jit` (for example functools.partial(intent.jit, backend="hip"))."""
        return cls(partials=jit(paged_gqa_decode_partials,
                                constexprs=dict(PAGE_SIZE=page_size, HEAD_GROUP=head_group, SPLITS=splits)),
                   merge=jit(splitk_attention_f32_to_f16_reduce))

    def _bind(self, tables: tuple, scale, buffers=None) -> PreparedSequence:
        split_call = self.partials.prepare(*tables, scale, outputs=None if buffers is None else tuple(buffers[:2]))
        partial_lse, partial_rows = split_call.result()
        merge_call = self.merge.prepare(partial_rows, partial_lse, outputs=None if buffers is None else (buffers[2],))
        return PreparedSequence((split_call, merge_call), outputs=merge_call.result())

    def prepare(self, q, key_cache, value_cache, page_offsets, page_indices, lengths, split_offsets, scale):
        return self._bind((q, key_cache, value_cache, page_offsets, page_indices, lengths, split_offsets), scale)

    def run(self, q, key_cache, value_cache, page_offsets, page_indices, lengths, split_offsets, scale):
        bound = self.prepare(q, key_cache, value_cache, page_offsets, page_indices, lengths, split_offsets, scale)
        bound.launch()
        return bound.result()

    def into(self, q, key_cache, value_cache, page_offsets, page_indices, lengths, split_offsets, partial_lse,
             partial_output, output, scale):
        self._bind((q, key_cache, value_cache, page_offsets, page_indices, lengths, split_offsets), scale,
                   (partial_lse, partial_output, output)).launch()
        return output
