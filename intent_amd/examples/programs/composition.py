"""Author-owned partial/merge programs (the reference's `python/intent/examples/programs/composition.py`).

PagedDecode (composition.py:95-122 there): split-K paged grouped-query decode, the partials kernel
(paged_gqa_decode_partials) followed by the split merge (splitk_attention_f32_to_f16_reduce). The
composition is the author's: `run` allocates the intermediates through the partials call, `into`
writes caller-owned buffers, `prepare` binds both calls once, the merge bound to the partials'
exact output views, and returns a PreparedSequence whose launch replays the pair on the caller's
stream.
"""
from dataclasses import dataclass
from typing import ClassVar

from intent_amd.examples.kernels.streaming.paged_attention import paged_gqa_decode_partials
from intent_amd.examples.kernels.streaming.splitk_reduce import splitk_attention_f32_to_f16_reduce
from intent_amd.runtime import PreparedSequence


@dataclass
class PagedDecode:
    mutable_inputs: ClassVar[tuple[int, ...]] = ()
    partials: object
    merge: object

    @classmethod
    def from_jit(cls, jit, *, page_size, head_group, splits):
        """Compile both kernels through `jit` (e.g. functools.partial(intent.jit, backend="hip"))."""
        options = {"PAGE_SIZE": page_size, "HEAD_GROUP": head_group, "SPLITS": splits}
        return cls(jit(paged_gqa_decode_partials, constexprs=options), jit(splitk_attention_f32_to_f16_reduce))

    def run(self, q, key_cache, value_cache, page_offsets, page_indices, lengths, split_offsets, scale):
        lse, output = self.partials.run(q, key_cache, value_cache, page_offsets, page_indices, lengths,
                                        split_offsets, scale)
        return self.merge.run(output, lse)

    def into(self, q, key_cache, value_cache, page_offsets, page_indices, lengths, split_offsets, partial_lse,
             partial_output, output, scale):
        self.partials(q, key_cache, value_cache, page_offsets, page_indices, lengths, split_offsets, partial_lse,
                      partial_output, scale)
        self.merge(partial_output, partial_lse, output)
        return output

    def prepare(self, q, key_cache, value_cache, page_offsets, page_indices, lengths, split_offsets, scale):
        partials = self.partials.prepare(q, key_cache, value_cache, page_offsets, page_indices, lengths,
                                         split_offsets, scale)
        partial_lse, partial_output = partials.result()
        merge = self.merge.prepare(partial_output, partial_lse)
        return PreparedSequence((partials, merge), outputs=merge.result())
