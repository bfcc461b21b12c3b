"""Grouped-query attention backward as one prepared program of three kernels.

Public names and call shapes are those of the reference program
(`python/intent/examples/programs/attention_backward.py`): `AttentionBackward.from_jit(jit, *,
head_group, causal)`, `prepare(query, key, value, output, grad_output, lse, scale, *, outputs=None,
workspace=None)` and `run`.

A prepared backward binds, in launch order:

1. `attention_backward_delta`: delta[b, h, q] = sum_d output * grad_output, in f32. It writes
   into `workspace` when one is given, otherwise into a buffer allocated at prepare;
2. `attention_backward_dkdv`: dK and dV of every key head;
3. `attention_backward_dq`: dQ of every query head.

The two gradient kernels read delta and nothing the other writes. The result is (dQ, dK, dV);
`outputs`, when given, supplies those three buffers in that order. `lse` is the natural
logarithm of the forward's softmax denominator.
"""
from __future__ import annotations

from dataclasses import dataclass

from intent_amd.examples.kernels.backward.attention import (attention_backward_delta, attention_backward_dkdv,
                                                            attention_backward_dq)
from intent_amd.runtime import PreparedSequence


@dataclass(frozen=True)
class AttentionBackward:
    delta: object       # JIT kernel of attention_backward_delta
    dkdv: object        # JIT kernel of attention_backward_dkdv
    dq: object          # JIT kernel of attention_backward_dq

    @classmethod
    def from_jit(cls, jit, *, head_group, causal):
        """Jit the three kernels; the two gradient kernels share the HEAD_GROUP/CAUSAL specialization."""
        specialization = dict(HEAD_GROUP=head_group, CAUSAL=causal)
        return cls(delta=jit(attention_backward_delta),
                   dkdv=jit(attention_backward_dkdv, constexprs=specialization),
                   dq=jit(attention_backward_dq, constexprs=specialization))

    def prepare(self, query, key, value, output, grad_output, lse, scale, *, outputs=None, workspace=None):
        if outputs is not None and len(outputs) != 3:
            raise TypeError("outputs holds (grad_query, grad_key, grad_value)")
        row_dots = self.delta.prepare(output, grad_output, outputs=None if workspace is None else (workspace,))
        operands = (query, key, value, grad_output, lse, row_dots.result(), scale)
        key_grads = self.dkdv.prepare(*operands, outputs=None if outputs is None else tuple(outputs[1:]))
        query_grad = self.dq.prepare(*operands, outputs=None if outputs is None else (outputs[0],))
        grad_key, grad_value = key_grads.result()
        return PreparedSequence((row_dots, key_grads, query_grad),
                                outputs=(query_grad.result(), grad_key, grad_value))

    def run(self, *arguments, **bindings):
        """Prepare, launch and return (dQ, dK, dV)."""
        prepared = self.prepare(*arguments, **bindings)
        prepared.launch()
        return prepared.result()
