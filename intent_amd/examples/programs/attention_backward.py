"""The three-kernel backward pass of grouped-query attention (the reference's
`python/intent/examples/programs/attention_backward.py:1-41`): delta, then dK/dV, then dQ, bound
once and launched as a PreparedSequence."""
from dataclasses import dataclass

from intent_amd.examples.kernels.backward.attention import (attention_backward_delta, attention_backward_dkdv,
                                                            attention_backward_dq)
from intent_amd.runtime import PreparedSequence


@dataclass
class AttentionBackward:
    delta: object
    dkdv: object
    dq: object

    @classmethod
    def from_jit(cls, jit, *, head_group, causal):
        options = {"HEAD_GROUP": head_group, "CAUSAL": causal}
        return cls(jit(attention_backward_delta), jit(attention_backward_dkdv, constexprs=options),
                   jit(attention_backward_dq, constexprs=options))

    def prepare(self, query, key, value, output, grad_output, lse, scale, *, outputs=None, workspace=None):
        """Bind dQ, dK and dV in that order. LSE is the natural logarithm."""
        delta = self.delta.prepare(output, grad_output, outputs=None if workspace is None else (workspace,))
        common = (query, key, value, grad_output, lse, delta.result(), scale)
        dq_outputs = dkdv_outputs = None
        if outputs is not None:
            grad_q, grad_k, grad_v = outputs
            dq_outputs, dkdv_outputs = (grad_q,), (grad_k, grad_v)
        dkdv = self.dkdv.prepare(*common, outputs=dkdv_outputs)
        dq = self.dq.prepare(*common, outputs=dq_outputs)
        return PreparedSequence((delta, dkdv, dq), outputs=(dq.result(), *dkdv.result()))

    def run(self, *arguments, **bindings):
        call = self.prepare(*arguments, **bindings)
        call.launch()
        return call.result()
