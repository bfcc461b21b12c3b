"""Prepared calls whose kernels share a workspace or rewrite a caller buffer, captured in a HIP
graph: SpMV (row lists and cuts in the plan workspace), packed-sequence attention (work items in
the workspace), the key-biased attention, the continuous decode (split states, then the merge)
and the packed decode (block maxima written into block_logits, then rewritten as logits).

Each graph is replayed three times, with the outputs cleared and eager work on the same inputs in
between; every replay must equal the eager result bit for bit. No kernel in these calls clears
memory with hipMemsetAsync: every workspace entry a kernel reads was written earlier in the same
call."""
import numpy as np
import pytest
import torch

import intent_amd as intent
from intent_amd.examples import inputs
from intent_amd.examples.kernels.sparse.csr_spmv import csr_spmv
from intent_amd.examples.kernels.streaming.attention import (continuous_gqa_decode, flash_attention_bias_fwd,
                                                            flash_varlen_gqa_prefill,
                                                            varlen_gqa_decode_with_sink_logits)
from tests.gpu_util import announce

pytestmark = pytest.mark.gpu


def t(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def replay_matches_eager(call, outputs, other):
    """`call` is a prepared call; `outputs` the tensors it writes; `other` an eager closure run
    between replays."""
    call.launch()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outputs]
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            call.launch()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for _ in range(3):
        for o in outputs:
            o.zero_()
        other()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(outputs, eager):
            assert torch.equal(got, want)


def test_graph_replay_spmv(device):
    announce("graph replay: spmv")
    rng = np.random.default_rng(7)
    lengths = np.concatenate([rng.integers(0, 5, 4000), rng.integers(5, 128, 500), rng.integers(128, 3000, 40),
                              [40000, 70000]])
    rng.shuffle(lengths)
    offsets, columns = inputs.csr_matrix(rng, lengths.astype(np.int64), 200000)
    values = inputs.uniform(rng, offsets[-1], -1.0, 1.0)
    x = inputs.uniform(rng, 200000, -1.0, 1.0)
    args = [t(a, device) for a in (offsets, columns, values, x)]
    call = intent.jit(csr_spmv, backend="hip").prepare(*args)
    other = intent.jit(csr_spmv, backend="hip")
    replay_matches_eager(call, [call.result()], lambda: other.run(*args))


def test_graph_replay_varlen_prefill_and_bias(device):
    announce("graph replay: varlen prefill, bias attention")
    g = np.random.default_rng(8)
    lengths = np.array([300, 1, 0, 700], np.int32)
    cu = np.concatenate(([0], np.cumsum(lengths))).astype(np.int32)
    q = inputs.normal(g, (int(cu[-1]), 8, 128), "f16")
    k, v = inputs.normal(g, (int(cu[-1]), 2, 128), "f16"), inputs.normal(g, (int(cu[-1]), 2, 128), "f16")
    args = [t(a, device) for a in (q, k, v, lengths, cu)]
    prefill = intent.jit(flash_varlen_gqa_prefill, backend="hip", constexprs={"HEAD_GROUP": 4})
    call = prefill.prepare(*args, 0.088)
    replay_matches_eager(call, [call.result()], lambda: prefill.run(*args, 0.088))
    qb, kb, vb = (t(inputs.normal(g, (2, 4, 300, 64), "f16"), device) for _ in range(3))
    bias = t((2.0 * g.standard_normal((2, 4, 300))).astype(np.float32), device)
    biased = intent.jit(flash_attention_bias_fwd, backend="hip")
    call = biased.prepare(qb, kb, vb, bias, 0.125)
    replay_matches_eager(call, [call.result()], lambda: biased.run(qb, kb, vb, bias, 0.125))


def test_graph_replay_decodes(device):
    announce("graph replay: continuous and packed decode")
    g = np.random.default_rng(9)
    q = t(inputs.normal(g, (3, 16, 128), "f16"), device)
    k, v = (t(inputs.normal(g, (3, 2000, 4, 128), "f16"), device) for _ in range(2))
    mask = t((g.random((3, 2000, 4)) < 0.5).astype(np.uint8), device)
    cont = intent.jit(continuous_gqa_decode, backend="hip", constexprs={"HEAD_GROUP": 4})
    call = cont.prepare(q, k, v, mask, 0.088)
    replay_matches_eager(call, [call.result()], lambda: cont.run(q, k, v, mask, 0.088))
    lengths = np.array([0, 65, 1000, 5000])
    cu = t(np.concatenate(([0], np.cumsum(lengths))).astype(np.int32), device)
    qd = t(inputs.normal(g, (4, 32, 64), "f16"), device)
    kd, vd = (t(inputs.normal(g, (int(lengths.sum()), 8, 64), "f16"), device) for _ in range(2))
    sink = t(g.uniform(0.0, 2.0, 32).astype(np.float32), device)
    packed = intent.jit(varlen_gqa_decode_with_sink_logits, backend="hip",
                        constexprs={"HEAD_GROUP": 4, "MAX_BLOCKS": 64})
    call = packed.prepare(qd, kd, vd, cu, sink, 0.125)
    out, logits = call.result()
    replay_matches_eager(call, [out, logits], lambda: packed.run(qd, kd, vd, cu, sink, 0.125))
