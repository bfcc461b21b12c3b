"""GPU parity of the attention backward (delta, dK/dV, dQ) through the AttentionBackward program
(the reference's programs/attention_backward.py) and intent.jit, and of the authored-backward
autograd registration flow (the reference's examples/softmax_forward_backward.py:11-28).

Bar: f16 gradients within rel 2e-2 of the oracle plus an absolute 1e-2 of the tensor's largest
magnitude (the f16 roundings of P and dS and the reassociated sums); delta (f32) within rel 1e-5
of the oracle. Inputs are finite; causally excluded pairs then contribute exactly zero in both."""
import numpy as np
import pytest
import torch

import intent_amd as intent
import oracle
from intent_amd.examples import inputs
from intent_amd.examples.programs.attention_backward import AttentionBackward
from tests.gpu_util import announce, assert_f32_rel

pytestmark = pytest.mark.gpu


def close(got, want, rel=2e-2, frac=1e-2):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert not np.isnan(got).any()
    bound = rel * np.abs(want) + frac * max(np.abs(want).max(), 1e-3)
    worst = np.unravel_index(np.argmax(np.abs(got - want) - bound), got.shape)
    assert np.all(np.abs(got - want) <= bound), f"at {worst}: got {got[worst]} want {want[worst]}"


def case(seed, batch, hq, hk, sq, sk, d):
    rng = np.random.default_rng(seed)
    q = inputs.normal(rng, (batch, hq, sq, d), "f16")
    k = inputs.normal(rng, (batch, hk, sk, d), "f16")
    v = inputs.normal(rng, (batch, hk, sk, d), "f16")
    o = inputs.normal(rng, (batch, hq, sq, d), "f16")
    do = inputs.normal(rng, (batch, hq, sq, d), "f16")
    lse = (rng.standard_normal((batch, hq, sq)) * 0.5 + np.log(max(sk, 1))).astype(np.float32)
    return q, k, v, o, do, lse


@pytest.mark.parametrize("shape,causal", [((2, 8, 2, 1024, 1024, 64), True), ((1, 4, 4, 300, 300, 64), True),
                                          ((1, 2, 1, 200, 333, 64), False), ((1, 4, 2, 257, 257, 128), True),
                                          ((2, 2, 2, 130, 70, 128), False), ((1, 1, 1, 1, 1, 64), True)])
def test_attention_backward_matches_oracle(device, shape, causal):
    batch, hq, hk, sq, sk, d = shape
    announce("attention backward", shape, causal)
    q, k, v, o, do, lse = case(sq + sk + d, batch, hq, hk, sq, sk, d)
    scale = float(np.float32(1 / np.sqrt(d)))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    program = AttentionBackward.from_jit(lambda defn, **kw: intent.jit(defn, backend="hip", **kw),
                                         head_group=hq // hk, causal=causal)
    grad_q, grad_k, grad_v = program.run(t(q), t(k), t(v), t(o), t(do), t(lse), scale)
    delta = oracle.attention_bwd_delta(o, do)
    want_dq = oracle.attention_bwd_dq(q, k, v, do, lse, delta, scale, causal, head_group=hq // hk)
    want_dk, want_dv = oracle.attention_bwd_dkdv(q, k, v, do, lse, delta, scale, causal, head_group=hq // hk)
    close(grad_q.cpu().numpy(), want_dq)
    close(grad_k.cpu().numpy(), want_dk)
    close(grad_v.cpu().numpy(), want_dv)


def test_attention_backward_delta_and_explicit_outputs(device):
    announce("attention backward delta / outputs")
    from intent_amd.examples.kernels.backward.attention import attention_backward_delta

    q, k, v, o, do, lse = case(3, 2, 4, 2, 96, 96, 64)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    delta = intent.jit(attention_backward_delta, backend="hip").run(t(o), t(do)).cpu().numpy()
    assert_f32_rel(delta, oracle.attention_bwd_delta(o, do), rel=1e-5, floor=1e-4)
    program = AttentionBackward.from_jit(lambda defn, **kw: intent.jit(defn, backend="hip", **kw), head_group=2,
                                         causal=True)
    outputs = (torch.empty(2, 4, 96, 64, dtype=torch.float16, device=device),
               torch.empty(2, 2, 96, 64, dtype=torch.float16, device=device),
               torch.empty(2, 2, 96, 64, dtype=torch.float16, device=device))
    call = program.prepare(t(q), t(k), t(v), t(o), t(do), t(lse), 0.125, outputs=outputs)
    assert call.kernel_count == 3
    call.launch()
    assert call.result()[0] is outputs[0]
    reference = program.run(t(q), t(k), t(v), t(o), t(do), t(lse), 0.125)
    for got, want in zip(outputs, reference):
        assert torch.equal(got, want)


def test_authored_softmax_backward_autograd(device):
    """examples/softmax_forward_backward.py: forward and authored backward as torch ops, the
    backward registered with register_autograd."""
    announce("softmax autograd registration")
    from intent_amd.examples.kernels.backward.softmax import softmax_backward
    from intent_amd.examples.kernels.normalization.softmax import stable_softmax

    x = torch.randn((4096, 4097), dtype=torch.float32, device=device, requires_grad=True)
    upstream = torch.randn_like(x)
    forward = intent.jit(stable_softmax, backend="hip")
    backward = intent.jit(softmax_backward, backend="hip")
    probabilities = forward.prepare(x.detach()).result()
    backward.prepare(probabilities, upstream)
    operation = forward.as_torch_op("intent_amd_tests::softmax_forward")
    backward_operation = backward.as_torch_op("intent_amd_tests::softmax_backward")

    def setup_context(ctx, inputs, output):  # noqa: F811 (torch passes these by keyword)
        ctx.save_for_backward(output)

    def backward_formula(ctx, grad):
        p, = ctx.saved_tensors
        return backward_operation(p, grad)

    operation.register_autograd(backward_formula, setup_context=setup_context)
    y = operation(x)
    y.backward(upstream)
    reference = x.detach().clone().requires_grad_(True)
    torch.softmax(reference, dim=1).backward(upstream)
    assert torch.allclose(y, torch.softmax(x.detach(), dim=1), rtol=1e-5, atol=1e-7)
    assert torch.allclose(x.grad, reference.grad, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("shape", [(2, 8, 2, 1024, 1024, 64), (1, 6, 3, 300, 200, 128), (1, 4, 4, 300, 300, 64)])
def test_dkdv_split_matches_unsplit_through_the_c_abi(device, shape):
    """intent_hip_attention_bwd_dkdv_ws with a workspace (query heads and ranges of their query
    tiles split over workgroups, f32 partials folded by a second kernel) against the same entry
    with no workspace (one workgroup walks every head of the group): the sums differ only in
    association, so within 2 f16 ulp plus 1e-3 of the largest magnitude; both against the
    oracle. The third shape has one query head per key head, split by query range alone."""
    import ctypes

    from intent_amd.runtime.hip.library import library

    batch, hq, hk, sq, sk, d = shape
    announce("dK/dV split vs unsplit", shape)
    q, k, v, o, do, lse = case(sum(shape), batch, hq, hk, sq, sk, d)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    tq, tk, tv, tdo, tlse = t(q), t(k), t(v), t(do), t(lse)
    delta_np = oracle.attention_bwd_delta(o, do)
    tdelta = t(delta_np)
    lib = library()
    size = ctypes.c_size_t(0)
    assert lib.fn["attention_bwd_dkdv_workspace_bytes"](batch, hq, hq // hk, sq, sk, d, ctypes.byref(size)) == 0
    per_range = 2 * hq * batch * sk * d * 4                     # dK and dV partials of one range per head
    assert size.value > 0 and size.value % per_range == 0 and size.value // per_range <= 8
    workspace = torch.empty(size.value, dtype=torch.uint8, device=device)
    results = []
    for ws in (workspace, None):
        dk = torch.empty_like(tk)
        dv = torch.empty_like(tv)
        st = [x for a in (tq, tk, tv, tdo) for x in a.stride()] + list(tlse.stride()) + list(tdelta.stride()) + \
            list(dk.stride()) + list(dv.stride())
        strides = (ctypes.c_int64 * 30)(*st)
        rc = lib.fn["attention_bwd_dkdv_ws"](tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), tdo.data_ptr(),
                                             tlse.data_ptr(), tdelta.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                             batch, hq, hq // hk, sq, sk, d, strides, float(np.float32(d ** -0.5)),
                                             1, ws.data_ptr() if ws is not None else None,
                                             size.value if ws is not None else 0,
                                             torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        results.append((dk.cpu().numpy().astype(np.float64), dv.cpu().numpy().astype(np.float64)))
    torch.cuda.synchronize()
    want_dk, want_dv = oracle.attention_bwd_dkdv(q, k, v, do, lse, delta_np, float(np.float32(d ** -0.5)), True,
                                                 head_group=hq // hk)
    for i, want in enumerate((want_dk, want_dv)):
        split, unsplit = results[0][i], results[1][i]
        bound = 2 * 2.0 ** -10 * np.abs(unsplit) + 1e-3 * np.abs(unsplit).max()
        assert np.all(np.abs(split - unsplit) <= bound)
        close(split, want)
    small = ctypes.c_size_t(0)
    assert lib.fn["attention_bwd_dkdv_workspace_bytes"](4, 32, 4, 4096, 4096, 128, ctypes.byref(small)) == 0
    assert small.value == 0                                     # large grids never split


# Calls with at least 256 x 256 rows (batch x heads x sequence) take the 8-wave kernels: dQ with
# 256-query workgroups, dK/dV as two kernels (dK, then dV) with 256-key workgroups. These shapes
# reach that bound with short sequences so the oracle stays fast; 260 and 300 leave ragged blocks.
@pytest.mark.parametrize("shape,causal", [((64, 4, 4, 256, 256, 128), True), ((64, 8, 4, 260, 260, 64), True),
                                          ((70, 4, 4, 240, 300, 64), False)])
def test_attention_backward_wide_grids_match_oracle(device, shape, causal):
    batch, hq, hk, sq, sk, d = shape
    assert batch * hk * sk >= 256 * 256 and batch * hq * sq >= 256 * 256
    announce("attention backward, wide grid", shape, causal)
    q, k, v, o, do, lse = case(sq + sk + d + batch, batch, hq, hk, sq, sk, d)
    scale = float(np.float32(1 / np.sqrt(d)))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    program = AttentionBackward.from_jit(lambda defn, **kw: intent.jit(defn, backend="hip", **kw),
                                         head_group=hq // hk, causal=causal)
    grad_q, grad_k, grad_v = program.run(t(q), t(k), t(v), t(o), t(do), t(lse), scale)
    delta = oracle.attention_bwd_delta(o, do)
    want_dq = oracle.attention_bwd_dq(q, k, v, do, lse, delta, scale, causal, head_group=hq // hk)
    want_dk, want_dv = oracle.attention_bwd_dkdv(q, k, v, do, lse, delta, scale, causal, head_group=hq // hk)
    close(grad_q.cpu().numpy(), want_dq)
    close(grad_k.cpu().numpy(), want_dk)
    close(grad_v.cpu().numpy(), want_dv)


@pytest.mark.parametrize("shape", [(17, 8, 4, 1000, 1000, 64), (17, 4, 4, 1000, 1000, 128)])
def test_wide_grid_equals_per_batch_calls_through_the_c_abi(device, shape):
    """Batch elements are independent, and every kernel variant gives each output element the same
    arithmetic in the same order: the whole batch (8-wave kernels) must equal, bit for bit, one
    call per batch element (4-wave kernels, dK and dV together; no workspace, so no head split)."""
    import ctypes

    from intent_amd.runtime.hip.library import library

    batch, hq, hk, sq, sk, d = shape
    assert batch * hk * sk >= 256 * 256 and hq * sq < 256 * 256
    announce("attention backward wide vs per-batch", shape)
    q, k, v, o, do, lse = case(sum(shape), batch, hq, hk, sq, sk, d)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    tq, tk, tv, tdo, tlse = t(q), t(k), t(v), t(do), t(lse)
    tdelta = t(oracle.attention_bwd_delta(o, do))
    lib = library()
    scale = float(np.float32(d ** -0.5))
    stream = torch.cuda.current_stream().cuda_stream

    def run(sl):
        a = [x[sl] for x in (tq, tk, tv, tdo, tlse, tdelta)]
        dq, dk, dv = torch.empty_like(a[0]), torch.empty_like(a[1]), torch.empty_like(a[2])
        base = [s for x in a[:4] for s in x.stride()] + list(a[4].stride()) + list(a[5].stride())
        st_q = (ctypes.c_int64 * 26)(*base, *dq.stride())
        st_k = (ctypes.c_int64 * 30)(*base, *dk.stride(), *dv.stride())
        n = a[0].shape[0]
        ptrs = [x.data_ptr() for x in a]
        assert lib.fn["attention_bwd_dq"](*ptrs, dq.data_ptr(), n, hq, hq // hk, sq, sk, d, st_q, scale, 1,
                                          stream) == 0
        assert lib.fn["attention_bwd_dkdv"](*ptrs, dk.data_ptr(), dv.data_ptr(), n, hq, hq // hk, sq, sk, d, st_k,
                                            scale, 1, stream) == 0
        return dq, dk, dv

    whole = run(slice(None))
    parts = [run(slice(i, i + 1)) for i in range(batch)]
    torch.cuda.synchronize()
    for j, name in enumerate(("dq", "dk", "dv")):
        joined = torch.cat([p[j] for p in parts])
        assert torch.equal(whole[j], joined), name
    delta_np = tdelta.cpu().numpy()
    want_dk, want_dv = oracle.attention_bwd_dkdv(q[:1], k[:1], v[:1], do[:1], lse[:1], delta_np[:1], scale, True,
                                                 head_group=hq // hk)
    close(whole[1][:1].cpu().numpy(), want_dk)
    close(whole[2][:1].cpu().numpy(), want_dv)


@pytest.mark.parametrize("shape,causal", [((2, 8, 2, 1024, 1024, 64), True), ((1, 3, 1, 200, 700, 128), False),
                                          ((1, 2, 2, 130, 130, 64), True)])
def test_dq_split_matches_unsplit_through_the_c_abi(device, shape, causal):
    """intent_hip_attention_bwd_dq_ws with a workspace (each query block's key tiles divided over
    up to 8 workgroups, f32 partials folded in range order) against the same entry with no
    workspace: within 2 f16 ulp plus 1e-3 of the largest magnitude; both against the oracle."""
    import ctypes

    from intent_amd.runtime.hip.library import library

    batch, hq, hk, sq, sk, d = shape
    announce("dQ split vs unsplit", shape, causal)
    q, k, v, o, do, lse = case(sum(shape), batch, hq, hk, sq, sk, d)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    tq, tk, tv, tdo, tlse = t(q), t(k), t(v), t(do), t(lse)
    delta_np = oracle.attention_bwd_delta(o, do)
    tdelta = t(delta_np)
    lib = library()
    size = ctypes.c_size_t(0)
    assert lib.fn["attention_bwd_dq_workspace_bytes"](batch, hq, hq // hk, sq, sk, d, ctypes.byref(size)) == 0
    per_range = batch * hq * sq * d * 4
    assert size.value > 0 and size.value % per_range == 0 and 2 <= size.value // per_range <= 8
    workspace = torch.empty(size.value, dtype=torch.uint8, device=device)
    scale = float(np.float32(d ** -0.5))
    results = []
    for ws in (workspace, None):
        dq = torch.empty_like(tq)
        st = [x for a in (tq, tk, tv, tdo) for x in a.stride()] + list(tlse.stride()) + list(tdelta.stride()) + \
            list(dq.stride())
        strides = (ctypes.c_int64 * 26)(*st)
        rc = lib.fn["attention_bwd_dq_ws"](tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), tdo.data_ptr(), tlse.data_ptr(),
                                           tdelta.data_ptr(), dq.data_ptr(), batch, hq, hq // hk, sq, sk, d, strides,
                                           scale, int(causal), ws.data_ptr() if ws is not None else None,
                                           size.value if ws is not None else 0, torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        results.append(dq.cpu().numpy().astype(np.float64))
    torch.cuda.synchronize()
    split, unsplit = results
    assert np.all(np.abs(split - unsplit) <= 2 * 2.0 ** -10 * np.abs(unsplit) + 1e-3 * np.abs(unsplit).max())
    close(split, oracle.attention_bwd_dq(q, k, v, do, lse, delta_np, scale, causal, head_group=hq // hk))
    large = ctypes.c_size_t(0)
    assert lib.fn["attention_bwd_dq_workspace_bytes"](4, 32, 4, 4096, 4096, 128, ctypes.byref(large)) == 0
    assert large.value == 0                                     # large grids never split
