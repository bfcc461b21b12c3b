"""GPU parity of the attention backward (delta, dK/dV, dQ) through the AttentionBackward program
(the reference's programs/attention_backward.py) and intent.jit, and of the authored-backward
autograd registration flow (the reference's examples/softmax_forward_backward.py:11-28).

Bar: the stated 16-bit tolerance, |got - want| <= 2e-2 |want| + 1e-2, with the absolute term
tightened to 1e-2 of the tensor's largest magnitude where that is smaller (the gradients of long
sequences are far below 1, where a flat 1e-2 would accept almost anything). delta (f32) within rel
1e-5 of the oracle. Non-finite entries must match exactly: NaN positions, and infinities with their
sign. Causally excluded pairs contribute nothing even when their operands are non-finite, as in the
reference's masked_gradient_product (backward/attention.py:37-44)."""
import numpy as np
import pytest
import torch

import intent_amd as intent
import oracle
from intent_amd.examples import inputs
from intent_amd.examples.programs.attention_backward import AttentionBackward
from tests.gpu_util import announce, assert_f32_rel

pytestmark = pytest.mark.gpu


def close(got, want, rel=2e-2, abs_=1e-2, frac=1e-2):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    nan_got, nan_want = np.isnan(got), np.isnan(want)
    assert (nan_got == nan_want).all(), f"NaN positions differ: {np.argwhere(nan_got != nan_want)[:4].tolist()}"
    inf_want = np.isinf(want)
    assert (np.isinf(got) == inf_want).all() and (got[inf_want] == want[inf_want]).all(), "infinities differ"
    finite = np.isfinite(want)
    got, want = got[finite], want[finite]
    if want.size == 0:
        return
    bound = rel * np.abs(want) + min(abs_, frac * max(np.abs(want).max(), 1e-3))
    worst = np.argmax(np.abs(got - want) - bound)
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


def plant_nonfinite(q, k, v, do, seed):
    """Write NaN and +-inf into a few rows of Q, K, V and dO, inside the tiles that cross the causal
    diagonal: each row is excluded for some (query, key) pairs and valid for others."""
    rng = np.random.default_rng(seed)
    sq, sk, d = q.shape[2], k.shape[2], q.shape[3]
    marks = [(k, (0, 0), 70 % sk, np.nan), (v, (0, k.shape[1] - 1), 100 % sk, np.inf),
             (q, (0, q.shape[1] - 1), 40 % sq, -np.inf), (do, (q.shape[0] - 1, 0), 130 % sq, np.nan),
             (q, (q.shape[0] - 1, 0), 201 % sq, np.nan), (k, (k.shape[0] - 1, k.shape[1] - 1), (sk - 1), np.inf)]
    for array, (b, h), row, value in marks:
        array[b, h, row, rng.integers(0, d)] = value


@pytest.mark.parametrize("shape,causal", [((1, 4, 2, 300, 300, 64), True),       # dQ and dK/dV split
                                          ((4, 8, 8, 1000, 1000, 64), True),     # 4-wave, unsplit
                                          ((2, 4, 4, 600, 600, 128), True),      # 4-wave / split, D = 128
                                          ((64, 4, 4, 256, 256, 128), True),     # 8-wave dQ, dK, dV
                                          ((64, 8, 4, 260, 260, 64), True),      # 8-wave, D = 64, ragged
                                          ((70, 4, 4, 240, 300, 64), False)])    # rows past the end only
def test_excluded_pairs_with_nonfinite_operands_match_oracle(device, shape, causal):
    """NaN and infinities in rows of Q, K, V and dO that are causally excluded for some pairs (or
    past the end): the excluded pairs must not carry them into dQ, dK or dV."""
    batch, hq, hk, sq, sk, d = shape
    announce("attention backward, non-finite excluded rows", shape, causal)
    q, k, v, o, do, lse = case(sq + sk + d + batch + 7, batch, hq, hk, sq, sk, d)
    plant_nonfinite(q, k, v, do, seed=sum(shape))
    scale = float(np.float32(1 / np.sqrt(d)))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    program = AttentionBackward.from_jit(lambda defn, **kw: intent.jit(defn, backend="hip", **kw),
                                         head_group=hq // hk, causal=causal)
    grad_q, grad_k, grad_v = program.run(t(q), t(k), t(v), t(o), t(do), t(lse), scale)
    delta = oracle.attention_bwd_delta(o, do)
    want_dq = oracle.attention_bwd_dq(q, k, v, do, lse, delta, scale, causal, head_group=hq // hk)
    want_dk, want_dv = oracle.attention_bwd_dkdv(q, k, v, do, lse, delta, scale, causal, head_group=hq // hk)
    for got, want in ((grad_q, want_dq), (grad_k, want_dk), (grad_v, want_dv)):
        want = want.astype(np.float64)
        assert np.isfinite(want).mean() > 0.2           # a good part of each tensor stays finite
        close(got.cpu().numpy(), want)


def test_benchmarked_shape_matches_autograd_and_oracle(device):
    """The benchmarked shape, B4 HQ32 HK8 S4096 D128 causal: all of dQ, dK, dV against float32
    autograd of grouped-head attention on the GPU (o and lse from the same float32 forward), and
    the first key head of batch 0 (its four query heads) against the oracle."""
    batch, hq, hk, s, d = 4, 32, 8, 4096, 128
    group = hq // hk
    announce("attention backward, benchmarked shape", (batch, hq, hk, s, d))
    rng = np.random.default_rng(5)
    q = inputs.normal(rng, (batch, hq, s, d), "f16")
    k = inputs.normal(rng, (batch, hk, s, d), "f16")
    v = inputs.normal(rng, (batch, hk, s, d), "f16")
    do = inputs.normal(rng, (batch, hq, s, d), "f16")
    scale = float(np.float32(1 / np.sqrt(d)))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    tq, tk, tv, tdo = t(q), t(k), t(v), t(do)
    mask = torch.ones(s, s, dtype=torch.bool, device=device).tril()
    o16 = torch.empty_like(tq)
    lse = torch.empty(batch, hq, s, dtype=torch.float32, device=device)
    want = [torch.empty(x.shape, dtype=torch.float32, device=device) for x in (tq, tk, tv)]
    for b in range(batch):   # float32 forward and autograd, one batch element at a time
        qb = tq[b].float().requires_grad_(True)
        kb = tk[b].float().requires_grad_(True)
        vb = tv[b].float().requires_grad_(True)
        kx = kb.repeat_interleave(group, dim=0)
        vx = vb.repeat_interleave(group, dim=0)
        scores = torch.matmul(qb, kx.transpose(1, 2).contiguous()) * scale
        scores = scores.masked_fill(~mask, float("-inf"))
        lse[b] = torch.logsumexp(scores, dim=-1).detach()
        out = torch.matmul(torch.softmax(scores, dim=-1), vx)
        o16[b] = out.detach().half()
        out.backward(tdo[b].float())
        want[0][b], want[1][b], want[2][b] = qb.grad, kb.grad, vb.grad
        del scores, out, qb, kb, vb, kx, vx
    program = AttentionBackward.from_jit(lambda defn, **kw: intent.jit(defn, backend="hip", **kw),
                                         head_group=group, causal=True)
    grads = program.run(tq, tk, tv, o16, tdo, lse, scale)
    torch.cuda.synchronize()
    for got, ref in zip(grads, want):
        close(got.cpu().numpy(), ref.cpu().numpy())
    o_np, lse_np = o16[:1, :group].cpu().numpy(), lse[:1, :group].cpu().numpy()
    delta = oracle.attention_bwd_delta(o_np, do[:1, :group])
    want_dq = oracle.attention_bwd_dq(q[:1, :group], k[:1, :1], v[:1, :1], do[:1, :group], lse_np, delta, scale, True,
                                      head_group=group)
    want_dk, want_dv = oracle.attention_bwd_dkdv(q[:1, :group], k[:1, :1], v[:1, :1], do[:1, :group], lse_np, delta,
                                                 scale, True, head_group=group)
    close(grads[0][:1, :group].cpu().numpy(), want_dq)
    close(grads[1][:1, :1].cpu().numpy(), want_dk)
    close(grads[2][:1, :1].cpu().numpy(), want_dv)


@pytest.mark.parametrize("shape,causal", [((1, 2, 1, 128, 128, 64), True), ((1, 4, 2, 300, 300, 128), True),
                                          ((1, 2, 2, 200, 333, 64), False)])
def test_static_workspace_option_runs_the_unsplit_kernels(device, shape, causal):
    """backend_options={"workspace": "static"}: prepare allocates no partial-sum workspace, so small grids
    run unsplit; the results hold the same bar against the oracle."""
    batch, hq, hk, sq, sk, d = shape
    announce("attention backward workspace=static", shape, causal)
    q, k, v, o, do, lse = case(sq * 7 + d, batch, hq, hk, sq, sk, d)
    scale = float(np.float32(1 / np.sqrt(d)))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    jit = lambda defn, **kw: intent.jit(defn, backend="hip", backend_options={"workspace": "static"}, **kw)  # noqa: E731
    prepared = AttentionBackward.from_jit(jit, head_group=hq // hk, causal=causal).prepare(
        t(q), t(k), t(v), t(o), t(do), t(lse), scale)
    for call in prepared.calls[1:]:
        chosen, *others = call.inspect_configurations()
        assert dict(chosen.configuration)["workspace_bytes"] == 0 and dict(chosen.configuration)["split"] == 0
        assert all(not a.eligible and a.reasons for a in others)
    prepared.launch()
    grad_q, grad_k, grad_v = prepared.result()
    delta = oracle.attention_bwd_delta(o, do)
    want_dk, want_dv = oracle.attention_bwd_dkdv(q, k, v, do, lse, delta, scale, causal, head_group=hq // hk)
    close(grad_q.cpu().numpy(), oracle.attention_bwd_dq(q, k, v, do, lse, delta, scale, causal, head_group=hq // hk))
    close(grad_k.cpu().numpy(), want_dk)
    close(grad_v.cpu().numpy(), want_dv)


def test_tuning_config_pins_the_unsplit_kernels(device, tmp_path):
    """tuning_config {"hip.attention_backward": [[0]]} at the reference's example shape (which splits by
    default): the unsplit kernels run, tuning_configurations lists only that row, and both bindings
    meet the oracle. The default table lists the split row first and takes it here."""
    import json

    batch, hq, hk, sq, sk, d = 2, 8, 2, 1024, 1024, 64
    announce("attention backward tuning_config")
    q, k, v, o, do, lse = case(77, batch, hq, hk, sq, sk, d)
    scale = float(np.float32(1 / np.sqrt(d)))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    config = tmp_path / "tuning.json"
    config.write_text(json.dumps({"columns": ["split"], "families": {"hip.attention_backward": [[0]]}}))
    delta = oracle.attention_bwd_delta(o, do)
    want_dq = oracle.attention_bwd_dq(q, k, v, do, lse, delta, scale, True, head_group=hq // hk)
    from intent_amd.examples.kernels.backward.attention import attention_backward_dq

    for tuning, rows in ((None, [(1,), (0,)]), (config, [(0,)])):
        kernel = intent.jit(attention_backward_dq, backend="hip", tuning_config=tuning,
                            constexprs={"HEAD_GROUP": hq // hk, "CAUSAL": True})
        args = (t(q), t(k), t(v), t(do), t(lse), t(delta), scale)
        call = kernel.prepare(*args)
        call.launch()
        assert dict(call.inspect_configurations()[0].configuration)["split"] == rows[0][0]
        out = torch.empty_like(args[0])
        listed = kernel.artifacts[0].tuning_configurations(*args[:6], out, scale)
        assert [c.values for c in listed] == rows and all(c.parameters[0].name == "split" for c in listed)
        close(call.result().cpu().numpy(), want_dq)
