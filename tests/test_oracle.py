"""Pins the CPU oracle (oracle/) before it is trusted as the parity reference.

Each oracle function is checked against the float64 golden fixtures (closed forms
computed without the oracle), against library routines (torch float64, scipy), and
against exact special cases chosen so that a dropped term, a wrong sign, index or
transposed operand fails at least one of them."""
import numpy as np
import pytest
import torch

import oracle
from intent_amd.examples import inputs

TINY = 1e-30


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return np.max(np.abs(got - want) / (np.abs(want) + TINY))


# ------------------------------------------------------------------------------ conversions
def test_half_to_float_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.half_to_float(bits)
    want = bits.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def test_float_to_half_matches_numpy():
    rng = np.random.default_rng(0)
    samples = np.concatenate([
        (rng.standard_normal(200_000) * 10.0 ** rng.integers(-9, 6, 200_000)).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e10, -1e10, np.inf, -np.inf, 6.1035156e-05,
                  5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 8.940697e-08], np.float32),
        # every f16 value and the midpoints between neighbours (ties to even)
        np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32),
    ])
    samples = samples.astype(np.float32)
    got = oracle.float_to_half_bits(samples)
    want = samples.astype(np.float16).view(np.uint16)
    nan = np.isnan(samples)
    assert (got[~nan] == want[~nan]).all()
    assert np.isnan(got[nan].view(np.float16)).all()
    halves = np.arange(0, 0x7bff, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((halves[:-1] + halves[1:]) / 2).astype(np.float32)  # exact in f32
    assert (oracle.float_to_half_bits(mids) == mids.astype(np.float16).view(np.uint16)).all()


def test_float_to_bf16_matches_torch():
    rng = np.random.default_rng(1)
    samples = np.concatenate([rng.standard_normal(100_000).astype(np.float32) * 1e3,
                              rng.integers(0, 2**32, 100_000, dtype=np.uint64).astype(np.uint32).view(np.float32),
                              np.array([np.inf, -np.inf, 0.0, -0.0, 3.3895314e38], np.float32)])
    got = oracle.float_to_bf16_bits(samples)
    want = torch.from_numpy(samples).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(samples)
    assert (got[~nan] == want[~nan]).all()
    assert np.isnan(oracle.bf16_bits_to_float(got[nan])).all()
    assert (inputs._bf16_bits(samples)[~nan] == want[~nan]).all()


# ------------------------------------------------------------------------------ softmax
def test_softmax_f32_golden(golden):
    g = golden("softmax")
    y = oracle.softmax_fwd(g["softmax_f32_x"])
    assert rel_err(y, g["softmax_f32_y"]) < 1e-5
    assert (y[2, ::3] == 0).all()                       # -inf entries give exact zeros
    assert y[3, 17] == 1.0 and (np.delete(y[3], 17) == 0).all()  # exp(-120) underflows in f32
    assert np.allclose(y[1], 1.0 / 1000, rtol=1e-6)


def test_softmax_16bit_golden(golden):
    g = golden("softmax")
    y16 = oracle.softmax_fwd(g["softmax_f16_x"]).astype(np.float64)
    want = g["softmax_f16_y"]
    assert np.all(np.abs(y16 - want) <= 1e-2 * 0 + 2e-2 * np.abs(want) + 1e-7)
    # within one f16 rounding of the exact value
    assert np.max(np.abs(y16 - want) / np.maximum(np.abs(want), 6.1e-5)) < 2 ** -10
    yb = oracle.bf16_bits_to_float(oracle.softmax_fwd(g["softmax_bf16_x"], storage="bf16")).astype(np.float64)
    assert np.max(np.abs(yb - g["softmax_bf16_y"]) / np.maximum(g["softmax_bf16_y"], 1e-30)) < 2 ** -7
    y2 = oracle.softmax_fwd(g["softmax_pow2_x"])
    assert (y2 == np.float32(1 / 1024)).all()


def test_softmax_matches_torch_and_invariants():
    rng = np.random.default_rng(5)
    x = inputs.normal(rng, (64, 777), "f32", 5)
    y = oracle.softmax_fwd(x)
    ref = torch.softmax(torch.from_numpy(x).double(), dim=1).numpy()
    assert rel_err(y, ref) < 1e-5
    assert np.allclose(y.astype(np.float64).sum(axis=1), 1.0, atol=777 * 2**-24)
    shifted = oracle.softmax_fwd((x + np.float32(3.0)).astype(np.float32))
    assert rel_err(shifted, ref) < 1e-5


def test_softmax_nan_semantics():
    x = np.zeros((3, 64), np.float32)
    x[0, 5] = np.nan                     # NaN anywhere -> all-NaN row (through the sum)
    x[1, :] = -np.inf                    # all -inf -> NaN row
    x[2, 9] = np.inf                     # +inf -> inf - inf = NaN -> NaN row
    y = oracle.softmax_fwd(x)
    assert np.isnan(y).all()


def test_softmax_bwd_golden_and_autograd(golden):
    g = golden("softmax_bwd")
    dx = oracle.softmax_bwd(g["softmax_bwd_f32_p"], g["softmax_bwd_f32_dy"])
    want = g["softmax_bwd_f32_dx"]
    scale = np.abs(g["softmax_bwd_f32_p"].astype(np.float64)) * (np.abs(g["softmax_bwd_f32_dy"]).max() + 1)
    assert np.all(np.abs(dx - want) <= 1e-5 * scale + TINY)
    dx16 = oracle.softmax_bwd(g["softmax_bwd_f16_p"], g["softmax_bwd_f16_dy"]).astype(np.float64)
    w16 = g["softmax_bwd_f16_dx"]
    assert np.all(np.abs(dx16 - w16) <= 2e-2 * np.abs(w16) + 1e-2 * np.abs(w16).max())
    # Jacobian-vector product of softmax in float64 equals the closed form.
    rng = np.random.default_rng(6)
    logits = torch.from_numpy(inputs.normal(rng, (5, 300), "f32", 2)).double().requires_grad_()
    p = torch.softmax(logits, dim=1)
    dy = torch.from_numpy(inputs.normal(rng, (5, 300), "f32")).double()
    (grad,) = torch.autograd.grad(p, logits, dy)
    got = oracle.softmax_bwd(p.detach().float().numpy(), dy.float().numpy())
    assert np.max(np.abs(got - grad.numpy())) < 1e-5 * np.abs(grad.numpy()).max() + 1e-6


def test_softmax_bwd_constant_upstream_is_zero():
    rng = np.random.default_rng(7)
    p = oracle.softmax_fwd(inputs.normal(rng, (4, 64), "f32"))
    # sum(p) is 1 within rounding, so dy - sum(p dy) is tiny but not exactly zero in general;
    # with one-hot p it is exact.
    onehot = np.zeros((4, 64), np.float32)
    onehot[np.arange(4), [0, 5, 9, 63]] = 1.0
    assert (oracle.softmax_bwd(onehot, np.full((4, 64), 3.0, np.float32)) == 0).all()
    dx = oracle.softmax_bwd(p, np.full((4, 64), 2.0, np.float32))
    assert np.abs(dx).max() < 1e-6


# ------------------------------------------------------------------------------ GEMM
def test_gemm_golden(golden):
    g = golden("gemm")
    c = oracle.bf16_bits_to_float(oracle.gemm_bf16(g["gemm_a"], g["gemm_b"])).astype(np.float64)
    want = g["gemm_c64"]
    assert np.all(np.abs(c - want) <= 2e-2 * np.abs(want) + 1e-2)
    assert np.max(np.abs(c - want) / np.maximum(np.abs(want), 1e-3)) <= 2 ** -8 + 1e-3
    ci = oracle.gemm_bf16(g["gemm_int_a"], g["gemm_int_b"])
    assert (ci == g["gemm_int_c"]).all()                 # exact integer case, bit for bit


def test_gemm_identity_and_permutation():
    rng = np.random.default_rng(8)
    a = inputs.uniform(rng, (24, 24), -1, 1, "bf16")
    eye = inputs._bf16_bits(np.eye(24, dtype=np.float32))
    assert (oracle.gemm_bf16(a, eye) == a).all()
    assert (oracle.gemm_bf16(eye, a) == a).all()
    perm = rng.permutation(24)
    pm = inputs._bf16_bits(np.eye(24, dtype=np.float32)[perm])
    assert (oracle.gemm_bf16(pm, a) == a[perm]).all()     # rows permuted: catches a transposed operand


# ------------------------------------------------------------------------------ attention
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("chunk", [16, 64, 128])
def test_attention_golden(golden, causal, chunk):
    g = golden("attention")
    for prefix in ("attn", "attn_rect"):
        q, k, v = g[f"{prefix}_q"], g[f"{prefix}_k"], g[f"{prefix}_v"]
        o = oracle.attention_fwd_f16(q, k, v, float(g["attn_scale"]), causal, chunk=chunk).astype(np.float64)
        want = g[f"{prefix}_causal_o" if causal else f"{prefix}_full_o"].astype(np.float64)
        assert np.all(np.abs(o - want) <= 2e-2 * np.abs(want) + 1e-2)


def test_attention_special_rows():
    rng = np.random.default_rng(9)
    q, k, v, scale = inputs.attention_f16(seed=9, batch=1, heads=2, seq=70, dim=128)
    o = oracle.attention_fwd_f16(q, k, v, scale, True)
    assert (o[:, :, 0, :] == v[:, :, 0, :]).all()        # one valid key: p = 1, den = 1
    zq = np.zeros_like(q)
    oz = oracle.attention_fwd_f16(zq, k, v, scale, True).astype(np.float64)
    prefix_mean = np.cumsum(v.astype(np.float64), axis=2) / np.arange(1, 71)[None, None, :, None]
    assert np.abs(oz - prefix_mean).max() < 1e-2
    # Rows with no valid key (sq > sk under the top-left causal rule cannot happen; use sk = 0 rows)
    assert not np.isnan(o.astype(np.float32)).any()
    torch_o = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).float(), torch.from_numpy(k).float(), torch.from_numpy(v).float(), is_causal=True,
        scale=scale).numpy()
    assert np.all(np.abs(o.astype(np.float64) - torch_o) <= 2e-2 * np.abs(torch_o) + 1e-2)


# ------------------------------------------------------------------------------ SpMV
def test_spmv_golden(golden):
    g = golden("spmv")
    y = oracle.csr_spmv(g["spmv_offsets"], g["spmv_columns"], g["spmv_values"], g["spmv_x"])
    lengths = g["spmv_lengths"].astype(np.float64)
    bound = (np.maximum(lengths - 1, 0) * 2 ** -24 + 2 ** -24) * g["spmv_abs"]
    assert np.all(np.abs(y - g["spmv_y64"]) <= bound + TINY)
    assert y[5] == 0 and y[6] == 0                       # empty rows


def test_spmv_exact_probes(golden):
    g = golden("spmv")
    off, col, val = g["spmv_offsets"], g["spmv_columns"], g["spmv_values"]
    ones = oracle.csr_spmv(off, col, np.ones_like(val), np.ones(off.shape[0] - 1, np.float32))
    assert (ones == g["spmv_lengths"]).all()
    assert (oracle.csr_spmv(off, col, val, g["spmv_onehot_x"]) == g["spmv_onehot_y"]).all()
    rng = np.random.default_rng(10)
    ival = rng.integers(-4, 5, val.shape).astype(np.float32)
    ix = rng.integers(-4, 5, off.shape[0] - 1).astype(np.float32)
    y = oracle.csr_spmv(off, col, ival, ix)
    want = np.zeros(off.shape[0] - 1)
    np.add.at(want, np.repeat(np.arange(off.shape[0] - 1), np.diff(off)), ival.astype(np.float64) * ix[col])
    assert (y == want).all()


def test_spmv_strict_left_fold():
    """The oracle folds each row left to right with the product rounded first."""
    off = np.array([0, 3], np.int32)
    col = np.array([0, 1, 2], np.int32)
    val = np.array([1.0, 1e-8, 1e-8], np.float32)
    x = np.ones(3, np.float32)
    # ((0 + 1) + 1e-8) + 1e-8 == 1 in f32, whereas 1 + (1e-8 + 1e-8) != 1
    assert oracle.csr_spmv(off, col, val, x)[0] == np.float32(1.0)
    val2 = np.array([1e-8, 1e-8, 1.0], np.float32)
    assert oracle.csr_spmv(off, col, val2, x)[0] == np.float32(np.float32(2e-8) + np.float32(1.0))


def test_softmax_reduction_keeps_small_terms():
    """A dominant entry plus many terms below half an ulp of the running sum: a strictly
    sequential f32 sum drops all 4095 of them (relative error 1.7e-4 here); the oracle's
    64-accumulator reduction drops only the 63 that share the dominant entry's accumulator."""
    x = np.full((1, 4096), -17.0, np.float32)
    x[0, 0] = 0.0
    y = oracle.softmax_fwd(x)
    want = torch.softmax(torch.from_numpy(x).double(), dim=1).numpy()
    assert rel_err(y, want) < 5e-6


# ------------------------------------------------------------------------------ GEMM family
def test_gemm16_golden_relu_and_exact(golden):
    g = golden("gemm_family")
    a, b, want = g["gemm16_a"], g["gemm16_b"], g["gemm16_c64"]
    c = oracle.gemm16(a, b).astype(np.float64)
    assert np.all(np.abs(c - want) <= 2 ** -10 * np.abs(want) + 1e-3)     # f16 output rounding
    r = oracle.gemm16(a, b, relu=True).astype(np.float64)
    assert np.all(np.abs(r - g["gemm16_relu64"]) <= 2 ** -10 * np.abs(g["gemm16_relu64"]) + 1e-3)
    assert (r[want < -1e-3] == 0).all() and not np.signbit(r).any()       # relu gives +0, never -0
    np.testing.assert_array_equal(r, np.maximum(c, 0.0))                   # relu after the same sums
    exact = oracle.gemm16(g["gemm16_int_a"], g["gemm16_int_b"])
    assert (exact.view(np.uint16) == g["gemm16_int_c"].view(np.uint16)).all()


def test_gemm16_nan_and_signed_zero():
    a = np.array([[np.nan, 1.0], [-1.0, 0.0], [0.0, 0.0]], np.float16)
    b = np.array([[1.0, 2.0], [3.0, 4.0]], np.float16)
    plain = oracle.gemm16(a, b)
    relu = oracle.gemm16(a, b, relu=True)
    assert np.isnan(relu[0]).all() and np.isnan(plain[0]).all()           # maximum propagates NaN
    assert (relu[1] == 0).all() and not np.signbit(relu[1]).any()         # negative sums -> +0
    assert (plain[1] == np.array([-1.0, -2.0], np.float16)).all()
    assert not np.signbit(relu[2]).any()


def test_gemm16_bf16_matches_gemm_bf16():
    rng = np.random.default_rng(12)
    a = inputs.uniform(rng, (20, 36), -1, 1, "bf16")
    b = inputs.uniform(rng, (36, 28), -1, 1, "bf16")
    assert (oracle.gemm16(a, b, storage="bf16") == oracle.gemm_bf16(a, b)).all()


def test_gemm_f32_golden_linear_and_exact(golden):
    g = golden("gemm_family")
    a, b, want, bound = g["gemm32_a"], g["gemm32_b"], g["gemm32_c64"], g["gemm32_abs64"]
    c = oracle.gemm_f32(a, b)
    assert np.all(np.abs(c - want) <= 1e-5 * bound)                        # backward-error bound
    lin = oracle.gemm_f32(a, np.ascontiguousarray(b.T), transpose_b=True)
    assert (lin == c).all()                                                # same sums, transposed layout
    rng = np.random.default_rng(13)
    ai = rng.integers(-8, 9, (17, 50)).astype(np.float32)
    bi = rng.integers(-8, 9, (50, 9)).astype(np.float32)
    assert (oracle.gemm_f32(ai, bi) == (ai.astype(np.float64) @ bi).astype(np.float32)).all()
    eye = np.eye(50, dtype=np.float32)
    assert (oracle.gemm_f32(ai, eye) == ai).all()
    perm = rng.permutation(9)
    assert (oracle.gemm_f32(ai, np.ascontiguousarray(bi[:, perm])) == oracle.gemm_f32(ai, bi)[:, perm]).all()


# ------------------------------------------------------------------------------ attention family
@pytest.mark.parametrize("causal", [True, False])
def test_attention_grouped_golden(golden, causal):
    g = golden("attention_family")
    tag = "causal" if causal else "full"
    scale = float(g["gqa_scale"])
    o = oracle.attention_fwd(g["gqa_q"], g["gqa_k"], g["gqa_v"], scale, causal, head_group=int(g["gqa_group"]))
    want = g[f"gqa_{tag}_o"].astype(np.float64)
    assert np.all(np.abs(o.astype(np.float64) - want) <= 2e-2 * np.abs(want) + 1e-2)
    ob = oracle.attention_fwd(g["bf16_q"], g["bf16_k"], g["bf16_v"], scale, causal,
                              head_group=int(g["bf16_group"]), storage="bf16")
    got = oracle.bf16_bits_to_float(ob).astype(np.float64)
    want = g[f"bf16_{tag}_o"].astype(np.float64)
    assert np.all(np.abs(got - want) <= 4e-2 * np.abs(want) + 2e-2)       # bf16 P and output rounding


def test_attention_grouped_equals_repeated_heads():
    g = np.random.default_rng(14)
    q = inputs.normal(g, (2, 6, 33, 128), "f16")
    k = inputs.normal(g, (2, 2, 41, 128), "f16")
    v = inputs.normal(g, (2, 2, 41, 128), "f16")
    scale = float(np.float32(1 / np.sqrt(128)))
    grouped = oracle.attention_fwd(q, k, v, scale, True, head_group=3)
    heads = np.arange(6) // 3
    repeated = oracle.attention_fwd(q, np.ascontiguousarray(k[:, heads]), np.ascontiguousarray(v[:, heads]), scale,
                                    True)
    assert (grouped.view(np.uint16) == repeated.view(np.uint16)).all()
    assert (repeated.view(np.uint16) == oracle.attention_fwd_f16(
        q, np.ascontiguousarray(k[:, heads]), np.ascontiguousarray(v[:, heads]), scale, True).view(np.uint16)).all()
    wrong = oracle.attention_fwd(q, np.ascontiguousarray(k[:, ::-1]), np.ascontiguousarray(v[:, ::-1]), scale, True,
                                 head_group=3)
    assert (wrong.view(np.uint16) != grouped.view(np.uint16)).any()         # the head mapping matters


@pytest.mark.parametrize("d,dv", [(128, 64), (64, 128)])
@pytest.mark.parametrize("storage", [None, "bf16"])
def test_attention_value_width_independent_of_key_width(d, dv, storage):
    """DV != D: against float64 softmax attention, and split along the value columns. The weights do
    not depend on V, so the first 64 columns of an output with DV = 128 equal, bit for bit, the
    output with V cut to its first 64 columns (and the same for the last 64)."""
    g = np.random.default_rng(d + 3 * dv + (storage is None))
    kind = storage or "f16"
    q = inputs.normal(g, (1, 4, 37, d), kind)
    k = inputs.normal(g, (1, 2, 45, d), kind)
    v = inputs.normal(g, (1, 2, 45, dv), kind)
    scale = float(np.float32(1 / np.sqrt(d)))
    o = oracle.attention_fwd(q, k, v, scale, True, head_group=2, storage=storage)
    assert o.shape == (1, 4, 37, dv)
    as64 = (lambda a: oracle.bf16_bits_to_float(a).astype(np.float64)) if storage else (lambda a: a.astype(np.float64))
    heads = np.arange(4) // 2
    s = np.einsum("bhqd,bhkd->bhqk", as64(q), as64(k)[:, heads]) * scale
    s[..., np.triu_indices(37, 1, 45)[0], np.triu_indices(37, 1, 45)[1]] = -np.inf
    w = np.exp(s - s.max(-1, keepdims=True))
    want = np.einsum("bhqk,bhkd->bhqd", w / w.sum(-1, keepdims=True), as64(v)[:, heads])
    tol = (4e-2, 2e-2) if storage else (2e-2, 1e-2)
    assert np.all(np.abs(as64(o) - want) <= tol[0] * np.abs(want) + tol[1])
    if dv == 128:
        for part in (slice(0, 64), slice(64, 128)):
            piece = oracle.attention_fwd(q, k, np.ascontiguousarray(v[..., part]), scale, True, head_group=2,
                                         storage=storage)
            assert (piece.view(np.uint16) == o[..., part].view(np.uint16)).all()


def test_attention_bf16_first_causal_row():
    g = np.random.default_rng(15)
    q, k, v = (inputs.normal(g, (1, 2, 20, 128), "bf16") for _ in range(3))
    o = oracle.attention_fwd(q, k, v, float(np.float32(1 / np.sqrt(128))), True, storage="bf16")
    assert (o[:, :, 0, :] == v[:, :, 0, :]).all()                            # one valid key: p = 1, den = 1
    with pytest.raises(ValueError):
        oracle.attention_fwd(q, k[:, :1], v[:, :1], 1.0, True, head_group=3, storage="bf16")


# ------------------------------------------------------------------------------ attention backward
def _attention_autograd64(q, k, v, do, scale, causal, group):
    """float64 reference: forward with grouped heads, lse, and autograd gradients."""
    tq, tk, tv = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (q, k, v))
    kk, vv = tk.repeat_interleave(group, dim=1), tv.repeat_interleave(group, dim=1)
    s = torch.einsum("bhqd,bhkd->bhqk", tq, kk) * scale
    if causal:
        s = s.masked_fill(torch.ones(q.shape[2], k.shape[2], dtype=torch.bool).triu(1), float("-inf"))
    lse = torch.logsumexp(s, -1)
    o = torch.einsum("bhqk,bhkd->bhqd", torch.softmax(s, -1), vv)
    o.backward(torch.tensor(do, dtype=torch.float64))
    return o.detach().numpy(), lse.detach().numpy(), tq.grad.numpy(), tk.grad.numpy(), tv.grad.numpy()


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("d,group", [(64, 4), (128, 1)])
def test_attention_backward_matches_autograd(causal, d, group):
    rng = np.random.default_rng(16 + d + group)
    hk, sq = 2, 45
    q = inputs.normal(rng, (1, hk * group, sq, d), "f16")
    k = inputs.normal(rng, (1, hk, sq, d), "f16")
    v = inputs.normal(rng, (1, hk, sq, d), "f16")
    do = inputs.normal(rng, (1, hk * group, sq, d), "f16")
    scale = float(np.float32(1 / np.sqrt(d)))
    o, lse, gq, gk, gv = _attention_autograd64(q, k, v, do, scale, causal, group)
    o16 = o.astype(np.float16)
    delta = oracle.attention_bwd_delta(o16, do)
    np.testing.assert_allclose(delta, np.sum(o16.astype(np.float64) * do.astype(np.float64), -1), rtol=1e-5,
                               atol=1e-5)
    lse32 = lse.astype(np.float32)
    dq = oracle.attention_bwd_dq(q, k, v, do, lse32, delta, scale, causal, head_group=group)
    dk, dv = oracle.attention_bwd_dkdv(q, k, v, do, lse32, delta, scale, causal, head_group=group)
    for got, want in ((dq, gq), (dk, gk), (dv, gv)):
        err = np.abs(got.astype(np.float64) - want)
        assert np.all(err <= 2e-2 * np.abs(want) + 5e-3 * max(1.0, np.abs(want).max()))


def test_attention_backward_grouped_sums_heads():
    """dK/dV of a key head equal the sum of the ungrouped results of its query heads."""
    rng = np.random.default_rng(17)
    q = inputs.normal(rng, (1, 4, 30, 64), "f16")
    k = inputs.normal(rng, (1, 2, 30, 64), "f16")
    v = inputs.normal(rng, (1, 2, 30, 64), "f16")
    do = inputs.normal(rng, (1, 4, 30, 64), "f16")
    lse = rng.standard_normal((1, 4, 30)).astype(np.float32) + 6.0
    delta = rng.standard_normal((1, 4, 30)).astype(np.float32)
    dk, dv = oracle.attention_bwd_dkdv(q, k, v, do, lse, delta, 0.125, True, head_group=2)
    heads = np.arange(4) // 2
    kr, vr = np.ascontiguousarray(k[:, heads]), np.ascontiguousarray(v[:, heads])
    dk1, dv1 = oracle.attention_bwd_dkdv(q, kr, vr, do, lse, delta, 0.125, True, head_group=1)
    for grouped, single in ((dk, dk1), (dv, dv1)):
        summed = single.astype(np.float64).reshape(1, 2, 2, 30, 64).sum(axis=2)
        assert np.all(np.abs(grouped.astype(np.float64) - summed) <= 2e-3 * np.abs(summed) + 2e-3)
    dq = oracle.attention_bwd_dq(q, k, v, do, lse, delta, 0.125, True, head_group=2)
    dq1 = oracle.attention_bwd_dq(q, kr, vr, do, lse, delta, 0.125, True, head_group=1)
    assert (dq.view(np.uint16) == dq1.view(np.uint16)).all()                # dq only reads K/V


# ------------------------------------------------------------------------------ paged decode
def _decode64(q, kc, vc, page_offsets, page_indices, lengths, scale, group, page_size):
    """float64 decode attention over each sequence's logical tokens; also the base-2 lse."""
    batch, heads, d = q.shape
    out = np.zeros((batch, heads, vc.shape[3]))
    lse2 = np.zeros((batch, heads))
    for b in range(batch):
        tokens = np.arange(lengths[b])
        physical = page_indices[page_offsets[b] + tokens // page_size]
        for h in range(heads):
            k = kc[physical, tokens % page_size, h // group].astype(np.float64)
            v = vc[physical, tokens % page_size, h // group].astype(np.float64)
            s = k @ q[b, h].astype(np.float64) * scale
            m = s.max()
            w = np.exp(s - m)
            out[b, h] = w @ v / w.sum()
            lse2[b, h] = (m + np.log(w.sum())) / np.log(2)
    return out, lse2


def test_paged_decode_partials_one_split_is_attention():
    q, kc, vc, po, pi, ln, so = inputs.paged_decode(seed=18, batch=3, query_heads=8, kv_heads=2, dim=64,
                                                    page_size=16, lengths=(200, 37, 64), splits=1)
    scale = float(np.float32(1 / np.sqrt(64)))
    lse, out = oracle.paged_decode_partials(q, kc, vc, po, pi, ln, so, scale, page_size=16, head_group=4, splits=1)
    want, want_lse = _decode64(q, kc, vc, po, pi, ln, scale, 4, 16)
    assert np.all(np.abs(out[:, :, 0] - want) <= 2e-2 * np.abs(want) + 1e-2)
    assert np.all(np.abs(lse[:, :, 0] - want_lse) <= 1e-4 * np.abs(want_lse) + 1e-4)


def test_paged_decode_split_partials_merge_in_base_two():
    q, kc, vc, po, pi, ln, so = inputs.paged_decode(seed=19, batch=2, query_heads=4, kv_heads=1, dim=64,
                                                    page_size=16, lengths=(250, 90), splits=4)
    scale = 0.125
    lse, out = oracle.paged_decode_partials(q, kc, vc, po, pi, ln, so, scale, page_size=16, head_group=4, splits=4)
    assert np.isneginf(lse[1, :, 3]).all() and (out[1, :, 3] == 0).all()   # sequence 1 ends before split 3
    m = lse.max(axis=-1, keepdims=True)
    w = np.exp2(lse.astype(np.float64) - m)
    merged = np.einsum("bhs,bhsd->bhd", w, out.astype(np.float64)) / w.sum(-1)[..., None]
    want, _ = _decode64(q, kc, vc, po, pi, ln, scale, 4, 16)
    assert np.all(np.abs(merged - want) <= 2e-2 * np.abs(want) + 1e-2)


def test_splitk_reduce_formula_and_empty_rows():
    rng = np.random.default_rng(20)
    partial = rng.standard_normal((2, 3, 5, 64)).astype(np.float32)
    lse = (rng.standard_normal((2, 3, 5)) * 3).astype(np.float32)
    lse[0, 1, 2] = -np.inf
    lse[1, 2, :] = -np.inf
    out = oracle.splitk_reduce_f32_to_f16(partial, lse).astype(np.float64)
    l64 = lse.astype(np.float64)
    with np.errstate(invalid="ignore"):
        w = np.exp(l64 - l64.max(-1, keepdims=True))                   # natural exp, as the definition writes
        want = np.einsum("bhs,bhsd->bhd", w, partial.astype(np.float64)) / w.sum(-1)[..., None]
    ok = ~np.isnan(want)
    assert np.isnan(out[1, 2]).all() and np.isnan(want[1, 2]).all()    # every split empty -> NaN
    assert np.all(np.abs(out[ok] - want[ok]) <= 2e-3 * np.abs(want[ok]) + 1e-3)


def test_csr_spmm_columns_are_pinned_spmv_folds():
    """Every output column is csr_spmv of that dense column, bit for bit (same left fold, product
    rounded then added); the csr_spmv oracle is pinned by its golden vectors."""
    offsets, columns, values, dense = inputs.csr_spmm(seed=21, rows=300, cols=257, per_row=9, features=13)
    out = oracle.csr_spmm(offsets, columns, values, dense)
    for f in range(dense.shape[1]):
        assert (out[:, f] == oracle.csr_spmv(offsets, columns, values, np.ascontiguousarray(dense[:, f]))).all()


def test_csr_spmm_against_scipy_float64_and_probes():
    import scipy.sparse

    offsets, columns, values, dense = inputs.csr_spmm(seed=22, rows=512, cols=400, per_row=17, features=64)
    out = oracle.csr_spmm(offsets, columns, values, dense).astype(np.float64)
    a = scipy.sparse.csr_matrix((values.astype(np.float64), columns, offsets), shape=(512, 400))
    want = a @ dense.astype(np.float64)
    mag = abs(a) @ np.abs(dense.astype(np.float64))
    assert np.all(np.abs(out - want) <= 17 * 2.0 ** -24 * mag + 1e-38)
    # identity dense: out[r, c] = value of (r, c) (exact); ragged rows with empty ones
    lengths = np.array([0, 3, 1, 0, 5], np.int64)
    rng = np.random.default_rng(23)
    off, col = inputs.csr_matrix(rng, lengths, 6)
    val = inputs.uniform(rng, off[-1], -1, 1)
    got = oracle.csr_spmm(off, col, val, np.eye(6, dtype=np.float32))
    expect = np.zeros((5, 6), np.float32)
    for r in range(5):
        for nz in range(off[r], off[r + 1]):
            expect[r, col[nz]] = val[nz]
    assert (got == expect).all()


# ------------------------------------------------------------------------------ packed sequences
def _varlen64(q, k, v, cu, scale, causal, group):
    """float64 softmax attention of each packed sequence, written out directly (no oracle call)."""
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    o = np.zeros((q.shape[0], q.shape[1], v.shape[2]))
    for s in range(len(cu) - 1):
        lo, hi = cu[s], cu[s + 1]
        if hi <= lo:
            continue
        for h in range(q.shape[1]):
            logits = q[lo:hi, h] @ k[lo:hi, h // group].T * scale
            if causal:
                logits[np.triu_indices(hi - lo, 1)] = -np.inf
            w = np.exp(logits - logits.max(axis=1, keepdims=True))
            o[lo:hi, h] = (w / w.sum(axis=1, keepdims=True)) @ v[lo:hi, h // group]
    return o


@pytest.mark.parametrize("causal,group", [(True, 1), (False, 1), (True, 4)])
def test_attention_varlen_against_float64(causal, group):
    """Sequences of 0, 1, 63, 64, 65 and 300 rows packed back to back: every row matches float64
    attention over its own sequence only (a wrong offset, an off-by-one at a boundary or a wrong
    key head breaks it)."""
    g = np.random.default_rng(13 + group + causal)
    lengths = np.array([65, 0, 1, 300, 63, 64], np.int32)
    cu = np.concatenate(([0], np.cumsum(lengths))).astype(np.int32)
    total = int(cu[-1])
    q = inputs.normal(g, (total, 4 if group > 1 else 2, 64), "f16")
    hq = q.shape[1]
    k = inputs.normal(g, (total, hq // group, 64), "f16")
    v = inputs.normal(g, (total, hq // group, 128), "f16")
    scale = float(np.float32(1 / 8))
    o = oracle.attention_varlen_fwd(q, k, v, cu, scale, causal, head_group=group)
    want = _varlen64(q, k, v, cu, scale, causal, group)
    assert np.all(np.abs(o.astype(np.float64) - want) <= 2e-2 * np.abs(want) + 1e-2)
    q2 = q[:, 0, :].copy()
    o2 = oracle.attention_varlen_fwd(q2, np.ascontiguousarray(k[:, 0, :]), np.ascontiguousarray(v[:, 0, :]), cu,
                                     scale, causal)
    assert o2.shape == (total, 128) and (o2.view(np.uint16) == oracle.attention_varlen_fwd(
        q2[:, None], np.ascontiguousarray(k[:, :1]), np.ascontiguousarray(v[:, :1]), cu, scale,
        causal)[:, 0].view(np.uint16)).all()


def test_attention_varlen_equals_batched_and_isolates_sequences():
    """Equal lengths: the packed result is the batched oracle's, bit for bit. Changing the rows of
    one sequence leaves every other sequence's output unchanged."""
    g = np.random.default_rng(17)
    batch, seq, heads = 3, 96, 2
    q, k, v = (inputs.normal(g, (batch, heads, seq, 64), "f16") for _ in range(3))
    packed = [np.ascontiguousarray(t.transpose(0, 2, 1, 3).reshape(batch * seq, heads, 64)) for t in (q, k, v)]
    cu = np.arange(0, batch * seq + 1, seq, dtype=np.int32)
    o = oracle.attention_varlen_fwd(*packed, cu, 0.125, True)
    want = oracle.attention_fwd(q, k, v, 0.125, True).transpose(0, 2, 1, 3).reshape(batch * seq, heads, 64)
    assert (o.view(np.uint16) == want.view(np.uint16)).all()
    changed = [t.copy() for t in packed]
    for t in changed:
        t[seq:2 * seq] = inputs.normal(g, t[seq:2 * seq].shape, "f16")
    o2 = oracle.attention_varlen_fwd(*changed, cu, 0.125, True)
    keep = np.r_[0:seq, 2 * seq:3 * seq]
    assert (o2[keep].view(np.uint16) == o[keep].view(np.uint16)).all()
    assert not (o2[seq:2 * seq].view(np.uint16) == o[seq:2 * seq].view(np.uint16)).all()


# ------------------------------------------------------------------------------ key bias
def _bias64(q, k, v, bias, scale):
    """float64 softmax attention with an additive per-key bias, written out directly."""
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    logits = q @ k.transpose(0, 1, 3, 2) * scale + bias.astype(np.float64)[:, :, None, :]
    w = np.exp(logits - logits.max(axis=3, keepdims=True))
    return (w / w.sum(axis=3, keepdims=True)) @ v


@pytest.mark.parametrize("sq,sk,d,dv", [(70, 200, 64, 128), (33, 64, 128, 64), (5, 1, 64, 64)])
def test_attention_bias_against_float64(sq, sk, d, dv):
    """Random biases of spread 3 (they move the softmax well away from the unbiased one): the
    oracle meets float64 attention on every row, and a bias row of zeros gives the unbiased
    non-causal oracle (bit for bit where the scale is a power of two), so a dropped or misplaced
    bias term breaks one of the two."""
    g = np.random.default_rng(sq + sk + d)
    q, k = inputs.normal(g, (2, 3, sq, d), "f16"), inputs.normal(g, (2, 3, sk, d), "f16")
    v = inputs.normal(g, (2, 3, sk, dv), "f16")
    bias = (3.0 * g.standard_normal((2, 3, sk))).astype(np.float32)
    scale = float(np.float32(d ** -0.5))
    o = oracle.attention_bias_fwd(q, k, v, bias, scale).astype(np.float64)
    want = _bias64(q, k, v, bias, scale)
    assert np.all(np.abs(o - want) <= 2e-2 * np.abs(want) + 1e-2)
    unbiased = _bias64(q, k, v, np.zeros_like(bias), scale)
    assert sk == 1 or np.abs(want - unbiased).max() > 0.1   # the bias matters at this spread
    zero = oracle.attention_bias_fwd(q, k, v, np.zeros_like(bias), scale)
    plain = oracle.attention_fwd(q, k, v, scale, False)
    if d == 64:     # scale 1/8: (dot scale) log2 e rounds as dot (scale log2 e) does
        assert (zero.view(np.uint16) == plain.view(np.uint16)).all()
    else:
        assert np.abs(zero.astype(np.float64) - plain.astype(np.float64)).max() <= 2e-3


def test_attention_bias_row_selection_and_layout():
    """The bias of (batch b, head h) reaches only that row: a dominant key j0 (bias +40) returns
    v[j0] in that head and leaves every other head unchanged; a constant bias row leaves its head
    at the unbiased result; a strided bias view equals its contiguous copy."""
    g = np.random.default_rng(5)
    q, k = inputs.normal(g, (2, 2, 40, 64), "f16"), inputs.normal(g, (2, 2, 150, 64), "f16")
    v = inputs.normal(g, (2, 2, 150, 64), "f16")
    base = np.zeros((2, 2, 150), np.float32)
    plain = oracle.attention_bias_fwd(q, k, v, base, 0.125)
    dominant = base.copy()
    dominant[1, 0, 97] = 40.0
    o = oracle.attention_bias_fwd(q, k, v, dominant, 0.125)
    assert np.abs(o[1, 0].astype(np.float64) - v[1, 0, 97].astype(np.float64)[None, :]).max() <= 2e-3
    others = [(0, 0), (0, 1), (1, 1)]
    for b, h in others:
        assert (o[b, h].view(np.uint16) == plain[b, h].view(np.uint16)).all()
    shifted = base.copy()
    shifted[0, 1] = 7.5
    o = oracle.attention_bias_fwd(q, k, v, shifted, 0.125).astype(np.float64)
    assert np.abs(o[0, 1] - plain[0, 1].astype(np.float64)).max() <= 2e-3
    wide = (g.standard_normal((2, 2, 160))).astype(np.float32)
    view = wide[:, :, 5:155]
    assert (oracle.attention_bias_fwd(q, k, v, view, 0.125).view(np.uint16)
            == oracle.attention_bias_fwd(q, k, v, np.ascontiguousarray(view), 0.125).view(np.uint16)).all()


def test_attention_bias_minus_infinity():
    """-inf removes a key (weight 0) while its chunk keeps a finite score; a chunk whose every
    score is -inf makes the row NaN, as the reference's chunk summary does (max - max of -inf)."""
    g = np.random.default_rng(8)
    q, k = inputs.normal(g, (1, 1, 8, 64), "f16"), inputs.normal(g, (1, 1, 128, 64), "f16")
    v = inputs.normal(g, (1, 1, 128, 64), "f16")
    bias = np.zeros((1, 1, 128), np.float32)
    bias[0, 0, ::3] = -np.inf
    o = oracle.attention_bias_fwd(q, k, v, bias, 0.125).astype(np.float64)
    keep = np.isfinite(bias[0, 0])
    want = _bias64(q[:, :, :, :], k[:, :, keep], v[:, :, keep], bias[:, :, keep], 0.125)
    assert np.all(np.abs(o - want) <= 2e-2 * np.abs(want) + 1e-2)
    bias[0, 0, 64:] = -np.inf
    assert np.isnan(oracle.attention_bias_fwd(q, k, v, bias, 0.125, chunk=64).astype(np.float32)).all()


# ------------------------------------------------------------------------------ latent attention
def test_mla_prefill_oracle_pinned():
    """Zero position parts give the causal grouped attention oracle bit for bit; in general the
    oracle meets float64 causal attention over the concatenated [q | qpe] . [k | kpe] scores with
    one kpe row shared by every head, and the pinned attention oracle over the concatenation."""
    g = np.random.default_rng(31)
    B, H, HK, S, D, P = 2, 8, 2, 150, 64, 64
    q, qpe = inputs.normal(g, (B, H, S, D), "f16"), inputs.normal(g, (B, H, S, P), "f16")
    k, kpe, v = (inputs.normal(g, (B, HK, S, D), "f16"), inputs.normal(g, (B, 1, S, P), "f16"),
                 inputs.normal(g, (B, HK, S, D), "f16"))
    scale = float(np.float32((D + P) ** -0.5))
    zq, zk = np.zeros_like(qpe), np.zeros_like(kpe)
    plain = oracle.attention_fwd(q, k, v, scale, True, head_group=4)
    assert (oracle.mla_prefill(q, zq, k, zk, v, scale).view(np.uint16) == plain.view(np.uint16)).all()
    o = oracle.mla_prefill(q, qpe, k, kpe, v, scale).astype(np.float64)
    kq = np.repeat(k, 4, axis=1).astype(np.float64)
    logits = (q.astype(np.float64) @ kq.transpose(0, 1, 3, 2)
              + qpe.astype(np.float64) @ kpe.astype(np.float64).transpose(0, 1, 3, 2)) * scale
    logits[..., np.triu_indices(S, 1)[0], np.triu_indices(S, 1)[1]] = -np.inf
    w = np.exp(logits - logits.max(axis=3, keepdims=True))
    want = (w / w.sum(axis=3, keepdims=True)) @ np.repeat(v, 4, axis=1).astype(np.float64)
    assert np.all(np.abs(o - want) <= 2e-2 * np.abs(want) + 1e-2)
    assert np.abs(o - plain.astype(np.float64)).max() > 0.05         # the position part matters
    cat_q = np.concatenate([q, qpe], axis=3)
    cat_k = np.concatenate([k, np.repeat(kpe, HK, axis=1)], axis=3)
    cat = oracle.attention_fwd(cat_q, cat_k, v, scale, True, head_group=4)
    assert np.abs(o - cat.astype(np.float64)).max() <= 4e-3


# ------------------------------------------------------------------------------ decode variants
def _dense_decode64(q, k, v, scale, active=None):
    """float64 softmax of one query row per (batch, query head) over its key rows k [B,HQ,K,D]
    (already gathered per query head); returns (output, log2 of the sum of exp2 of the base-2
    logits)."""
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    logits = np.einsum("bhd,bhkd->bhk", q, k) * scale * np.log2(np.e)
    if active is not None:
        logits = np.where(active, logits, -np.inf)
    peak = logits.max(axis=2, keepdims=True)
    w = np.exp2(logits - np.where(np.isfinite(peak), peak, 0.0))
    total = w.sum(axis=2, keepdims=True)
    out = np.einsum("bhk,bhkd->bhd", w, v) / np.where(total > 0, total, 1.0)
    return out, (peak + np.log2(np.where(total > 0, total, 1.0)))[..., 0]


def test_grouped_decode_partials_oracle_pinned():
    """One part over every key is the bf16 attention oracle bit for bit; parts merged by their
    base-2 log-sums give float64 attention; a part past K is empty (-inf, 0); changing the keys of
    one part leaves the other parts' bits unchanged."""
    g = np.random.default_rng(21)
    B, HQ, HK, K, D = 2, 8, 2, 300, 64
    q = inputs._bf16_bits(g.standard_normal((B, HQ, 1, D)).astype(np.float32))
    k = inputs._bf16_bits(g.standard_normal((B, HK, K, D)).astype(np.float32))
    v = inputs._bf16_bits(g.standard_normal((B, HK, K, D)).astype(np.float32))
    lse, out = oracle.grouped_decode_partials(q, k, v, 0.125, parts=1, split_size=512)
    whole = oracle.attention_fwd(q, k, v, 0.125, False, head_group=4, storage="bf16")
    assert (out[:, :, 0] == whole[:, :, 0]).all()
    qf, kf, vf = (oracle.bf16_bits_to_float(a) for a in (q, k, v))
    want, want_lse = _dense_decode64(qf[:, :, 0], np.repeat(kf, 4, axis=1), np.repeat(vf, 4, axis=1), 0.125)
    assert np.abs(lse[:, :, 0] - want_lse).max() < 1e-3
    lse, out = oracle.grouped_decode_partials(q, k, v, 0.125, parts=6, split_size=60)    # part 5: keys 300..359
    assert np.isneginf(lse[:, :, 5]).all() and (out[:, :, 5] == 0).all()
    weights = np.exp2(lse[:, :, :5] - lse[:, :, :5].max(axis=2, keepdims=True))
    merged = (weights[..., None] * oracle.bf16_bits_to_float(out[:, :, :5])).sum(axis=2) / weights.sum(axis=2)[..., None]
    assert np.all(np.abs(merged - want) <= 2e-2 * np.abs(want) + 1e-2)
    k2 = k.copy()
    k2[:, :, 60:120] = inputs._bf16_bits(g.standard_normal((B, HK, 60, D)).astype(np.float32))
    lse2, out2 = oracle.grouped_decode_partials(q, k2, v, 0.125, parts=6, split_size=60)
    keep = [0, 2, 3, 4, 5]
    assert (out2[:, :, keep] == out[:, :, keep]).all() and (lse2[:, :, keep] == lse[:, :, keep]).all()
    assert not (lse2[:, :, 1] == lse[:, :, 1]).all()


def test_continuous_decode_oracle_pinned():
    """With every key admitted the oracle is the attention oracle bit for bit (token-major caches
    transposed); a random mask matches float64 attention over the admitted keys; a head whose
    mask is all zero gives 0; a key head's mask reaches only its own query heads."""
    g = np.random.default_rng(22)
    B, HQ, HK, K, D = 2, 8, 2, 300, 64
    q = inputs.normal(g, (B, HQ, D), "f16")
    k, v = inputs.normal(g, (B, K, HK, D), "f16"), inputs.normal(g, (B, K, HK, D), "f16")
    ones = np.ones((B, K, HK), np.uint8)
    o = oracle.continuous_gqa_decode(q, k, v, ones, 0.125)
    whole = oracle.attention_fwd(q[:, :, None].copy(), np.ascontiguousarray(k.transpose(0, 2, 1, 3)),
                                 np.ascontiguousarray(v.transpose(0, 2, 1, 3)), 0.125, False, head_group=4)
    assert (o.view(np.uint16) == whole[:, :, 0].view(np.uint16)).all()
    mask = (g.random((B, K, HK)) < 0.4).astype(np.uint8)
    mask[1, :, 1] = 0
    o = oracle.continuous_gqa_decode(q, k, v, mask, 0.125).astype(np.float64)
    kq = np.repeat(k.transpose(0, 2, 1, 3), 4, axis=1)
    vq = np.repeat(v.transpose(0, 2, 1, 3), 4, axis=1)
    active = np.repeat(mask.transpose(0, 2, 1), 4, axis=1) != 0
    want, _ = _dense_decode64(q, kq, vq, 0.125, active)
    assert np.all(np.abs(o - want) <= 2e-2 * np.abs(want) + 1e-2)
    assert (o[1, 4:] == 0).all() and (np.abs(o[1, :4]) > 0).any()
    mask2 = mask.copy()
    mask2[:, :, 0] = 1 - mask2[:, :, 0]
    o2 = oracle.continuous_gqa_decode(q, k, v, mask2, 0.125).astype(np.float64)
    assert (o2[:, 4:] == o[:, 4:]).all() and not (o2[:, :4] == o[:, :4]).all()


def test_varlen_decode_sink_oracle_pinned():
    """Sequences of 0, 1, 64, 65, 200 and 300 keys with MAX_BLOCKS 4 (256 keys read at most).
    With a zero sink the output is the attention oracle over the sequence's first 256 keys, bit for
    bit; the block logits and a nonzero sink match float64; keys past the cap change nothing."""
    g = np.random.default_rng(23)
    lengths = np.array([0, 1, 64, 65, 200, 300])
    cu = np.concatenate(([0], np.cumsum(lengths))).astype(np.int32)
    B, HQ, HK, D, U, cap = len(lengths), 4, 2, 64, int(cu[-1]), 4
    q = inputs.normal(g, (B, HQ, D), "f16")
    k, v = inputs.normal(g, (U, HK, D), "f16"), inputs.normal(g, (U, HK, D), "f16")
    zero = np.zeros(HQ, np.float32)
    o, logits = oracle.varlen_decode_sink(q, k, v, cu, zero, 0.125, max_blocks=cap)
    sink = np.array([0.0, 0.5, 3.0, 40.0], np.float32)
    o_s, logits_s = oracle.varlen_decode_sink(q, k, v, cu, sink, 0.125, max_blocks=cap)
    for b, n in enumerate(lengths):
        if n == 0:
            assert (o[b] == 0).all() and (logits[b] == 0).all() and (o_s[b] == 0).all()
            continue
        taken = min(n, 64 * cap)
        rows = slice(cu[b], cu[b] + taken)
        kb = np.ascontiguousarray(k[rows].transpose(1, 0, 2))[None]
        vb = np.ascontiguousarray(v[rows].transpose(1, 0, 2))[None]
        whole = oracle.attention_fwd(q[b][None, :, None].copy(), kb, vb, 0.125, False, head_group=2)[0, :, 0]
        assert (o[b].view(np.uint16) == whole.view(np.uint16)).all()
        scores = np.einsum("hd,hkd->hk", q[b].astype(np.float64),
                           np.repeat(kb[0], 2, axis=0).astype(np.float64)) * 0.125 * np.log2(np.e)
        peak = scores.max(axis=1)
        den = np.exp2(scores - peak[:, None]).sum(axis=1)
        blocks = -(-n // 64)
        for j in range(cap):
            if j < blocks:
                block_peak = scores[:, 64 * j:64 * (j + 1)].max(axis=1)
                for s_, lg in ((zero, logits), (sink, logits_s)):
                    want = np.exp2(block_peak - peak) / (den + s_)
                    assert np.allclose(lg[b, :, j], want, rtol=2e-3, atol=1e-6)
            else:
                assert (logits[b, :, j] == 0).all()
        ratio = den / (den + sink)
        assert np.all(np.abs(o_s[b].astype(np.float64) - o[b].astype(np.float64) * ratio[:, None])
                      <= 2e-2 * np.abs(o[b].astype(np.float64)) + 1e-2)
    k2, v2 = k.copy(), v.copy()
    tail = slice(cu[-2] + 256, cu[-1])           # keys 256..299 of the last sequence
    k2[tail], v2[tail] = 9.0, 9.0
    o2, logits2 = oracle.varlen_decode_sink(q, k2, v2, cu, sink, 0.125, max_blocks=cap)
    assert (o2.view(np.uint16) == o_s.view(np.uint16)).all() and (logits2 == logits_s).all()


# ------------------------------------------------------------------------------ int8 GEMM
def test_gemm_i8_oracle_pinned():
    """gemm_i8: against a scalar loop on a small case, an identity operand (c = b + bias exactly),
    and int32 wraparound, where a bias near the int32 limit plus a positive sum must wrap."""
    g = np.random.default_rng(19)
    a = g.integers(-128, 128, (5, 7)).astype(np.int8)
    b = g.integers(-128, 128, (7, 3)).astype(np.int8)
    bias = g.integers(-1000, 1000, 3).astype(np.int32)
    c = oracle.gemm_i8(a, b, bias)
    for i in range(5):
        for j in range(3):
            assert c[i, j] == sum(int(a[i, t]) * int(b[t, j]) for t in range(7)) + int(bias[j])
    eye = np.eye(7, dtype=np.int8)
    assert (oracle.gemm_i8(eye, b, bias) == b.astype(np.int32) + bias).all()
    top = np.full(3, 2**31 - 10, np.int32)
    ones = np.ones((1, 7), np.int8)
    wrapped = oracle.gemm_i8(ones, np.full((7, 3), 2, np.int8), top)
    assert (wrapped == np.int32(-2**31 + 4)).all()             # 2^31 - 10 + 14 wraps
    assert oracle.gemm_i8(np.zeros((2, 0), np.int8), np.zeros((0, 3), np.int8), bias).tolist() == [bias.tolist()] * 2


def test_quantized_gemm_oracle_pinned():
    """quantized_gemm: a scalar f32 chain on a small case; small integers (every step exact) against
    integer arithmetic with an exact division; ReLU before the residual, saturation on both sides,
    and truncation toward zero for negative halves."""
    g = np.random.default_rng(23)
    a = g.normal(size=(4, 6)).astype(np.float16)
    b = g.normal(size=(6, 5)).astype(np.float16)
    bias = g.normal(size=5).astype(np.float32)
    residual = (g.normal(size=(4, 5)) * 3).astype(np.float16)
    scale = g.uniform(0.05, 0.5, 5).astype(np.float32)
    out = oracle.quantized_gemm(a, b, bias, residual, scale)
    for i in range(4):
        for j in range(5):
            acc = np.float32(sum(float(a[i, t]) * float(b[t, j]) for t in range(6)))
            v = np.float32(max(np.float32(acc + bias[j]), np.float32(0)) + np.float32(residual[i, j]))
            v = min(max(np.float32(v / scale[j]), np.float32(-128)), np.float32(127))
            assert out[i, j] == int(np.trunc(v))
    ia = g.integers(-3, 4, (16, 8)).astype(np.float16)
    ib = g.integers(-3, 4, (8, 12)).astype(np.float16)
    ibias = g.integers(-20, 21, 12).astype(np.float32)
    ires = g.integers(-9, 10, (16, 12)).astype(np.float16)
    exact = np.maximum(ia.astype(np.int64) @ ib.astype(np.int64) + ibias.astype(np.int64), 0) + ires.astype(np.int64)
    assert (oracle.quantized_gemm(ia, ib, ibias, ires, np.full(12, 0.25, np.float32)) ==
            np.clip(exact * 4, -128, 127)).all()                       # division by 1/4 is exact
    halves = oracle.quantized_gemm(np.ones((1, 1), np.float16), np.ones((1, 3), np.float16),
                                   np.array([-10.0, 300.0, 0.0], np.float32), np.array([[-3.0, 0.0, -3.0]], np.float16),
                                   np.array([2.0, 1.0, 2.0], np.float32))
    assert halves.tolist() == [[-1, 127, -1]]   # ReLU(-9) + -3 = -3 -> -1.5 -> -1; 301 saturates; (1 - 3) / 2
    low = oracle.quantized_gemm(np.zeros((1, 1), np.float16), np.zeros((1, 1), np.float16), np.zeros(1, np.float32),
                                np.array([[-1000.0]], np.float16), np.ones(1, np.float32))
    assert low.tolist() == [[-128]]
