"""GPU parity of the sibling definitions served by the same kernels: the f16 `gemm` with its
ACTIVATION constexpr, gemm_f32 / linear_f32, flash_gqa_attention_fwd (f16, grouped heads) and
flash_attention_bf16_fwd, all through intent.jit.

Bars:
  * 16-bit outputs within rel 2e-2 / abs 1e-2 of the oracle and of the float64 golden
    fixtures (bf16 attention: rel 4e-2 / abs 2e-2, the bf16 weight and output rounding);
    bit-exact on inputs whose sums are exact (small integers) and where the mathematics fixes
    the result (ReLU of NaN is NaN, of a negative sum +0; the first causal row equals v[0]);
  * f32 GEMM within |got - want| <= 1e-5 * sum_k |a||b| of the float64 product (a backward-error
    bound: the kernel reassociates the k sum), bit-exact on small integers."""
import numpy as np
import pytest
import torch

import intent_amd as intent
import oracle
from intent_amd.examples import inputs
from intent_amd.examples.kernels.contraction.gemm import Activation, gemm, gemm_f32, linear_f32
from intent_amd.examples.kernels.streaming.attention import flash_attention_bf16_fwd, flash_gqa_attention_fwd
from tests.gpu_util import announce, assert_16bit, bf16_tensor_bits, bf16_to_f32, to_bf16_tensor

pytestmark = pytest.mark.gpu


def t(array, device):
    return torch.from_numpy(np.ascontiguousarray(array)).to(device)


# ------------------------------------------------------------------------------ f16 gemm
def run_gemm16(device, a, b, activation):
    return intent.jit(gemm, backend="hip", constexprs={"ACTIVATION": activation}).run(
        t(a, device), t(b, device)).cpu().numpy()


def test_gemm16_golden(device, golden):
    announce("gemm f16 golden")
    g = golden("gemm_family")
    assert_16bit(run_gemm16(device, g["gemm16_a"], g["gemm16_b"], Activation.NONE), g["gemm16_c64"])
    assert_16bit(run_gemm16(device, g["gemm16_a"], g["gemm16_b"], Activation.RELU), g["gemm16_relu64"])
    exact = run_gemm16(device, g["gemm16_int_a"], g["gemm16_int_b"], Activation.NONE)
    assert (exact.view(np.uint16) == g["gemm16_int_c"].view(np.uint16)).all()


@pytest.mark.parametrize("m,n,k", [(256, 256, 64), (300, 520, 72), (513, 264, 1000), (33, 17, 19), (7, 3, 0),
                                   (1024, 768, 512)])
@pytest.mark.parametrize("activation", [Activation.NONE, Activation.RELU])
def test_gemm16_matches_oracle(device, m, n, k, activation):
    announce("gemm f16", m, n, k, activation.name)
    rng = np.random.default_rng(m + n + k)
    a = inputs.normal(rng, (m, k), "f16")
    b = inputs.normal(rng, (k, n), "f16")
    got = run_gemm16(device, a, b, activation)
    want = oracle.gemm16(a, b, relu=activation == Activation.RELU)
    assert_16bit(got, want)
    big = np.abs(want.astype(np.float32)) > 1e-2             # same sign: bit distance = ulp distance
    if big.sum() > 1000:
        ulps = np.abs(got.view(np.int16).astype(np.int32) - want.view(np.int16).astype(np.int32))[big]
        assert (ulps <= 2).mean() > 0.999
    if activation == Activation.RELU:
        assert not np.signbit(got).any()


def test_gemm16_relu_nan_and_zero(device):
    announce("gemm f16 relu specials")
    a = np.zeros((256, 64), np.float16)
    a[0, 0] = np.nan
    a[1, :] = -1.0
    b = np.ones((64, 256), np.float16)
    got = run_gemm16(device, a, b, Activation.RELU)
    assert np.isnan(got[0]).all()                            # maximum(NaN, 0) = NaN
    assert (got[1] == 0).all() and not np.signbit(got[1]).any()
    assert (got[2:] == 0).all() and not np.signbit(got[2:]).any()
    plain = run_gemm16(device, a, b, Activation.NONE)
    assert (plain[1] == -64.0).all()


def test_gemm16_large_vs_torch(device):
    announce("gemm f16 4096x4096x4096")
    rng = np.random.default_rng(5)
    a = t(inputs.uniform(rng, (4096, 4096), -1, 1, "f16"), device)
    b = t(inputs.uniform(rng, (4096, 4096), -1, 1, "f16"), device)
    c = intent.jit(gemm, backend="hip", constexprs={"ACTIVATION": Activation.RELU}).run(a, b)
    ref = torch.relu(torch.matmul(a.float(), b.float()))
    err = (c.float() - ref).abs()
    assert bool((err <= 1e-2 + 2e-2 * ref.abs()).all())


def test_gemm_bf16_relu_through_abi(device):
    """The generic entry point also serves bf16 (bf16_gemm's kernel) with the ReLU epilogue."""
    announce("gemm bf16 relu abi")
    import ctypes

    from intent_amd.runtime.hip.library import ACT_RELU, BF16, library

    rng = np.random.default_rng(6)
    a = inputs.uniform(rng, (256, 128), -1, 1, "bf16")
    b = inputs.uniform(rng, (128, 256), -1, 1, "bf16")
    ta, tb = to_bf16_tensor(a, device), to_bf16_tensor(b, device)
    c = torch.empty(256, 256, dtype=torch.bfloat16, device=device)
    lib = library()
    status = lib.fn["gemm"](BF16, ACT_RELU, ta.data_ptr(), tb.data_ptr(), c.data_ptr(), 256, 256, 128, 128, 256, 256,
                            ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream))
    assert status == 0
    torch.cuda.synchronize(device)
    want = oracle.gemm_bf16(a, b)
    want_f = np.maximum(bf16_to_f32(want), 0.0)
    assert_16bit(bf16_to_f32(bf16_tensor_bits(c)), want_f)
    assert lib.fn["gemm"](BF16, 5, ta.data_ptr(), tb.data_ptr(), c.data_ptr(), 256, 256, 128, 128, 256, 256,
                          None) != 0


# ------------------------------------------------------------------------------ f32 gemm / linear
def f32_bound(a, b):
    return np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))


@pytest.mark.parametrize("m,n,k", [(128, 128, 16), (300, 520, 72), (33, 17, 19), (257, 129, 1000), (5, 3, 0),
                                   (1024, 1024, 1024)])
def test_gemm_f32_and_linear(device, m, n, k):
    announce("gemm f32 / linear", m, n, k)
    rng = np.random.default_rng(m * 3 + n + k)
    a = inputs.normal(rng, (m, k), "f32")
    b = inputs.normal(rng, (k, n), "f32")
    w = np.ascontiguousarray(b.T)
    want64 = a.astype(np.float64) @ b.astype(np.float64)
    bound = 1e-5 * f32_bound(a, b) + 1e-30
    got = intent.jit(gemm_f32, backend="hip").run(t(a, device), t(b, device)).cpu().numpy()
    assert (np.abs(got - want64) <= bound).all()
    lin = intent.jit(linear_f32, backend="hip").run(t(a, device), t(w, device)).cpu().numpy()
    assert (np.abs(lin - want64) <= bound).all()
    want = oracle.gemm_f32(a, b)
    assert (np.abs(got - want) <= 2 * bound).all()


def test_gemm_f32_exact_and_strided(device):
    announce("gemm f32 exact / strided")
    rng = np.random.default_rng(21)
    ai = rng.integers(-8, 9, (200, 96)).astype(np.float32)
    bi = rng.integers(-8, 9, (96, 136)).astype(np.float32)
    exact = (ai.astype(np.float64) @ bi).astype(np.float32)
    assert (intent.jit(gemm_f32, backend="hip").run(t(ai, device), t(bi, device)).cpu().numpy() == exact).all()
    big = torch.zeros(200, 160, device=device)
    big[:, 32:128] = t(ai, device)
    view = big[:, 32:128]                                     # row stride 160
    out = intent.jit(gemm_f32, backend="hip").run(view, t(bi, device)).cpu().numpy()
    assert (out == exact).all()
    w = t(np.ascontiguousarray(bi.T), device)
    assert (intent.jit(linear_f32, backend="hip").run(view, w).cpu().numpy() == exact).all()
    odd = big[:, 33:129]                                      # misaligned rows: the scalar-load variant
    odd.copy_(t(ai, device))                                  # (overwrites the view above)
    assert (intent.jit(gemm_f32, backend="hip").run(odd, t(bi, device)).cpu().numpy() == exact).all()
    assert (intent.jit(linear_f32, backend="hip").run(odd, w).cpu().numpy() == exact).all()


# ------------------------------------------------------------------------------ grouped / bf16 attention
def run_attention(device, defn, q, k, v, scale, group, causal, bf16):
    conv = (lambda a: to_bf16_tensor(a, device)) if bf16 else (lambda a: t(a, device))
    out = intent.jit(defn, backend="hip", constexprs={"HEAD_GROUP": group, "CAUSAL": causal}).run(
        conv(q), conv(k), conv(v), scale)
    return bf16_tensor_bits(out) if bf16 else out.cpu().numpy()


@pytest.mark.parametrize("causal", [True, False])
def test_attention_family_golden(device, golden, causal):
    announce("attention family golden", causal)
    g = golden("attention_family")
    tag = "causal" if causal else "full"
    scale = float(g["gqa_scale"])
    o = run_attention(device, flash_gqa_attention_fwd, g["gqa_q"], g["gqa_k"], g["gqa_v"], scale,
                      int(g["gqa_group"]), causal, False)
    assert_16bit(o, g[f"gqa_{tag}_o"])
    ob = run_attention(device, flash_attention_bf16_fwd, g["bf16_q"], g["bf16_k"], g["bf16_v"], scale,
                       int(g["bf16_group"]), causal, True)
    assert_16bit(bf16_to_f32(ob), g[f"bf16_{tag}_o"], rel=4e-2, abs_=2e-2)


@pytest.mark.parametrize("shape,group,causal", [((1, 8, 300, 2), 4, True), ((2, 6, 513, 3), 2, False),
                                                ((1, 4, 1000, 4), 1, True), ((1, 2, 1, 1), 2, True)])
def test_gqa_matches_oracle(device, shape, group, causal):
    b, hq, s, hk = shape
    announce("gqa", shape, group, causal)
    assert hk * group == hq
    rng = np.random.default_rng(s + hq)
    q = inputs.normal(rng, (b, hq, s, 128), "f16")
    k = inputs.normal(rng, (b, hk, s + 17, 128), "f16")
    v = inputs.normal(rng, (b, hk, s + 17, 128), "f16")
    scale = float(np.float32(1 / np.sqrt(128)))
    o = run_attention(device, flash_gqa_attention_fwd, q, k, v, scale, group, causal, False)
    assert_16bit(o, oracle.attention_fwd(q, k, v, scale, causal, head_group=group))
    assert not np.isnan(o).any()


@pytest.mark.parametrize("shape,group,causal", [((1, 4, 300, 2), 2, True), ((2, 2, 200, 2), 1, False),
                                                ((1, 8, 700, 1), 8, True)])
def test_attention_bf16_matches_oracle(device, shape, group, causal):
    b, hq, s, hk = shape
    announce("attention bf16", shape, group, causal)
    rng = np.random.default_rng(s + hq + 1)
    q = inputs.normal(rng, (b, hq, s, 128), "bf16")
    k = inputs.normal(rng, (b, hk, s, 128), "bf16")
    v = inputs.normal(rng, (b, hk, s, 128), "bf16")
    scale = float(np.float32(1 / np.sqrt(128)))
    o = run_attention(device, flash_attention_bf16_fwd, q, k, v, scale, group, causal, True)
    want = oracle.attention_fwd(q, k, v, scale, causal, head_group=group, storage="bf16")
    assert_16bit(bf16_to_f32(o), bf16_to_f32(want), rel=4e-2, abs_=2e-2)
    if causal:
        heads = np.arange(hq) // group
        assert (o[:, :, 0, :] == v[:, heads, 0, :]).all()   # one valid key: exactly v[0]


def test_reference_streaming_example_attention(device):
    """The reference's streaming example (examples/programs/streaming.py:15-21):
    flash_attention_bf16_fwd with HEAD_GROUP 4, causal, q (2, 8, 256, 64), k and v (2, 2, 256, 64),
    scale 64 ** -0.5."""
    announce("reference streaming example attention")
    rng = np.random.default_rng(21)
    q = inputs.normal(rng, (2, 8, 256, 64), "bf16")
    k = inputs.normal(rng, (2, 2, 256, 64), "bf16")
    v = inputs.normal(rng, (2, 2, 256, 64), "bf16")
    scale = float(np.float32(64 ** -0.5))
    o = run_attention(device, flash_attention_bf16_fwd, q, k, v, scale, 4, True, True)
    want = oracle.attention_fwd(q, k, v, scale, True, head_group=4, storage="bf16")
    assert_16bit(bf16_to_f32(o), bf16_to_f32(want), rel=4e-2, abs_=2e-2)
    assert (o[:, :, 0, :] == v[:, np.arange(8) // 4, 0, :]).all()


@pytest.mark.parametrize("kind,shape,sk,group,causal", [
    ("f16", (1, 4, 1024, 128), 1024, 1, True),      # 16 workgroups: 8 key splits
    ("gqa", (1, 8, 640, 64), 640, 4, True),        # 24 workgroups: 5 splits
    ("bf16", (1, 8, 768, 64), 768, 4, True),       # 24 workgroups: 6 splits
    ("f16", (1, 2, 300, 128), 700, 1, False),      # non-causal, rectangular: 5 splits
])
def test_attention_key_split_matches_oracle(device, tmp_path, kind, shape, sk, group, causal):
    """Grids too small to fill the device split each query block's keys over workgroups (tuning
    family hip.attention_forward, chosen first when eligible) and merge the split states with exp2
    factors, the algebra of merge_attention_summaries (streaming/attention.py:82-114). Checked against
    the oracle, against the unsplit launch the tuning row [[0]] pins (the two differ only in the
    association of that f32 merge), and with workspace='static', which allows no workspace and so
    runs unsplit."""
    import json

    from intent_amd.examples.kernels.streaming.attention import flash_attention_fwd

    b, hq, sq, d = shape
    announce("attention key split", kind, shape, sk, group, causal)
    rng = np.random.default_rng(sq + hq + d)
    storage = "bf16" if kind == "bf16" else "f16"
    q = inputs.normal(rng, (b, hq, sq, d), storage)
    k = inputs.normal(rng, (b, hq // group, sk, d), storage)
    v = inputs.normal(rng, (b, hq // group, sk, d), storage)
    scale = float(np.float32(d ** -0.5))
    defn = {"f16": flash_attention_fwd, "gqa": flash_gqa_attention_fwd, "bf16": flash_attention_bf16_fwd}[kind]
    constexprs = {"CAUSAL": causal} if kind == "f16" else {"HEAD_GROUP": group, "CAUSAL": causal}
    conv = (lambda a: to_bf16_tensor(a, device)) if kind == "bf16" else (lambda a: t(a, device))  # noqa: E731
    args = (conv(q), conv(k), conv(v), scale)
    config = tmp_path / "tuning.json"
    config.write_text(json.dumps({"columns": ["split"], "families": {"hip.attention_forward": [[0]]}}))
    outs = {}
    for label, kwargs in (("split", {}), ("unsplit", {"tuning_config": config}),
                          ("static", {"backend_options": {"workspace": "static"}})):
        call = intent.jit(defn, backend="hip", constexprs=constexprs, **kwargs).prepare(*args)
        call.launch()
        assert dict(call.inspect_configurations()[0].configuration)["split"] == (label == "split"), label
        got = call.result()
        outs[label] = bf16_to_f32(bf16_tensor_bits(got)) if kind == "bf16" else got.cpu().numpy()
    if kind == "bf16":
        want = bf16_to_f32(oracle.attention_fwd(q, k, v, scale, causal, head_group=group, storage="bf16"))
        tol = {"rel": 4e-2, "abs_": 2e-2}
    else:
        want = oracle.attention_fwd(q, k, v, scale, causal, head_group=group)
        tol = {}
    for label, got in outs.items():
        assert not np.isnan(got).any(), label
        assert_16bit(got, want, **tol)
    assert np.array_equal(outs["unsplit"], outs["static"])
    assert_16bit(outs["split"], outs["unsplit"], **tol)
    if causal:
        first = v[:, np.arange(hq) // group, 0, :]
        assert np.array_equal(outs["split"][:, :, 0, :], bf16_to_f32(first) if kind == "bf16" else first)


def test_attention_short_key_range_stays_unsplit(device):
    """The reference streaming example (16 workgroups, 4 key tiles): too few tiles for a split to pay
    for its merge launch, so the unsplit row is the first eligible one."""
    rng = np.random.default_rng(22)
    q = inputs.normal(rng, (2, 8, 256, 64), "bf16")
    k, v = (inputs.normal(rng, (2, 2, 256, 64), "bf16") for _ in range(2))
    call = intent.jit(flash_attention_bf16_fwd, backend="hip", constexprs={"HEAD_GROUP": 4, "CAUSAL": True}).prepare(
        to_bf16_tensor(q, device), to_bf16_tensor(k, device), to_bf16_tensor(v, device), 0.125)
    chosen, *others = call.inspect_configurations()
    assert dict(chosen.configuration)["split"] == 0
    assert [c.eligible for c in others] == [False] and "nothing to split" in others[0].reasons[0]


def test_gqa_head_dim_64_matches_oracle(device):
    announce("gqa d=64")
    rng = np.random.default_rng(64)
    q = inputs.normal(rng, (1, 6, 333, 64), "f16")
    k = inputs.normal(rng, (1, 2, 400, 64), "f16")
    v = inputs.normal(rng, (1, 2, 400, 64), "f16")
    scale = float(np.float32(0.125))
    for causal in (True, False):
        o = run_attention(device, flash_gqa_attention_fwd, q, k, v, scale, 3, causal, False)
        assert_16bit(o, oracle.attention_fwd(q, k, v, scale, causal, head_group=3))


def test_gqa_head_mismatch_is_value_error(device):
    announce("gqa head mismatch")
    q = torch.zeros(1, 6, 8, 128, dtype=torch.float16, device=device)
    k = torch.zeros(1, 4, 8, 128, dtype=torch.float16, device=device)
    with pytest.raises(ValueError):
        intent.jit(flash_gqa_attention_fwd, backend="hip", constexprs={"HEAD_GROUP": 2, "CAUSAL": True}).run(
            q, k, k, 1.0)


@pytest.mark.parametrize("d,dv", [(128, 64), (64, 128)])
@pytest.mark.parametrize("kind,group,causal", [("f16", 1, True), ("f16", 3, False), ("bf16", 2, True),
                                               ("bf16", 1, False)])
def test_attention_value_width_differs_from_key_width(device, d, dv, kind, group, causal):
    """D and DV chosen independently from {64, 128} (flash_attention_fwd, flash_gqa_attention_fwd and
    flash_attention_bf16_fwd declare them as separate symbols): against the oracle, and with DV = 128
    split along the value columns, bit for bit against the DV = 64 kernel on each half (the weights do
    not depend on V)."""
    from intent_amd.examples.kernels.streaming.attention import flash_attention_fwd

    announce("attention d != dv", d, dv, kind, group, causal)
    rng = np.random.default_rng(d * 7 + dv + group)
    hq = 6 if group == 3 else 4
    q = inputs.normal(rng, (2, hq, 300, d), kind)
    k = inputs.normal(rng, (2, hq // group, 333, d), kind)
    v = inputs.normal(rng, (2, hq // group, 333, dv), kind)
    scale = float(np.float32(1 / np.sqrt(d)))
    bf16 = kind == "bf16"
    defn = flash_attention_bf16_fwd if bf16 else flash_gqa_attention_fwd
    o = run_attention(device, defn, q, k, v, scale, group, causal, bf16)
    assert o.shape == (2, hq, 300, dv)
    want = oracle.attention_fwd(q, k, v, scale, causal, head_group=group, storage="bf16" if bf16 else None)
    if bf16:
        assert_16bit(bf16_to_f32(o), bf16_to_f32(want), rel=4e-2, abs_=2e-2)
    else:
        assert_16bit(o, want)
    if group == 1 and not bf16:
        plain = intent.jit(flash_attention_fwd, backend="hip", constexprs={"CAUSAL": causal}).run(
            t(q, device), t(k, device), t(v, device), scale).cpu().numpy()
        assert (plain.view(np.uint16) == o.view(np.uint16)).all()
    if dv == 128:
        for part in (slice(0, 64), slice(64, 128)):
            piece = run_attention(device, defn, q, k, np.ascontiguousarray(v[..., part]), scale, group, causal, bf16)
            assert (piece.view(np.uint16) == o[..., part].view(np.uint16)).all()


@pytest.mark.parametrize("d,dv,bf16", [(96, 96, False), (40, 112, True)])
def test_grouped_attention_other_head_dims(device, d, dv, bf16):
    """flash_gqa_attention_fwd / flash_attention_bf16_fwd with head widths other than 64 and 128
    (zero-padded to the kernel width by the provider)."""
    announce("gqa d/dv", d, dv, bf16)
    rng = np.random.default_rng(d + dv)
    kind = "bf16" if bf16 else "f16"
    q = inputs.normal(rng, (1, 4, 150, d), kind)
    k = inputs.normal(rng, (1, 2, 170, d), kind)
    v = inputs.normal(rng, (1, 2, 170, dv), kind)
    scale = float(np.float32(d ** -0.5))
    definition = flash_attention_bf16_fwd if bf16 else flash_gqa_attention_fwd
    o = run_attention(device, definition, q, k, v, scale, 2, True, bf16)
    want = oracle.attention_fwd(q, k, v, scale, True, head_group=2, storage="bf16" if bf16 else None)
    if bf16:
        assert_16bit(bf16_to_f32(o), bf16_to_f32(want))
    else:
        assert_16bit(o, want)
