"""GPU parity of the bf16 GEMM.

Bars: bf16 outputs within rel 2e-2 / abs 1e-2 of the fp32-accumulated reference (the oracle,
and hipBLASLt through torch in float32 on the full 8192^3 config); bit-exact on inputs whose
products and partial sums are exact in f32 (small integers, permutation matrices)."""
import numpy as np
import pytest
import torch

import intent_amd as intent
import oracle
from intent_amd.examples import inputs
from intent_amd.examples.kernels.contraction.gemm import bf16_gemm
from tests.gpu_util import announce, assert_16bit, bf16_tensor_bits, bf16_to_f32, to_bf16_tensor

pytestmark = pytest.mark.gpu


def run(device, a_bits, b_bits):
    c = intent.jit(bf16_gemm, backend="hip").run(to_bf16_tensor(a_bits, device), to_bf16_tensor(b_bits, device))
    return bf16_tensor_bits(c)


def test_gemm_golden(device, golden):
    announce("gemm golden")
    g = golden("gemm")
    c = bf16_to_f32(run(device, g["gemm_a"], g["gemm_b"]))
    assert_16bit(c, g["gemm_c64"])
    assert (run(device, g["gemm_int_a"], g["gemm_int_b"]) == g["gemm_int_c"]).all()


@pytest.mark.parametrize("m,n,k", [(256, 256, 64), (300, 520, 72), (1, 8, 8), (513, 264, 1000), (33, 17, 19),
                                   (64, 24, 4096), (1024, 2048, 512), (7, 3, 0)])
def test_gemm_shapes(device, m, n, k):
    announce("gemm", m, n, k)
    a, b = inputs.gemm_bf16(seed=m + n + k, m=m, n=n, k=k)
    c = run(device, a, b)
    want = oracle.gemm_bf16(a, b)
    assert_16bit(bf16_to_f32(c), bf16_to_f32(want))
    diff = np.abs(c.astype(np.int32) - want.astype(np.int32))
    assert (diff <= 2).mean() > 0.999 if diff.size else True


def test_gemm_exact_cases(device):
    announce("gemm exact")
    rng = np.random.default_rng(11)
    a = inputs._bf16_bits(rng.integers(-8, 9, (512, 768)).astype(np.float32))
    b = inputs._bf16_bits(rng.integers(-8, 9, (768, 256)).astype(np.float32))
    assert (run(device, a, b) == oracle.gemm_bf16(a, b)).all()          # exact integer sums
    perm = rng.permutation(512)
    p = inputs._bf16_bits(np.eye(512, dtype=np.float32)[perm])
    x = inputs.uniform(rng, (512, 264), -1, 1, "bf16")
    assert (run(device, p, x) == x[perm]).all()                          # rows permuted exactly
    perm2 = rng.permutation(264)
    q = inputs._bf16_bits(np.eye(264, dtype=np.float32)[perm2])
    assert (run(device, x, q) == x[:, np.argsort(perm2)]).all()         # columns permuted exactly


def test_gemm_strided_views(device):
    announce("gemm strided")
    a, b = inputs.gemm_bf16(seed=3, m=384, n=640, k=512)
    big_a = torch.zeros(384, 1024, dtype=torch.bfloat16, device=device)
    big_a[:, 256:768] = to_bf16_tensor(a, device)
    ta = big_a[:, 256:768]                                 # row stride 1024
    tb = to_bf16_tensor(np.ascontiguousarray(b.T), device).t()   # inner stride 512: staged copy
    c = intent.jit(bf16_gemm, backend="hip").run(ta, tb)
    assert (bf16_tensor_bits(c) == run(device, a, b)).all()
    out = torch.empty(640, 384, dtype=torch.bfloat16, device=device).t()   # strided output
    intent.jit(bf16_gemm, backend="hip")(ta, to_bf16_tensor(b, device), out)
    assert (bf16_tensor_bits(out.contiguous()) == run(device, a, b)).all()


def test_gemm_config3_full(device):
    announce("gemm config 3 8192^3")
    a, b = inputs.gemm_bf16()
    ta, tb = to_bf16_tensor(a, device), to_bf16_tensor(b, device)
    c = intent.jit(bf16_gemm, backend="hip").run(ta, tb)
    ref = torch.matmul(ta.float(), tb.float())             # fp32-accumulated library reference
    err = (c.float() - ref).abs()
    assert bool((err <= 1e-2 + 2e-2 * ref.abs()).all())
    rows = np.array([0, 1, 255, 256, 1000, 4095, 4096, 5555, 8190, 8191])
    want = oracle.gemm_bf16(np.ascontiguousarray(a[rows]), b)
    got = bf16_tensor_bits(c)[rows]
    assert_16bit(bf16_to_f32(got), bf16_to_f32(want))
    assert (np.abs(got.astype(np.int32) - want.astype(np.int32)) <= 2).mean() > 0.999
