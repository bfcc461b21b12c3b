"""GPU parity of quantized_gemm (f16 GEMM, int8 output through bias, ReLU, residual, scale,
saturation and truncation) through intent.jit.

Bar: the kernel's f32 accumulator differs from the exact sum by rounding (at most
K * 2^-24 * sum_k |a b| for any summation order). Where the value before the cast lies farther
than that bound (carried through the epilogue) from an integer, the truncation is decided and the
int8 output equals the oracle's exactly; elsewhere it may differ by one."""
import numpy as np
import pytest
import torch

import intent_amd as intent
import oracle
from intent_amd.examples.kernels.contraction.gemm import quantized_gemm
from tests.gpu_util import announce

pytestmark = pytest.mark.gpu


def run(device, a, b, bias, residual, scale):
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(device)  # noqa: E731
    return intent.jit(quantized_gemm, backend="hip").run(t(a), t(b), t(bias), t(residual), t(scale)).cpu().numpy()


def check(got, a, b, bias, residual, scale):
    want = oracle.quantized_gemm(a, b, bias, residual, scale)
    value = oracle.quantized_gemm(a, b, bias, residual, scale, pre_cast=True).astype(np.float64)
    k = a.shape[1]
    magnitude = np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))
    slack = ((k + 4) * 2.0**-24 * (magnitude + np.abs(bias)[None, :] + np.abs(residual.astype(np.float64)))
             / np.abs(scale.astype(np.float64))[None, :])
    decided = np.abs(value - np.round(value)) > slack + 1e-12
    decided |= (value <= -128) | (value >= 127)                   # saturated on both sides of the bound
    diff = np.abs(got.astype(np.int32) - want.astype(np.int32))
    assert (diff <= 1).all()
    assert (diff[decided] == 0).all()
    assert decided.mean() > 0.2                                   # the worst-case bound still decides many
    assert (diff != 0).mean() < 0.01
    return want


@pytest.mark.parametrize("m,n,k", [(512, 512, 1024), (300, 264, 72), (256, 256, 4096), (33, 50, 7), (64, 24, 0)])
def test_quantized_gemm_matches_oracle(device, m, n, k):
    """MFMA DMA kernel (the first and third), its ragged-edge kernel (the second), the general one."""
    announce("quantized_gemm", m, n, k)
    g = np.random.default_rng(m * 7 + n + k)
    a = g.normal(size=(m, k)).astype(np.float16)
    b = (g.normal(size=(k, n)) / 8).astype(np.float16)
    bias = g.normal(size=n).astype(np.float32)
    residual = (g.normal(size=(m, n)) * 4).astype(np.float16)
    scale = g.uniform(0.02, 0.3, n).astype(np.float32)
    want = check(run(device, a, b, bias, residual, scale), a, b, bias, residual, scale)
    assert (want == 127).any() and (want == -128).any() and (want == 0).any()


def test_quantized_gemm_exact_on_small_integers(device):
    """Small integers with a power-of-two scale: every step is exact, so the output is the oracle's
    bit for bit, on the MFMA kernel."""
    announce("quantized_gemm exact")
    g = np.random.default_rng(29)
    a = g.integers(-3, 4, (256, 512)).astype(np.float16)
    b = g.integers(-3, 4, (512, 256)).astype(np.float16)
    bias = g.integers(-20, 21, 256).astype(np.float32)
    residual = g.integers(-9, 10, (256, 256)).astype(np.float16)
    scale = np.full(256, 0.5, np.float32)
    assert (run(device, a, b, bias, residual, scale) == oracle.quantized_gemm(a, b, bias, residual, scale)).all()
