"""GPU parity of gemm_i8 (int8 operands, int32 accumulator and bias) through intent.jit.

Bar: bit-exact against the oracle (oracle.gemm_i8: exact int64 sums reduced mod 2^32), for the
MFMA kernel (K a multiple of 64, N of 256, aligned rows; any M) and the general-shape kernel,
including int32 wraparound."""
import numpy as np
import pytest
import torch

import intent_amd as intent
import oracle
from intent_amd.examples.kernels.contraction.gemm import gemm_i8
from tests.gpu_util import announce

pytestmark = pytest.mark.gpu


def run(device, a, b, bias):
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(device)  # noqa: E731
    return intent.jit(gemm_i8, backend="hip").run(t(a), t(b), t(bias)).cpu().numpy()


def test_gemm_i8_reference_example(device):
    """The reference's matrix program (programs/matrix.py:38-43): a (128, 256) and b (256, 192) with
    integers in [-16, 16), bias = arange(192)."""
    announce("gemm_i8 reference example")
    g = np.random.default_rng(3)
    a = g.integers(-16, 16, (128, 256)).astype(np.int8)
    b = g.integers(-16, 16, (256, 192)).astype(np.int8)
    bias = np.arange(192, dtype=np.int32)
    assert (run(device, a, b, bias) == oracle.gemm_i8(a, b, bias)).all()


@pytest.mark.parametrize("m,n,k", [(256, 256, 64), (300, 512, 1024), (1000, 768, 4096), (512, 1024, 2048),
                                   (33, 200, 100), (257, 250, 64), (1, 256, 128), (64, 256, 0)])
def test_gemm_i8_matches_oracle(device, m, n, k):
    """Full int8 range. The first four take the MFMA kernel (a ragged M among them), the others the
    general one (N or K off the tile grid, K = 0 giving the bias)."""
    announce("gemm_i8", m, n, k)
    g = np.random.default_rng(m + n + k)
    a = g.integers(-128, 128, (m, k)).astype(np.int8)
    b = g.integers(-128, 128, (k, n)).astype(np.int8)
    bias = g.integers(-2**31, 2**31, n).astype(np.int32)
    assert (run(device, a, b, bias) == oracle.gemm_i8(a, b, bias)).all()


def test_gemm_i8_wraps_like_int32(device):
    """Sums near the int32 limit: bias 2^31 - 2^20 plus products of up to 16129 over K = 4096
    overflow, and must wrap exactly as the oracle does, on both kernels."""
    announce("gemm_i8 wraparound")
    for n in (256, 200):
        a = np.full((64, 4096), 127, np.int8)
        b = np.full((4096, n), 127, np.int8)
        b[:, 1::2] = -128
        bias = np.full(n, 2**31 - 2**20, np.int32)
        want = oracle.gemm_i8(a, b, bias)
        assert (want[:, 0] < 0).all()                           # the wrap happened
        assert (run(device, a, b, bias) == want).all()


def test_gemm_i8_strided_views(device):
    """Row strides wider than the rows (views into larger arrays) take the general kernel."""
    announce("gemm_i8 strided")
    g = np.random.default_rng(5)
    big_a = torch.from_numpy(g.integers(-128, 128, (512, 1024 + 16)).astype(np.int8)).to(device)
    big_b = torch.from_numpy(g.integers(-128, 128, (1024, 512 + 48)).astype(np.int8)).to(device)
    bias = torch.from_numpy(g.integers(-100, 100, 512).astype(np.int32)).to(device)
    a, b = big_a[:, :1024], big_b[:, :512]
    c = intent.jit(gemm_i8, backend="hip").run(a, b, bias).cpu().numpy()
    assert (c == oracle.gemm_i8(a.cpu().numpy(), b.cpu().numpy(), bias.cpu().numpy())).all()
