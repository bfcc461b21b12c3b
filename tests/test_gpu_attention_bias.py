"""GPU parity of flash_attention_bias_fwd (attention with an additive per-key bias) through
intent.jit.

Bars: f16 outputs within rel 2e-2 / abs 1e-2 of the oracle (oracle.attention_bias_fwd, pinned
against float64 attention); a dominant key returns its value row within 2e-3; -inf biases remove
their keys where no 64-key chunk is removed whole (compared with float64 attention over the
remaining keys); where a chunk's keys are all removed, its weights exp2(-inf - (-inf)) are NaN in
the reference's summarizer, and the kernel's output is NaN exactly where the oracle's is."""
import numpy as np
import pytest
import torch

import intent_amd as intent
import oracle
from intent_amd.examples import inputs
from intent_amd.examples.kernels.streaming.attention import flash_attention_bias_fwd
from tests.gpu_util import announce, assert_16bit

pytestmark = pytest.mark.gpu


def run(device, q, k, v, bias, scale):
    kernel = intent.jit(flash_attention_bias_fwd, backend="hip")
    if not isinstance(bias, torch.Tensor):
        bias = torch.from_numpy(np.ascontiguousarray(bias)).to(device)
    args = [torch.from_numpy(np.ascontiguousarray(a)).to(device) for a in (q, k, v)]
    return kernel.run(*args, bias, scale).cpu().numpy()


def case(seed, batch, heads, sq, sk, d, dv, spread=3.0):
    g = np.random.default_rng(seed)
    q, k = inputs.normal(g, (batch, heads, sq, d), "f16"), inputs.normal(g, (batch, heads, sk, d), "f16")
    v = inputs.normal(g, (batch, heads, sk, dv), "f16")
    bias = (spread * g.standard_normal((batch, heads, sk))).astype(np.float32)
    return q, k, v, bias


@pytest.mark.parametrize("sq,sk,d,dv", [(300, 1000, 128, 128), (256, 64, 64, 64), (77, 65, 64, 128),
                                        (513, 1, 128, 64), (1, 777, 128, 128)])
def test_bias_attention_matches_oracle(device, sq, sk, d, dv):
    """Key counts on and off the 64-key tile (1, 64, 65, 777, 1000), query counts around the
    256-query block."""
    announce("attention bias", sq, sk, d, dv)
    q, k, v, bias = case(sq + sk + d + dv, 2, 3, sq, sk, d, dv)
    scale = float(np.float32(d ** -0.5))
    assert_16bit(run(device, q, k, v, bias, scale), oracle.attention_bias_fwd(q, k, v, bias, scale))


def test_bias_attention_dominant_key_and_broadcast_view(device):
    """A +40 bias on one key returns that key's value row in its (batch, head) only; a bias
    broadcast over heads (head stride 0) and a strided bias view meet the oracle."""
    announce("attention bias dominant key / views")
    q, k, v, bias = case(3, 2, 4, 200, 300, 128, 128, spread=0.0)
    bias[1, 2, 123] = 40.0
    o = run(device, q, k, v, bias, 0.0883883461356163)
    assert np.abs(o[1, 2].astype(np.float64) - v[1, 2, 123].astype(np.float64)[None, :]).max() <= 2e-3
    assert_16bit(o, oracle.attention_bias_fwd(q, k, v, bias, 0.0883883461356163))
    g = np.random.default_rng(4)
    per_batch = torch.from_numpy((2.0 * g.standard_normal((2, 1, 300))).astype(np.float32)).to(device)
    shared = per_batch.expand(2, 4, 300)
    o = run(device, q, k, v, shared, 0.0883883461356163)
    want = oracle.attention_bias_fwd(q, k, v, np.ascontiguousarray(shared.cpu().numpy()), 0.0883883461356163)
    assert_16bit(o, want)
    wide = torch.from_numpy((2.0 * g.standard_normal((2, 4, 307))).astype(np.float32)).to(device)
    view = wide[:, :, 7:]
    o = run(device, q, k, v, view, 0.0883883461356163)
    assert_16bit(o, oracle.attention_bias_fwd(q, k, v, np.ascontiguousarray(view.cpu().numpy()),
                                              0.0883883461356163))


def _float64_masked(q, k, v, bias, scale):
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    logits = q @ k.transpose(0, 1, 3, 2) * scale + bias.astype(np.float64)[:, :, None, :]
    peak = np.max(logits, axis=3, keepdims=True)
    w = np.exp(logits - np.where(np.isfinite(peak), peak, 0.0))
    den = w.sum(axis=3, keepdims=True)
    return np.where(den > 0, (w @ v) / np.where(den > 0, den, 1.0), 0.0)


def test_bias_attention_minus_infinity_masks_keys(device):
    """Every third key at -inf (every chunk keeps keys: those keys drop out), a head whose first 128
    keys are all -inf (two whole chunks: NaN weights, a NaN row, as the summarizer gives) and a head
    with every key at -inf (NaN)."""
    announce("attention bias -inf")
    q, k, v, bias = case(6, 1, 3, 100, 200, 64, 64, spread=1.0)
    bias[0, 0, ::3] = -np.inf
    bias[0, 1, :128] = -np.inf
    bias[0, 2, :] = -np.inf
    o = run(device, q, k, v, bias, 0.125)
    want = oracle.attention_bias_fwd(q, k, v, bias, 0.125)
    assert (np.isnan(o) == np.isnan(want)).all()
    assert np.isnan(o[0, 1]).all() and np.isnan(o[0, 2]).all()
    assert_16bit(o[0, 0], want[0, 0])
    assert_16bit(o[0, 0], _float64_masked(q, k, v, bias, 0.125)[0, 0])


def test_bias_attention_other_head_dims(device):
    """Head widths other than 64 and 128 (zero-padded to the kernel width by the provider)."""
    announce("attention bias d=72 dv=24")
    q, k, v, bias = case(7, 1, 2, 130, 190, 72, 24)
    scale = float(np.float32(72 ** -0.5))
    assert_16bit(run(device, q, k, v, bias, scale), oracle.attention_bias_fwd(q, k, v, bias, scale))
