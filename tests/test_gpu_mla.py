"""GPU parity of mla_prefill (streaming/attention.py:756-798): causal latent attention whose scores
add a position product qpe . kpe (one kpe row per key, shared by every head) to the content
product, through intent.jit.

Bars: f16 outputs within rel 2e-2 / abs 1e-2 of the oracle (oracle.mla_prefill, pinned against
float64 attention and the attention oracle); with zero position parts the unsplit kernel gives the
grouped attention kernel's bits exactly (the extra score steps add exact zeros). Small grids split
the keys over workgroups and merge their states (a reassociation of the fold): the split result
stays within 2e-3 |want| + 2e-3 of the unsplit one."""
import numpy as np
import pytest
import torch

import intent_amd as intent
import oracle
from intent_amd.examples import inputs
from intent_amd.examples.kernels.streaming.attention import flash_gqa_attention_fwd, mla_prefill
from tests.gpu_util import announce, assert_16bit

pytestmark = pytest.mark.gpu


def t(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def case(seed, batch, heads, kv_heads, sq, sk, d, p):
    g = np.random.default_rng(seed)
    return (inputs.normal(g, (batch, heads, sq, d), "f16"), inputs.normal(g, (batch, heads, sq, p), "f16"),
            inputs.normal(g, (batch, kv_heads, sk, d), "f16"), inputs.normal(g, (batch, 1, sk, p), "f16"),
            inputs.normal(g, (batch, kv_heads, sk, d), "f16"))


def run(device, arrays, scale, group, split=True):
    options = {} if split else {"workspace": "static"}       # no workspace: the unsplit launch
    kernel = intent.jit(mla_prefill, backend="hip", constexprs={"HEAD_GROUP": group}, backend_options=options)
    return kernel.run(*(t(a, device) for a in arrays), scale).cpu().numpy()


@pytest.mark.parametrize("batch,heads,kv_heads,sq,sk,d", [(1, 8, 2, 1024, 1024, 128), (2, 4, 4, 300, 300, 64),
                                                          (1, 4, 1, 100, 700, 128), (2, 2, 1, 600, 200, 64)])
def test_mla_prefill_matches_oracle(device, batch, heads, kv_heads, sq, sk, d):
    """The reference's example extents (B1 H8 HK2 S1024 D128 P64), D 64, a ragged query block, and
    query and key counts that differ (the causal rule on absolute indices)."""
    announce("mla prefill", batch, heads, kv_heads, sq, sk, d)
    arrays = case(sq + sk + d, batch, heads, kv_heads, sq, sk, d, 64)
    scale = float(np.float32((d + 64) ** -0.5))
    got = run(device, arrays, scale, heads // kv_heads)
    want = oracle.mla_prefill(*arrays, scale)
    assert_16bit(got, want)
    unsplit = run(device, arrays, scale, heads // kv_heads, split=False)
    assert_16bit(unsplit, want)
    diff = np.abs(got.astype(np.float64) - unsplit.astype(np.float64))
    assert (diff <= 2e-3 * np.abs(unsplit.astype(np.float64)) + 2e-3).all(), f"split vs unsplit {diff.max()}"


def test_mla_zero_positions_equal_grouped_attention(device):
    announce("mla zero positions")
    q, qpe, k, kpe, v = case(5, 2, 8, 2, 512, 512, 128, 64)
    scale = float(np.float32(192 ** -0.5))
    got = run(device, (q, np.zeros_like(qpe), k, np.zeros_like(kpe), v), scale, 4, split=False)
    gqa = intent.jit(flash_gqa_attention_fwd, backend="hip", constexprs={"HEAD_GROUP": 4, "CAUSAL": True},
                     backend_options={"workspace": "static"})   # unsplit, as the latent launch above
    want = gqa.run(t(q, device), t(k, device), t(v, device), scale).cpu().numpy()
    assert (got.view(np.uint16) == want.view(np.uint16)).all()
