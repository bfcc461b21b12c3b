"""GPU parity of the decode definitions of streaming/attention.py:556-754 against the C oracle:
grouped_flash_decode_partials (dense bf16 caches, per-part partials), continuous_gqa_decode
(token-major f16 caches with a validity mask) and varlen_gqa_decode_with_sink_logits (packed
sequences, per-head sink, block logits).

Bars: kernel and oracle fold the same 64-key chunks (parts, splits and blocks start on chunk
boundaries) and round the weights the same way, so they differ only in summation order and the
exp2/reciprocal instructions. Outputs in f16 are held to 2e-3 |want| + 2e-3; bf16 partials to
8e-3 |want| + 2e-4 max|want| (two bf16 ulp); base-2 log-sums to 1e-4 + 1e-5 |want| with the empty
(-inf) positions equal; block logits to 1e-3 |want| + 1e-6."""
import numpy as np
import pytest
import torch

import intent_amd as intent
import oracle
from intent_amd.examples import inputs
from intent_amd.examples.kernels.streaming.attention import (continuous_gqa_decode, grouped_flash_decode_partials,
                                                            varlen_gqa_decode_with_sink_logits)
from tests.gpu_util import announce

pytestmark = pytest.mark.gpu


def t(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def check_output(got, want, rel=2e-3, floor=2e-3):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert not np.isnan(got).any()
    err = np.abs(got - want)
    assert (err <= rel * np.abs(want) + floor).all(), f"max err {err.max()}"


def check_lse(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    empty = np.isneginf(want)
    assert (np.isneginf(got) == empty).all(), "empty positions differ"
    err = np.abs(got[~empty] - want[~empty])
    assert (err <= 1e-4 + 1e-5 * np.abs(want[~empty])).all(), f"lse max err {err.max() if err.size else 0}"


def bf16(g, shape):
    return inputs._bf16_bits(g.standard_normal(shape).astype(np.float32))


def bits_tensor(bits, device):
    return torch.from_numpy(np.ascontiguousarray(bits)).view(torch.bfloat16).to(device)


@pytest.mark.parametrize("keys,d,group,parts,split", [(1000, 128, 4, 4, 256), (1000, 128, 4, 5, 300),
                                                     (257, 64, 1, 3, 100), (4096, 64, 16, 2, 2048),
                                                     (65, 128, 8, 1, 4096)])
def test_grouped_decode_partials_match_oracle(device, keys, d, group, parts, split):
    """Parts that end inside the cache, parts past its end (empty) and one part over every key."""
    announce("grouped decode partials", keys, d, group, parts, split)
    g = np.random.default_rng(keys + d + group)
    batch, kv_heads = 2, 2
    q, k, v = bf16(g, (batch, kv_heads * group, 1, d)), bf16(g, (batch, kv_heads, keys, d)), bf16(g, (batch, kv_heads, keys, d))
    scale = float(np.float32(d ** -0.5))
    kernel = intent.jit(grouped_flash_decode_partials, backend="hip",
                        constexprs={"HEAD_GROUP": group, "P": parts, "SPLIT_SIZE": split})
    lse, out = kernel.run(bits_tensor(q, device), bits_tensor(k, device), bits_tensor(v, device), scale)
    want_lse, want_out = oracle.grouped_decode_partials(q, k, v, scale, parts=parts, split_size=split)
    check_lse(lse.cpu().numpy(), want_lse)
    got = out.float().cpu().numpy().astype(np.float64)
    want = oracle.bf16_bits_to_float(want_out).astype(np.float64)
    empty = np.isneginf(want_lse)
    assert (got[empty] == 0).all()
    bound = 8e-3 * np.abs(want) + 2e-4 * max(np.abs(want).max(), 1e-6)
    assert (np.abs(got - want) <= bound).all(), f"max err {np.abs(got - want).max()}"


@pytest.mark.parametrize("keys,d,group,density", [(2000, 128, 4, 0.5), (8192, 128, 4, 1.0), (65, 64, 8, 0.3),
                                                  (1, 64, 1, 1.0), (3000, 64, 16, 0.05)])
def test_continuous_decode_matches_oracle(device, keys, d, group, density):
    """Masks from dense to sparse; one (batch, key head) masked out entirely gives zeros."""
    announce("continuous decode", keys, d, group, density)
    g = np.random.default_rng(keys + d + group)
    batch, kv_heads = 3, 4
    q = inputs.normal(g, (batch, kv_heads * group, d), "f16")
    k, v = inputs.normal(g, (batch, keys, kv_heads, d), "f16"), inputs.normal(g, (batch, keys, kv_heads, d), "f16")
    mask = (g.random((batch, keys, kv_heads)) < density).astype(np.uint8)
    mask[2, :, 1] = 0
    scale = float(np.float32(d ** -0.5))
    kernel = intent.jit(continuous_gqa_decode, backend="hip", constexprs={"HEAD_GROUP": group})
    out = kernel.run(t(q, device), t(k, device), t(v, device), t(mask, device), scale).cpu().numpy()
    want = oracle.continuous_gqa_decode(q, k, v, mask, scale)
    check_output(out, want)
    assert (out[2, group:2 * group] == 0).all()


@pytest.mark.parametrize("max_blocks", [64, 8])
def test_varlen_decode_sink_matches_oracle(device, max_blocks):
    """The reference's example heads (32 over 8, D 64), sequences of 0, 1, 63, 64, 65, 1000, 4096 and
    5000 keys (the last past 64 blocks); with MAX_BLOCKS 8 the block_logits columns from 8 on keep
    what the caller's buffer held."""
    announce("varlen decode sink", max_blocks)
    g = np.random.default_rng(29 + max_blocks)
    lengths = np.array([0, 1, 63, 64, 65, 1000, 4096, 5000])
    cu = np.concatenate(([0], np.cumsum(lengths))).astype(np.int32)
    batch, q_heads, kv_heads, d, rows = len(lengths), 32, 8, 64, int(cu[-1])
    q = inputs.normal(g, (batch, q_heads, d), "f16")
    k, v = inputs.normal(g, (rows, kv_heads, d), "f16"), inputs.normal(g, (rows, kv_heads, d), "f16")
    sink = g.uniform(0.0, 4.0, q_heads).astype(np.float32)
    scale = 0.125
    kernel = intent.jit(varlen_gqa_decode_with_sink_logits, backend="hip",
                        constexprs={"HEAD_GROUP": 4, "MAX_BLOCKS": max_blocks})
    out = torch.empty((batch, q_heads, d), dtype=torch.float16, device=device)
    logits = torch.full((batch, q_heads, 64), 7.0, dtype=torch.float32, device=device)
    kernel(t(q, device), t(k, device), t(v, device), t(cu, device), t(sink, device), out, logits, scale)
    want_out, want_logits = oracle.varlen_decode_sink(q, k, v, cu, sink, scale, max_blocks=max_blocks)
    check_output(out.cpu().numpy(), want_out)
    got = logits.cpu().numpy()
    err = np.abs(got[:, :, :max_blocks] - want_logits)
    assert (err <= 1e-3 * np.abs(want_logits) + 1e-6).all(), f"block logits max err {err.max()}"
    assert (got[:, :, max_blocks:] == 7.0).all()


def test_decode_variants_refuse_bad_requests(device):
    """Plans raise before any launch: MAX_BLOCKS past the block_logits columns, partials shaped for
    another P, and workspace='static' for the two definitions that merge split states."""
    from intent_amd.diagnostics import CompilationStageError

    announce("decode variants: refusals")
    g = np.random.default_rng(3)
    q, k, v = (inputs.normal(g, shape, "f16") for shape in ((2, 8, 64), (100, 2, 64), (100, 2, 64)))
    cu = np.array([0, 40, 100], np.int32)
    sink = np.zeros(8, np.float32)
    kernel = intent.jit(varlen_gqa_decode_with_sink_logits, backend="hip", constexprs={"HEAD_GROUP": 4, "MAX_BLOCKS": 65})
    out = torch.empty((2, 8, 64), dtype=torch.float16, device=device)
    logits = torch.empty((2, 8, 64), dtype=torch.float32, device=device)
    with pytest.raises(ValueError, match="MAX_BLOCKS"):
        kernel(t(q, device), t(k, device), t(v, device), t(cu, device), t(sink, device), out, logits, 0.125)
    static = intent.jit(varlen_gqa_decode_with_sink_logits, backend="hip", backend_options={"workspace": "static"},
                        constexprs={"HEAD_GROUP": 4, "MAX_BLOCKS": 8})
    with pytest.raises(CompilationStageError):
        static(t(q, device), t(k, device), t(v, device), t(cu, device), t(sink, device), out, logits, 0.125)
    kc, vc = inputs.normal(g, (2, 100, 2, 64), "f16"), inputs.normal(g, (2, 100, 2, 64), "f16")
    mask = np.ones((2, 100, 2), np.uint8)
    static = intent.jit(continuous_gqa_decode, backend="hip", backend_options={"workspace": "static"},
                        constexprs={"HEAD_GROUP": 4})
    with pytest.raises(CompilationStageError):
        static.run(t(q, device), t(kc, device), t(vc, device), t(mask, device), 0.125)
    qb, kb = bits_tensor(bf16(g, (2, 8, 1, 64)), device), bits_tensor(bf16(g, (2, 2, 100, 64)), device)
    grouped = intent.jit(grouped_flash_decode_partials, backend="hip",
                         constexprs={"HEAD_GROUP": 4, "P": 4, "SPLIT_SIZE": 32})
    lse = torch.empty((2, 8, 5), dtype=torch.float32, device=device)
    part = torch.empty((2, 8, 5, 64), dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="partial_lse"):   # the interface binds P to the constexpr
        grouped(qb, kb, kb, lse, part, 0.125)
