"""GPU parity of split-K paged decode: paged_gqa_decode_partials, splitk_attention_f32_to_f16_reduce
and the PagedDecode program that chains them (the reference's programs/composition.py:95-122,
driven as programs/streaming.py:24-41 does), against the C oracle on the same inputs.

Bars: the partials use the same 64-token chunks and the same f16 rounding of P as the oracle and
differ only in summation order and the exp2 instruction, so partial_output is held to
|err| <= 2e-3 |want| + 2e-4 max|want| and partial_lse (base 2) to 1e-4 + 1e-5 |want|, with -inf
(empty job) positions equal; the merged f16 output to 2e-3 |want| + 2e-3 (a few f16 ulp)."""
import numpy as np
import pytest
import torch

import intent_amd as intent
import oracle
from intent_amd.examples import inputs
from intent_amd.examples.kernels.streaming.paged_attention import paged_gqa_decode_partials
from intent_amd.examples.kernels.streaming.splitk_reduce import splitk_attention_f32_to_f16_reduce
from intent_amd.examples.programs.composition import PagedDecode
from tests.gpu_util import announce

pytestmark = pytest.mark.gpu


def jit(defn, **kw):
    return intent.jit(defn, backend="hip", **kw)


def t(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def check_partials(lse, out, want_lse, want_out):
    lse, out = np.asarray(lse, np.float64), np.asarray(out, np.float64)
    want_lse, want_out = np.asarray(want_lse, np.float64), np.asarray(want_out, np.float64)
    empty = np.isneginf(want_lse)
    assert (np.isneginf(lse) == empty).all(), "empty-job positions differ"
    assert not np.isnan(lse).any() and not np.isnan(out).any()
    err = np.abs(lse[~empty] - want_lse[~empty])
    assert (err <= 1e-4 + 1e-5 * np.abs(want_lse[~empty])).all(), f"lse max err {err.max() if err.size else 0}"
    assert (out[empty] == 0).all()
    bound = 2e-3 * np.abs(want_out) + 2e-4 * max(np.abs(want_out).max(), 1e-6)
    worst = np.unravel_index(np.argmax(np.abs(out - want_out) - bound), out.shape)
    assert (np.abs(out - want_out) <= bound).all(), f"at {worst}: got {out[worst]} want {want_out[worst]}"


def check_output(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert (np.isnan(got) == np.isnan(want)).all(), "NaN positions differ"
    ok = ~np.isnan(want)
    err = np.abs(got[ok] - want[ok])
    assert (err <= 2e-3 * np.abs(want[ok]) + 2e-3).all(), f"max err {err.max() if err.size else 0}"


def ragged_case(seed, batch, query_heads, kv_heads, dim, ps, lengths, splits, pages_per_sequence):
    """Page tables with uneven (and empty) splits and a shuffled physical order."""
    rng = np.random.default_rng(seed)
    pages = batch * pages_per_sequence
    q = inputs.normal(rng, (batch, query_heads, dim), "f16")
    key_cache = inputs.normal(rng, (pages, ps, kv_heads, dim), "f16")
    value_cache = inputs.normal(rng, (pages, ps, kv_heads, dim), "f16")
    page_indices = rng.permutation(pages).astype(np.int32)
    page_offsets = np.arange(0, pages + 1, pages_per_sequence, dtype=np.int32)
    split_offsets = [0]
    for b in range(batch):
        cuts = np.sort(rng.integers(0, pages_per_sequence + 1, splits - 1))
        split_offsets += list(b * pages_per_sequence + cuts) + [(b + 1) * pages_per_sequence]
    return (q, key_cache, value_cache, page_offsets, page_indices, np.asarray(lengths, np.int32),
            np.asarray(split_offsets, np.int32))


CASES = {
    # the reference's own example program (programs/streaming.py:24-41): B2 HQ8 HK2 D64, 512 tokens,
    # 16-token pages in order, 8 splits
    "reference_example": dict(kind="uniform", batch=2, query_heads=8, kv_heads=2, dim=64, page_size=16,
                              lengths=(512, 512), splits=8, shuffle=False),
    # the BASELINE decode shape (paged_attention.py constants): B8 HQ32 HK8 D128, 64-token pages, 16 splits
    "baseline": dict(kind="uniform", batch=8, query_heads=32, kv_heads=8, dim=128, page_size=64,
                     lengths=(8191, 7937, 7683, 7429, 7175, 6921, 6667, 6413), splits=16, shuffle=True,
                     layout="exact"),
    "baseline_padded": dict(kind="uniform", batch=8, query_heads=32, kv_heads=8, dim=128, page_size=64,
                            lengths=(8191, 7937, 7683, 7429, 7175, 6921, 6667, 6413), splits=16, shuffle=True),
    "group1_d128": dict(kind="uniform", batch=2, query_heads=3, kv_heads=3, dim=128, page_size=32,
                        lengths=(1000, 77), splits=4, shuffle=True),
    "group16_d64": dict(kind="uniform", batch=1, query_heads=32, kv_heads=2, dim=64, page_size=16,
                        lengths=(700,), splits=2, shuffle=True),
    "group8_d128": dict(kind="uniform", batch=2, query_heads=16, kv_heads=2, dim=128, page_size=64,
                        lengths=(3000, 129), splits=4, shuffle=True),
    # groups of up to 4 score with coalesced K loads folded across lanes: a group of 2 at D 64 with
    # one-token and page-boundary lengths, and one split holding a whole sequence at D 128
    "group2_d64_short": dict(kind="uniform", batch=3, query_heads=4, kv_heads=2, dim=64, page_size=32,
                             lengths=(513, 64, 1), splits=3, shuffle=True),
    "group4_d128_one_split": dict(kind="uniform", batch=1, query_heads=8, kv_heads=2, dim=128, page_size=64,
                                  lengths=(4097,), splits=1, shuffle=True),
    "ragged_empty": dict(kind="ragged", batch=3, query_heads=6, kv_heads=2, dim=64, ps=16,
                         lengths=(0, 37, 300), splits=4, pages_per_sequence=20, page_size=16),
    "logical_page_larger": dict(kind="ragged", batch=2, query_heads=4, kv_heads=1, dim=128, ps=16,
                                lengths=(333, 90), splits=3, pages_per_sequence=24, page_size=20),
}


def make(name):
    spec = dict(CASES[name])
    kind = spec.pop("kind")
    page_size = spec["page_size"]
    if kind == "uniform":
        arrays = inputs.paged_decode(seed=len(name), **spec)
    else:
        spec.pop("page_size")
        arrays = ragged_case(len(name), **spec)
    head_group = spec["query_heads"] // spec["kv_heads"]
    return arrays, page_size, head_group, spec["splits"], float(np.float32(1 / np.sqrt(spec["dim"])))


@pytest.mark.parametrize("name", list(CASES))
def test_paged_decode_partials_match_oracle(device, name):
    announce("paged decode partials", name)
    arrays, page_size, group, splits, scale = make(name)
    kernel = jit(paged_gqa_decode_partials, constexprs={"PAGE_SIZE": page_size, "HEAD_GROUP": group,
                                                        "SPLITS": splits})
    lse, out = kernel.run(*(t(a, device) for a in arrays), scale)
    want_lse, want_out = oracle.paged_decode_partials(*arrays, scale, page_size=page_size, head_group=group,
                                                      splits=splits)
    check_partials(lse.cpu().numpy(), out.cpu().numpy(), want_lse, want_out)


@pytest.mark.parametrize("shape", [(8, 32, 16, 128), (2, 3, 1, 64), (1, 5, 7, 200), (3, 2, 40, 96)])
def test_splitk_reduce_matches_oracle(device, shape):
    announce("splitk reduce", shape)
    rng = np.random.default_rng(sum(shape))
    partial = rng.standard_normal(shape).astype(np.float32)
    lse = (rng.standard_normal(shape[:3]) * 4 + 10).astype(np.float32)
    if shape[2] > 1:
        lse[..., 0] = -np.inf                    # an empty split in every row
    out = jit(splitk_attention_f32_to_f16_reduce).run(t(partial, device), t(lse, device))
    check_output(out.cpu().numpy().astype(np.float32), oracle.splitk_reduce_f32_to_f16(partial, lse))


def test_splitk_reduce_strided_lse_and_all_empty_row(device):
    """lse read through its own strides (a transposed view); a row whose splits are all empty gives
    NaN, as the definition's exp(-inf - -inf) does."""
    announce("splitk reduce strided")
    rng = np.random.default_rng(5)
    partial = rng.standard_normal((2, 4, 6, 64)).astype(np.float32)
    lse_t = rng.standard_normal((2, 6, 4)).astype(np.float32)
    lse_t[1, :, 2] = -np.inf
    lse_view = t(lse_t, device).transpose(1, 2)
    out = jit(splitk_attention_f32_to_f16_reduce).run(t(partial, device), lse_view)
    want = oracle.splitk_reduce_f32_to_f16(partial, np.ascontiguousarray(lse_t.transpose(0, 2, 1)))
    got = out.cpu().numpy().astype(np.float32)
    assert np.isnan(got[1, 2]).all() and np.isnan(want[1, 2]).all()
    check_output(got, want)


@pytest.mark.parametrize("name", ["reference_example", "baseline", "ragged_empty"])
def test_paged_decode_program_run_into_prepare(device, name):
    announce("PagedDecode program", name)
    arrays, page_size, group, splits, scale = make(name)
    program = PagedDecode.from_jit(jit, page_size=page_size, head_group=group, splits=splits)
    args = [t(a, device) for a in arrays]
    want_lse, want_out = oracle.paged_decode_partials(*arrays, scale, page_size=page_size, head_group=group,
                                                      splits=splits)
    want = oracle.splitk_reduce_f32_to_f16(want_out, want_lse).astype(np.float32)

    got = program.run(*args, scale)
    check_output(got.cpu().numpy().astype(np.float32), want)

    batch, heads, dim = arrays[0].shape
    partial_lse = torch.empty((batch, heads, splits), dtype=torch.float32, device=device)
    partial_output = torch.empty((batch, heads, splits, dim), dtype=torch.float32, device=device)
    output = torch.empty((batch, heads, dim), dtype=torch.float16, device=device)
    assert program.into(*args, partial_lse, partial_output, output, scale) is output
    check_output(output.cpu().numpy().astype(np.float32), want)
    check_partials(partial_lse.cpu().numpy(), partial_output.cpu().numpy(), want_lse, want_out)

    sequence = program.prepare(*args, scale)
    assert sequence.kernel_count == 2
    sequence.launch()
    first = sequence.result().clone()
    sequence.launch()
    torch.cuda.synchronize()
    check_output(sequence.result().cpu().numpy().astype(np.float32), want)
    assert torch.allclose(first, sequence.result(), rtol=0, atol=0, equal_nan=True)   # replays agree bitwise
    kernels = [o.kernel for o in sequence.observations]
    assert kernels[0].startswith("paged_decode_partials") and kernels[1] == "splitk_reduce_f32_to_f16"


def test_paged_decode_errors_before_launch(device):
    arrays, page_size, group, splits, scale = make("group1_d128")
    args = [t(a, device) for a in arrays]
    with pytest.raises(ValueError, match="HEAD_GROUP"):
        jit(paged_gqa_decode_partials, constexprs={"PAGE_SIZE": page_size, "HEAD_GROUP": 2,
                                                   "SPLITS": splits}).run(*args, scale)
    good = jit(paged_gqa_decode_partials, constexprs={"PAGE_SIZE": page_size, "HEAD_GROUP": group,
                                                      "SPLITS": splits})
    bad_pages = list(args)
    bad_pages[3] = args[3][:-1]
    with pytest.raises(ValueError, match="page_offsets"):
        good.run(*bad_pages, scale)
    bad_splits = list(args)
    bad_splits[6] = torch.cat([args[6], args[6][-1:]])
    with pytest.raises(ValueError, match="split_offsets"):
        good.run(*bad_splits, scale)
    with pytest.raises(Exception, match="HEAD_GROUP|provider_configuration"):
        jit(paged_gqa_decode_partials, constexprs={"PAGE_SIZE": page_size, "HEAD_GROUP": 17,
                                                   "SPLITS": splits}).run(*args, scale)
