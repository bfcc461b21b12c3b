"""GPU parity of attention over packed sequences: flash_varlen_attention_fwd (one head, CAUSAL)
and flash_varlen_gqa_prefill (grouped heads, causal), through intent.jit.

Bars: f16 outputs within rel 2e-2 / abs 1e-2 of the oracle (oracle.attention_varlen_fwd, the
pinned batched oracle applied to each sequence); packed sequences of equal length equal the
batched kernel's output bit for bit (the same tiles in the same order); rows outside every
sequence keep what the caller's buffer held."""
import numpy as np
import pytest
import torch

import intent_amd as intent
import oracle
from intent_amd.examples import inputs
from intent_amd.examples.kernels.streaming.attention import (flash_gqa_attention_fwd, flash_varlen_attention_fwd,
                                                            flash_varlen_gqa_prefill)
from tests.gpu_util import announce, assert_16bit

pytestmark = pytest.mark.gpu


def t(array, device):
    return torch.from_numpy(np.ascontiguousarray(array)).to(device)


def offsets(lengths):
    return np.concatenate(([0], np.cumsum(lengths))).astype(np.int32)


def run_single(device, q, k, v, lengths, scale, causal, out=None):
    kernel = intent.jit(flash_varlen_attention_fwd, backend="hip", constexprs={"CAUSAL": causal})
    args = (t(q, device), t(k, device), t(v, device), t(np.asarray(lengths, np.int32), device),
            t(offsets(lengths), device))
    if out is None:
        return kernel.run(*args, scale).cpu().numpy()
    kernel(*args, out, scale)
    return out.cpu().numpy()


def run_gqa(device, q, k, v, lengths, scale, group):
    kernel = intent.jit(flash_varlen_gqa_prefill, backend="hip", constexprs={"HEAD_GROUP": group})
    return kernel.run(t(q, device), t(k, device), t(v, device), t(np.asarray(lengths, np.int32), device),
                      t(offsets(lengths), device), scale).cpu().numpy()


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("d,dv", [(128, 128), (64, 64), (64, 128)])
def test_varlen_single_head_matches_oracle(device, causal, d, dv):
    """Lengths around the 64-key tiles and 256-query blocks, with an empty and a one-row sequence."""
    announce("varlen single head", causal, d, dv)
    g = np.random.default_rng(31 + d + dv + causal)
    lengths = [257, 0, 1, 64, 255, 700, 256, 63, 1000]
    total = sum(lengths)
    q, k = inputs.normal(g, (total, d), "f16"), inputs.normal(g, (total, d), "f16")
    v = inputs.normal(g, (total, dv), "f16")
    scale = float(np.float32(1 / np.sqrt(d)))
    o = run_single(device, q, k, v, lengths, scale, causal)
    assert_16bit(o, oracle.attention_varlen_fwd(q, k, v, offsets(lengths), scale, causal))


@pytest.mark.parametrize("group", [1, 4])
def test_varlen_gqa_prefill_matches_oracle(device, group):
    announce("varlen gqa prefill", group)
    g = np.random.default_rng(41 + group)
    lengths = [1500, 3, 300, 0, 777]
    total, hq = sum(lengths), 8
    q = inputs.normal(g, (total, hq, 128), "f16")
    k, v = (inputs.normal(g, (total, hq // group, 128), "f16") for _ in range(2))
    o = run_gqa(device, q, k, v, lengths, 0.08838834764831845, group)
    assert o.shape == (total, hq, 128)
    assert_16bit(o, oracle.attention_varlen_fwd(q, k, v, offsets(lengths), 0.08838834764831845, True,
                                                head_group=group))


def test_varlen_equals_batched_kernel(device, tmp_path):
    """Four sequences of 1024 rows: the packed kernel and the batched kernel give the same bits. The
    batched grid is small enough to split its keys by default; the tuning row [[0]] runs it unsplit,
    as the packed kernel always is."""
    import json

    announce("varlen equals batched")
    g = np.random.default_rng(43)
    batch, seq, hq, group = 4, 1024, 8, 2
    q = inputs.normal(g, (batch, hq, seq, 128), "f16")
    k, v = (inputs.normal(g, (batch, hq // group, seq, 128), "f16") for _ in range(2))
    config = tmp_path / "tuning.json"
    config.write_text(json.dumps({"columns": ["split"], "families": {"hip.attention_forward": [[0]]}}))
    batched = intent.jit(flash_gqa_attention_fwd, backend="hip", constexprs={"HEAD_GROUP": group, "CAUSAL": True},
                         tuning_config=config).run(t(q, device), t(k, device), t(v, device), 0.125).cpu().numpy()
    pack = lambda a: np.ascontiguousarray(a.transpose(0, 2, 1, 3).reshape(batch * seq, a.shape[1], 128))  # noqa
    o = run_gqa(device, pack(q), pack(k), pack(v), [seq] * batch, 0.125, group)
    assert (o.view(np.uint16) == pack(batched).view(np.uint16)).all()


def test_varlen_rows_outside_sequences_keep_their_values(device):
    """Offsets that skip rows (between sequences and at the end): those rows of the caller's output
    buffer are not written."""
    announce("varlen uncovered rows")
    g = np.random.default_rng(47)
    total = 600
    q, k, v = (inputs.normal(g, (total, 64), "f16") for _ in range(3))
    cu = np.array([0, 100, 100, 350], np.int32)            # rows 350..599 belong to no sequence
    out = torch.full((total, 64), 7.0, dtype=torch.float16, device=device)
    kernel = intent.jit(flash_varlen_attention_fwd, backend="hip", constexprs={"CAUSAL": True})
    kernel(t(q, device), t(k, device), t(v, device), t(np.array([100, 0, 250], np.int32), device), t(cu, device),
           out, 0.125)
    o = out.cpu().numpy()
    assert (o[350:] == np.float16(7.0)).all()
    assert_16bit(o[:350], oracle.attention_varlen_fwd(q, k, v, cu, 0.125, True)[:350])


def test_varlen_static_workspace_is_refused(device):
    announce("varlen static workspace")
    q = torch.zeros((4, 64), dtype=torch.float16, device=device)
    kernel = intent.jit(flash_varlen_attention_fwd, backend="hip", constexprs={"CAUSAL": True},
                        backend_options={"workspace": "static"})
    with pytest.raises(Exception, match="workspace"):
        kernel.run(q, q, q, torch.tensor([4], dtype=torch.int32, device=device),
                   torch.tensor([0, 4], dtype=torch.int32, device=device), 0.125)


def test_varlen_other_head_dims(device):
    """Packed sequences with head widths other than 64 and 128 (zero-padded by the provider)."""
    announce("varlen d=48 dv=100")
    rng = np.random.default_rng(48)
    lengths = [70, 1, 300, 129]
    total = sum(lengths)
    q, k = inputs.normal(rng, (total, 4, 48), "f16"), inputs.normal(rng, (total, 2, 48), "f16")
    v = inputs.normal(rng, (total, 2, 100), "f16")
    scale = float(np.float32(48 ** -0.5))
    o = run_gqa(device, q, k, v, lengths, scale, 2)
    assert_16bit(o, oracle.attention_varlen_fwd(q, k, v, offsets(lengths), scale, True, head_group=2))
