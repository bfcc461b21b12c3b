"""The measurement probe of libintent_hip.so (the box's own MFMA rate, reported by bench.py beside
the published peak) does the work it is credited with."""
import pytest
import torch

from intent_amd.runtime.hip import library as hiplib

pytestmark = pytest.mark.gpu


def _stream():
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("varied", [0, 1])
@pytest.mark.parametrize("dtype", [hiplib.F16, hiplib.BF16])
def test_mfma_probe_writes_one_finite_sum_per_wave(dtype, varied):
    """Every wave runs its rounds and writes its sum: with the same operands in every wave, the
    sums are equal, positive (operands in [0.5, 1)), and grow linearly with the rounds."""
    lib = hiplib.library()
    blocks = 8
    sums = []
    for iterations in (16, 32):
        out = torch.full((blocks * 4,), float("nan"), dtype=torch.float32, device="cuda")
        lib.check(lib.fn["mfma_probe"](dtype, varied, blocks, iterations, out.data_ptr(), _stream()))
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        assert torch.all(out == out[0]) and out[0] > 0
        sums.append(float(out[0]))
    assert sums[1] == pytest.approx(2 * sums[0], rel=1e-5)
