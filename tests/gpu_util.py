"""Comparison helpers of the GPU parity tests (tolerances are stated in each helper)."""
import sys

import numpy as np


def announce(*parts):
    """Name the case on stdout before a GPU step, so a failed run still says what ran."""
    print("[gpu-case]", *parts, flush=True)
    sys.stdout.flush()


def assert_f32_rel(got, want, rel=1e-5, floor=1e-37):
    """fp32 outputs: |got - want| <= rel * |want| (+ a floor below the smallest normal)."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    nan_got, nan_want = np.isnan(got), np.isnan(want)
    assert (nan_got == nan_want).all(), "NaN positions differ"
    ok = ~nan_want
    err = np.abs(got[ok] - want[ok])
    bound = rel * np.abs(want[ok]) + floor
    worst = np.argmax(err - bound) if err.size else 0
    assert (err <= bound).all(), f"max rel err exceeded at {worst}: got {got[ok][worst]} want {want[ok][worst]}"


def assert_16bit(got, want, rel=2e-2, abs_=1e-2):
    """fp16/bf16 outputs: |got - want| <= abs + rel * |want| (the stated 16-bit tolerance)."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert (np.isnan(got) == np.isnan(want)).all(), "NaN positions differ"
    ok = ~np.isnan(want)
    err = np.abs(got[ok] - want[ok])
    assert (err <= abs_ + rel * np.abs(want[ok])).all(), f"max err {err.max()}"


def f16_ulp_distance(a, b):
    """Distance in units of the last place between two float16 arrays (same sign assumed)."""
    ia = np.asarray(a, np.float16).view(np.int16).astype(np.int32)
    ib = np.asarray(b, np.float16).view(np.int16).astype(np.int32)
    ia = np.where(ia < 0, -(ia & 0x7FFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFF), ib)
    return np.abs(ia - ib)


# bf16 conversions live beside the input generators (bench.py and smoke() use them too).
from intent_amd.examples.inputs import bf16_tensor as to_bf16_tensor  # noqa: E402,F401
from intent_amd.examples.inputs import bf16_tensor_bits, bf16_to_f32  # noqa: E402,F401
