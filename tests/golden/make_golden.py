"""Generate the committed golden fixtures (tests/golden/*.npz).

Expected values are computed in float64 from the closed form of each operator
(numpy/scipy only; neither the oracle nor the hip provider is involved), or are
exact by construction (integer-valued GEMM and SpMV probes). Inputs follow the
seeded conventions of intent_amd.examples.inputs. Run from the repository root:
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from intent_amd.examples import inputs  # noqa: E402

OUT = Path(__file__).resolve().parent


def bf16_to_f64(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def softmax64(x):
    x = x.astype(np.float64)
    m = np.max(x, axis=1, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=1, keepdims=True)


def softmax_cases():
    rng = np.random.default_rng(101)
    x32 = inputs.normal(rng, (8, 1000), "f32", 4)
    x32[1] = 0.75                                   # constant row -> exactly 1/N... N=1000 not a power of 2
    x32[2, ::3] = -np.inf                           # -inf entries -> exact zeros
    x32[3] = -60.0
    x32[3, 17] = 60.0                               # one dominant entry: exp(-120) underflows to 0 in f32
    x16 = inputs.normal(rng, (8, 512), "f16", 3)
    xb = inputs.normal(rng, (4, 256), "bf16", 3)
    const_pow2 = np.full((2, 1024), 2.5, np.float32)  # exactly 1/1024 in every precision
    return {
        "softmax_f32_x": x32, "softmax_f32_y": softmax64(x32),
        "softmax_f16_x": x16, "softmax_f16_y": softmax64(x16.astype(np.float64)),
        "softmax_bf16_x": xb, "softmax_bf16_y": softmax64(bf16_to_f64(xb)),
        "softmax_pow2_x": const_pow2, "softmax_pow2_y": softmax64(const_pow2),
    }


def softmax_bwd_cases():
    rng = np.random.default_rng(202)
    p32 = softmax64(inputs.normal(rng, (6, 257), "f32", 2)).astype(np.float32)
    g32 = inputs.normal(rng, (6, 257), "f32")
    p16 = softmax64(inputs.normal(rng, (6, 512), "f32", 2)).astype(np.float16)
    g16 = inputs.normal(rng, (6, 512), "f16")

    def bwd64(p, g):
        p, g = p.astype(np.float64), g.astype(np.float64)
        return p * (g - np.sum(p * g, axis=1, keepdims=True))

    return {"softmax_bwd_f32_p": p32, "softmax_bwd_f32_dy": g32, "softmax_bwd_f32_dx": bwd64(p32, g32),
            "softmax_bwd_f16_p": p16, "softmax_bwd_f16_dy": g16, "softmax_bwd_f16_dx": bwd64(p16, g16)}


def gemm_cases():
    rng = np.random.default_rng(303)
    a = inputs.uniform(rng, (48, 40), -1.0, 1.0, "bf16")
    b = inputs.uniform(rng, (40, 56), -1.0, 1.0, "bf16")
    c64 = bf16_to_f64(a) @ bf16_to_f64(b)
    # Small integers: every partial sum is an exact f32 integer; the only rounding is the
    # final cast, so the bf16 result is exact (round-to-nearest-even of the integer).
    ai = rng.integers(-8, 9, (32, 64)).astype(np.float32)
    bi = rng.integers(-8, 9, (64, 48)).astype(np.float32)
    ci = (ai.astype(np.float64) @ bi.astype(np.float64)).astype(np.float32)
    return {"gemm_a": a, "gemm_b": b, "gemm_c64": c64,
            "gemm_int_a": inputs._bf16_bits(ai), "gemm_int_b": inputs._bf16_bits(bi),
            "gemm_int_c": inputs._bf16_bits(ci)}


def attention64(q, k, v, scale, causal):
    q, k, v = (t.astype(np.float64) for t in (q, k, v))
    s = np.einsum("bhqd,bhkd->bhqk", q, k) * scale
    if causal:
        qi = np.arange(q.shape[2])[:, None]
        ki = np.arange(k.shape[2])[None, :]
        s = np.where(qi >= ki, s, -np.inf)
    m = np.max(s, axis=-1, keepdims=True)
    e = np.exp(s - m)
    return np.einsum("bhqk,bhkd->bhqd", e / e.sum(axis=-1, keepdims=True), v)


def attention_cases():
    rng = np.random.default_rng(404)
    q = inputs.normal(rng, (1, 2, 80, 128), "f16")
    k = inputs.normal(rng, (1, 2, 80, 128), "f16")
    v = inputs.normal(rng, (1, 2, 80, 128), "f16")
    q2 = inputs.normal(rng, (2, 1, 40, 128), "f16")
    k2 = inputs.normal(rng, (2, 1, 100, 128), "f16")
    v2 = inputs.normal(rng, (2, 1, 100, 128), "f16")
    scale = float(np.float32(1 / np.sqrt(128)))
    return {"attn_q": q, "attn_k": k, "attn_v": v, "attn_scale": np.float32(scale),
            "attn_causal_o": attention64(q, k, v, scale, True).astype(np.float32),
            "attn_full_o": attention64(q, k, v, scale, False).astype(np.float32),
            "attn_rect_q": q2, "attn_rect_k": k2, "attn_rect_v": v2,
            "attn_rect_causal_o": attention64(q2, k2, v2, scale, True).astype(np.float32),
            "attn_rect_full_o": attention64(q2, k2, v2, scale, False).astype(np.float32)}


def gemm_family_cases():
    """`gemm` (f16, ACTIVATION), gemm_f32 and linear_f32 (contraction/gemm.py:15-73)."""
    rng = np.random.default_rng(606)
    a16 = inputs.normal(rng, (40, 72), "f16")
    b16 = inputs.normal(rng, (72, 24), "f16")
    c64 = a16.astype(np.float64) @ b16.astype(np.float64)
    ai = rng.integers(-8, 9, (24, 40)).astype(np.float16)     # exact: integer sums < 2^11
    bi = rng.integers(-8, 9, (40, 16)).astype(np.float16)
    ci = ai.astype(np.float64) @ bi.astype(np.float64)
    a32 = inputs.normal(rng, (33, 70), "f32")
    b32 = inputs.normal(rng, (70, 45), "f32")
    prod = np.abs(a32.astype(np.float64)) @ np.abs(b32.astype(np.float64))
    return {"gemm16_a": a16, "gemm16_b": b16, "gemm16_c64": c64,
            "gemm16_relu64": np.where(np.isnan(c64), c64, np.where(c64 > 0, c64, 0.0)),
            "gemm16_int_a": ai, "gemm16_int_b": bi, "gemm16_int_c": ci.astype(np.float16),
            "gemm32_a": a32, "gemm32_b": b32, "gemm32_c64": a32.astype(np.float64) @ b32.astype(np.float64),
            "gemm32_abs64": prod}


def attention_grouped64(q, k, v, scale, causal, group):
    """Grouped heads: query head h attends with key/value head h // group."""
    heads = np.arange(q.shape[1]) // group
    return attention64(q, k[:, heads], v[:, heads], scale, causal)


def attention_family_cases():
    """flash_gqa_attention_fwd (f16) and flash_attention_bf16_fwd (attention.py:469-553)."""
    rng = np.random.default_rng(707)
    q = inputs.normal(rng, (1, 4, 70, 128), "f16")
    k = inputs.normal(rng, (1, 2, 90, 128), "f16")
    v = inputs.normal(rng, (1, 2, 90, 128), "f16")
    qb = inputs.normal(rng, (2, 2, 66, 128), "bf16")
    kb = inputs.normal(rng, (2, 1, 66, 128), "bf16")
    vb = inputs.normal(rng, (2, 1, 66, 128), "bf16")
    scale = float(np.float32(1 / np.sqrt(128)))
    out = {"gqa_q": q, "gqa_k": k, "gqa_v": v, "gqa_scale": np.float32(scale), "gqa_group": np.int64(2),
           "bf16_q": qb, "bf16_k": kb, "bf16_v": vb, "bf16_group": np.int64(2)}
    for causal in (True, False):
        tag = "causal" if causal else "full"
        out[f"gqa_{tag}_o"] = attention_grouped64(q, k, v, scale, causal, 2).astype(np.float32)
        out[f"bf16_{tag}_o"] = attention_grouped64(bf16_to_f64(qb), bf16_to_f64(kb), bf16_to_f64(vb), scale,
                                                   causal, 2).astype(np.float32)
    return out


def spmv_cases():
    rng = np.random.default_rng(505)
    rows = 700
    lengths = inputs.zipf_row_lengths(rows, cap=300, c=900.0)[rng.permutation(rows)]
    lengths[5] = 0                                  # empty rows
    lengths[6] = 0
    offsets, columns = inputs.csr_matrix(rng, lengths, rows)
    values = inputs.uniform(rng, int(offsets[-1]), -1.0, 1.0)
    x = inputs.uniform(rng, rows, -1.0, 1.0)
    products = values.astype(np.float64) * x[columns].astype(np.float64)
    starts = offsets[:-1].astype(np.int64)
    y64 = np.zeros(rows)
    abs_sum = np.zeros(rows)
    nonempty = lengths > 0
    y64[nonempty] = np.add.reduceat(products, starts[nonempty])
    abs_sum[nonempty] = np.add.reduceat(np.abs(products), starts[nonempty])
    # Exact probes: ones -> row lengths; one-hot x -> one column of A.
    onehot = np.zeros(rows, np.float32)
    onehot[123] = 1.0
    column = np.zeros(rows, np.float32)
    hit = columns == 123
    column[np.searchsorted(offsets, np.nonzero(hit)[0], side="right") - 1] = values[hit]
    return {"spmv_offsets": offsets, "spmv_columns": columns, "spmv_values": values, "spmv_x": x,
            "spmv_y64": y64, "spmv_abs": abs_sum, "spmv_lengths": lengths.astype(np.int32),
            "spmv_onehot_x": onehot, "spmv_onehot_y": column}


def main():
    np.savez_compressed(OUT / "softmax.npz", **softmax_cases())
    np.savez_compressed(OUT / "softmax_bwd.npz", **softmax_bwd_cases())
    np.savez_compressed(OUT / "gemm.npz", **gemm_cases())
    np.savez_compressed(OUT / "attention.npz", **attention_cases())
    np.savez_compressed(OUT / "spmv.npz", **spmv_cases())
    np.savez_compressed(OUT / "gemm_family.npz", **gemm_family_cases())
    np.savez_compressed(OUT / "attention_family.npz", **attention_family_cases())
    for path in sorted(OUT.glob("*.npz")):
        print(path.name, path.stat().st_size)


if __name__ == "__main__":
    main()
