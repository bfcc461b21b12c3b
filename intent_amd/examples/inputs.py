"""Seeded synthetic inputs of the benchmark configurations.

Conventions follow the reference's `python/intent/examples/programs/inputs.py:16-105`:
one `np.random.default_rng(seed)` stream per configuration, drawn in the listed order;
`normal(shape, dtype, scale)` draws `standard_normal(float32)`, casts to the storage
dtype, multiplies by float32(scale) in f32 and casts again; `uniform(lo, hi)` draws
float64 uniforms, rounds to float32, then to the storage dtype (round to nearest even).
bf16 has no numpy dtype: bf16 arrays are returned as torch tensors or uint16 bit patterns.
"""
from __future__ import annotations

import numpy as np

SPMV_ROWS = 4_194_304
SPMV_CAP = 65_536
SPMV_C = 3.920855e8


def _bf16_bits(values_f32: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns (NaN kept quiet)."""
    u = np.ascontiguousarray(values_f32, np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)


def bf16_to_f32(bits) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 values (exact)."""
    return (np.asarray(bits).astype(np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_tensor(bits, device):
    """bf16 bit patterns (uint16 array) -> a torch.bfloat16 tensor on `device`."""
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).astype(np.uint16).view(np.int16)).view(torch.bfloat16).to(device)


def bf16_tensor_bits(tensor) -> np.ndarray:
    """A torch.bfloat16 tensor -> its bit patterns as a host uint16 array."""
    import torch

    return tensor.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def normal(rng, shape, dtype: str = "f32", scale=None) -> np.ndarray:
    """float32/float16 array, or uint16 bf16 bits for dtype="bf16"."""
    sample = rng.standard_normal(shape, dtype=np.float32)
    if dtype == "f32":
        out = sample
        if scale is not None:
            out = (out * np.float32(scale)).astype(np.float32)
        return out
    if dtype == "f16":
        out = sample.astype(np.float16)
        if scale is not None:
            out = (out.astype(np.float32) * np.float32(scale)).astype(np.float16)
        return out
    if dtype == "bf16":
        bits = _bf16_bits(sample)
        if scale is not None:
            scaled = (bits.astype(np.uint32) << 16).view(np.float32) * np.float32(scale)
            bits = _bf16_bits(scaled)
        return bits
    raise ValueError(dtype)


def uniform(rng, shape, low: float, high: float, dtype: str = "f32") -> np.ndarray:
    sample = rng.uniform(low, high, shape).astype(np.float32)
    if dtype == "f32":
        return sample
    if dtype == "f16":
        return sample.astype(np.float16)
    if dtype == "bf16":
        return _bf16_bits(sample)
    raise ValueError(dtype)


# ------------------------------------------------------------------------------ configurations
def softmax_f32(seed: int = 0, rows: int = 4096, cols: int = 1024) -> np.ndarray:
    """Config 1: x = normal((4096, 1024), f32, scale=4)."""
    return normal(np.random.default_rng(seed), (rows, cols), "f32", 4)


def softmax_f16_fwd_bwd(seed: int = 0, rows: int = 16384, cols: int = 4096):
    """Config 2: x = normal(f16, scale=3) then dy = normal(f16)."""
    rng = np.random.default_rng(seed)
    x = normal(rng, (rows, cols), "f16", 3)
    dy = normal(rng, (rows, cols), "f16")
    return x, dy


def gemm_bf16(seed: int = 0, m: int = 8192, n: int = 8192, k: int = 8192):
    """Config 3: A = U(-1,1) [m,k] -> bf16, then B = U(-1,1) [k,n] -> bf16 (uint16 bits)."""
    rng = np.random.default_rng(seed)
    a = uniform(rng, (m, k), -1.0, 1.0, "bf16")
    b = uniform(rng, (k, n), -1.0, 1.0, "bf16")
    return a, b


def attention_f16(seed: int = 0, batch: int = 4, heads: int = 32, seq: int = 4096, dim: int = 128):
    """Config 4: q, k, v = normal((B,H,S,D), f16) in that order; scale = float32(1/sqrt(D))."""
    rng = np.random.default_rng(seed)
    q = normal(rng, (batch, heads, seq, dim), "f16")
    k = normal(rng, (batch, heads, seq, dim), "f16")
    v = normal(rng, (batch, heads, seq, dim), "f16")
    return q, k, v, float(np.float32(1.0 / np.sqrt(dim)))


def zipf_row_lengths(rows: int = SPMV_ROWS, cap: int = SPMV_CAP, c: float = SPMV_C) -> np.ndarray:
    """Rank-law Zipf(1.5) lengths L_r = min(cap, max(1, floor(c r^-1.5))), r = 1..rows."""
    ranks = np.arange(1, rows + 1, dtype=np.float64)
    return np.minimum(cap, np.maximum(1, np.floor(c * ranks ** -1.5))).astype(np.int64)


def csr_matrix(rng, lengths: np.ndarray, cols: int):
    """CSR arrays with `lengths[r]` distinct, sorted, uniform column indices per row."""
    rows = lengths.shape[0]
    offsets = np.zeros(rows + 1, np.int64)
    np.cumsum(lengths, out=offsets[1:])
    nnz = int(offsets[-1])
    row_of = np.repeat(np.arange(rows, dtype=np.int64), lengths)
    columns = rng.integers(0, cols, nnz, dtype=np.int64)
    while True:
        keys = row_of * cols + columns
        order = np.argsort(keys, kind="stable")
        keys = keys[order]
        columns = columns[order]
        duplicate = np.zeros(nnz, bool)
        duplicate[1:] = keys[1:] == keys[:-1]
        count = int(duplicate.sum())
        if count == 0:
            break
        columns[duplicate] = rng.integers(0, cols, count, dtype=np.int64)
    return offsets.astype(np.int32), columns.astype(np.int32)


def spmv_f32(seed: int = 0, rows: int = SPMV_ROWS, cap: int = SPMV_CAP, c: float = SPMV_C):
    """Config 5 (recipe A): rank-law row lengths scattered by rng.permutation(rows); per row
    distinct sorted uniform columns (duplicates redrawn); then values = U(-1,1), x = U(-1,1)."""
    rng = np.random.default_rng(seed)
    lengths = zipf_row_lengths(rows, cap, c)[rng.permutation(rows)]
    offsets, columns = csr_matrix(rng, lengths, rows)
    values = uniform(rng, offsets[-1], -1.0, 1.0)
    x = uniform(rng, rows, -1.0, 1.0)
    return offsets, columns, values, x


def csr_spmm(seed: int = 0, rows: int = 8192, cols: int = 8192, per_row: int = 32, features: int = 128):
    """Inputs of csr_spmm at the sparse/csr_spmm.py:5-9 constants by default: `per_row` distinct,
    sorted, uniform columns in every row; values = U(-1,1); dense = U(-1,1) [cols, features]."""
    rng = np.random.default_rng(seed)
    offsets, columns = csr_matrix(rng, np.full(rows, per_row, np.int64), cols)
    values = uniform(rng, offsets[-1], -1.0, 1.0)
    dense = uniform(rng, (cols, features), -1.0, 1.0)
    return offsets, columns, values, dense


def paged_decode(seed: int = 0, batch: int = 8, query_heads: int = 32, kv_heads: int = 8, dim: int = 128,
                 page_size: int = 64, lengths=(8191, 7937, 7683, 7429, 7175, 6921, 6667, 6413), splits: int = 16,
                 shuffle: bool = True, layout: str = "padded"):
    """Inputs of paged_gqa_decode_partials (streaming/paged_attention.py:13-22 constants by default),
    with physical pages in a permuted order when `shuffle`.

    layout "padded": every sequence gets ceil(max length / page_size) pages rounded up to a multiple
    of `splits`, and split j covers an equal run of them (trailing splits of a short sequence hold
    only inactive tokens). layout "exact": sequence b owns ceil(length_b / page_size) pages and its
    splits cover near-equal runs floor(j n / splits) .. floor((j + 1) n / splits).
    Returns (q, key_cache, value_cache, page_offsets, page_indices, lengths, split_offsets)."""
    rng = np.random.default_rng(seed)
    lengths = np.asarray(lengths, np.int32)[:batch]
    if layout == "padded":
        per_sequence = -(-int(lengths.max()) // page_size)
        per_sequence = -(-per_sequence // splits) * splits
        counts = np.full(batch, per_sequence, np.int64)
    elif layout == "exact":
        counts = -(-lengths.astype(np.int64) // page_size)
    else:
        raise ValueError(f"unknown layout {layout!r}")
    page_offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    pages = max(int(page_offsets[-1]), 1)
    q = normal(rng, (batch, query_heads, dim), "f16")
    key_cache = normal(rng, (pages, page_size, kv_heads, dim), "f16")
    value_cache = normal(rng, (pages, page_size, kv_heads, dim), "f16")
    page_indices = (rng.permutation(pages) if shuffle else np.arange(pages)).astype(np.int32)
    split_offsets = np.concatenate([[0]] + [page_offsets[b] + (np.arange(1, splits + 1) * counts[b]) // splits
                                            for b in range(batch)]).astype(np.int32)
    return q, key_cache, value_cache, page_offsets, page_indices, lengths, split_offsets
