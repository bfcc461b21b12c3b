"""ctypes wrapper of liboracle.so (built from intent_oracle.c by the Makefile here).

TEST INFRASTRUCTURE ONLY (see the package docstring)."""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "liboracle.so"
F32, F16, BF16 = 0, 1, 2
_DTYPE_CODES = {np.dtype(np.float32): F32}

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIBRARY


def lib():
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        handle = ctypes.CDLL(str(LIBRARY))
        p, i64, i, f = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        handle.oracle_softmax_fwd.argtypes = [i, p, p, i64, i64, i64, i64, i]
        handle.oracle_softmax_bwd.argtypes = [i, p, p, p, i64, i64, i64, i64, i64, i]
        handle.oracle_gemm_bf16.argtypes = [p, p, p, i64, i64, i64, i64, i64, i64, i]
        handle.oracle_gemm16.argtypes = [i, i, p, p, p, i64, i64, i64, i64, i64, i64, i]
        handle.oracle_gemm_f32.argtypes = [p, p, p, i64, i64, i64, i64, i64, i64, i, i]
        handle.oracle_attention_fwd.argtypes = [i, p, p, p, p, i64, i64, i64, i64, i64, i64, i64,
                                                ctypes.POINTER(i64), f, i, i64, i]
        handle.oracle_attention_fwd_f16.argtypes = [p, p, p, p, i64, i64, i64, i64, i64, i64,
                                                    ctypes.POINTER(i64), f, i, i64, i]
        handle.oracle_attention_bias_fwd.argtypes = [p, p, p, p, p, i64, i64, i64, i64, i64, i64,
                                                     ctypes.POINTER(i64), ctypes.POINTER(i64), f, i64, i]
        handle.oracle_mla_prefill.argtypes = [p, p, p, p, p, p, i64, i64, i64, i64, i64, i64, i64, f, i64, i]
        handle.oracle_csr_spmv_f32.argtypes = [p, p, p, p, p, i64, i]
        handle.oracle_csr_spmm_f32.argtypes = [p, p, p, p, p, i64, i64, i64, i64, i]
        handle.oracle_paged_decode_partials.argtypes = [p, p, p, p, p, p, p, p, p, i64, i64, i64, i64, i64, i64,
                                                        i64, i64, i64, f, i64, i]
        handle.oracle_splitk_reduce_f32_to_f16.argtypes = [p, p, p, i64, i64, i64, i64, i]
        handle.oracle_grouped_decode_partials.argtypes = [p, p, p, p, p, i64, i64, i64, i64, i64, i64, i64, i64, f,
                                                          i64, i]
        handle.oracle_continuous_gqa_decode.argtypes = [p, p, p, p, p, i64, i64, i64, i64, i64, i64, f, i64, i]
        handle.oracle_varlen_decode_sink.argtypes = [p, p, p, p, p, p, p, i64, i64, i64, i64, i64, i64, f, i]
        handle.oracle_attention_bwd_delta.argtypes = [p, p, p, i64, i64, i64, i64, ctypes.POINTER(i64), i]
        handle.oracle_attention_bwd_dq.argtypes = [p, p, p, p, p, p, p, i64, i64, i64, i64, i64, i64,
                                                   ctypes.POINTER(i64), f, i, i64, i]
        handle.oracle_attention_bwd_dkdv.argtypes = [p, p, p, p, p, p, p, p, i64, i64, i64, i64, i64, i64,
                                                     ctypes.POINTER(i64), f, i, i64, i]
        for name in ("oracle_halves_to_floats", "oracle_floats_to_halves", "oracle_floats_to_bf16"):
            getattr(handle, name).argtypes = [p, p, i64]
        _lib = handle
    return _lib


def default_workers() -> int:
    """The reference CPU default: min(8, CPUs allowed by affinity) (targets/execution.py:20-26)."""
    return min(8, len(os.sched_getaffinity(0)))


def _ptr(array: np.ndarray) -> int:
    return array.ctypes.data


def _code(array: np.ndarray, storage: str | None) -> int:
    if storage == "bf16":
        return BF16
    if array.dtype == np.float16:
        return F16
    if array.dtype == np.float32:
        return F32
    raise TypeError(f"unsupported oracle dtype {array.dtype} / {storage}")


def _rows(array: np.ndarray) -> int:
    return array.strides[0] // array.itemsize if array.shape[0] > 1 else array.shape[1]


def _check_2d(*arrays):
    for a in arrays:
        if a.ndim != 2 or (a.size and a.strides[1] != a.itemsize):
            raise ValueError("oracle expects 2-D arrays with unit inner stride")


# -------------------------------------------------------------------------- conversions
def half_to_float(values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, dtype=np.uint16)
    out = np.empty(values.shape, np.float32)
    lib().oracle_halves_to_floats(_ptr(values), _ptr(out), values.size)
    return out


def float_to_half_bits(values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(values.shape, np.uint16)
    lib().oracle_floats_to_halves(_ptr(values), _ptr(out), values.size)
    return out


def float_to_bf16_bits(values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(values.shape, np.uint16)
    lib().oracle_floats_to_bf16(_ptr(values), _ptr(out), values.size)
    return out


def bf16_bits_to_float(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# -------------------------------------------------------------------------- operators
def softmax_fwd(x: np.ndarray, *, storage: str | None = None, workers: int | None = None) -> np.ndarray:
    """x: float32 / float16 array, or uint16 bf16 bits with storage="bf16"."""
    _check_2d(x)
    y = np.empty(x.shape, x.dtype)
    lib().oracle_softmax_fwd(_code(x, storage), _ptr(x), _ptr(y), x.shape[0], x.shape[1], _rows(x), _rows(y),
                             workers or default_workers())
    return y


def softmax_bwd(p: np.ndarray, dy: np.ndarray, *, storage: str | None = None,
                workers: int | None = None) -> np.ndarray:
    _check_2d(p, dy)
    if p.shape != dy.shape or p.dtype != dy.dtype:
        raise ValueError("p and dy must match")
    dx = np.empty(p.shape, p.dtype)
    lib().oracle_softmax_bwd(_code(p, storage), _ptr(p), _ptr(dy), _ptr(dx), p.shape[0], p.shape[1], _rows(p),
                             _rows(dy), _rows(dx), workers or default_workers())
    return dx


def gemm_bf16(a_bits: np.ndarray, b_bits: np.ndarray, *, workers: int | None = None) -> np.ndarray:
    """a_bits [m,k], b_bits [k,n]: uint16 bf16 bit patterns; returns c bits [m,n]."""
    _check_2d(a_bits, b_bits)
    m, k = a_bits.shape
    n = b_bits.shape[1]
    c = np.empty((m, n), np.uint16)
    lib().oracle_gemm_bf16(_ptr(a_bits), _ptr(b_bits), _ptr(c), m, n, k, _rows(a_bits), _rows(b_bits), n,
                           workers or default_workers())
    return c


def gemm16(a: np.ndarray, b: np.ndarray, *, storage: str | None = None, relu: bool = False,
           workers: int | None = None) -> np.ndarray:
    """`gemm` (f16 operands, ACTIVATION NONE/RELU) or, with storage="bf16", the bf16 variant
    (operands given as uint16 bit patterns). a [m,k], b [k,n]; returns c [m,n] in the operand
    storage."""
    _check_2d(a, b)
    code = BF16 if storage == "bf16" else F16
    if code == F16 and (a.dtype != np.float16 or b.dtype != np.float16):
        raise TypeError("gemm16 f16 operands must be float16 arrays")
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), a.dtype)
    status = lib().oracle_gemm16(code, int(relu), _ptr(a), _ptr(b), _ptr(c), m, n, k, _rows(a), _rows(b), n,
                                 workers or default_workers())
    if status:
        raise ValueError(f"oracle_gemm16 rejected the call ({status})")
    return c


def gemm_f32(a: np.ndarray, b: np.ndarray, *, transpose_b: bool = False, workers: int | None = None) -> np.ndarray:
    """gemm_f32 (b [k,n]) or linear_f32 (transpose_b: b is the weight [n,k]); float32 arrays."""
    _check_2d(a, b)
    if a.dtype != np.float32 or b.dtype != np.float32:
        raise TypeError("gemm_f32 operands must be float32 arrays")
    m, k = a.shape
    n = b.shape[0] if transpose_b else b.shape[1]
    c = np.empty((m, n), np.float32)
    lib().oracle_gemm_f32(_ptr(a), _ptr(b), _ptr(c), m, n, k, _rows(a), _rows(b), n, int(transpose_b),
                          workers or default_workers())
    return c


def attention_fwd(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, causal: bool, *,
                  head_group: int = 1, storage: str | None = None, chunk: int = 64,
                  workers: int | None = None) -> np.ndarray:
    """Grouped-head attention: q [B,HQ,Q,D], k [B,HK,K,D], v [B,HK,K,DV] with HQ = HK * head_group;
    float16 arrays, or uint16 bf16 bit patterns with storage="bf16". Returns o [B,HQ,Q,DV]."""
    batch, heads, sq, d = q.shape
    sk, dv = k.shape[2], v.shape[3]
    if k.shape[1] * head_group != heads or v.shape[1] != k.shape[1]:
        raise ValueError("query heads must equal key heads * head_group")
    code = BF16 if storage == "bf16" else F16
    o = np.empty((batch, heads, sq, dv), q.dtype)
    strides = (ctypes.c_int64 * 16)(*(s // 2 for t in (q, k, v, o) for s in t.strides))
    status = lib().oracle_attention_fwd(code, _ptr(q), _ptr(k), _ptr(v), _ptr(o), batch, heads, head_group, sq, sk,
                                        d, dv, strides, float(np.float32(scale)), int(causal), chunk,
                                        workers or default_workers())
    if status:
        raise ValueError(f"oracle_attention_fwd rejected the call ({status})")
    return o


def gemm_i8(a: np.ndarray, b: np.ndarray, bias: np.ndarray) -> np.ndarray:
    """gemm_i8 (contraction/gemm.py:41-51): c = matmul(a, b, acc_dtype=i32) + bias, int8 operands.
    The products and sums are exact in int64; reducing mod 2^32 afterwards gives what int32
    arithmetic that wraps on overflow gives, in any summation order."""
    total = a.astype(np.int64) @ b.astype(np.int64) + bias.astype(np.int64)[None, :]
    return total.astype(np.uint64).astype(np.uint32).view(np.int32)


def quantized_gemm(a: np.ndarray, b: np.ndarray, bias: np.ndarray, residual: np.ndarray,
                   output_scale: np.ndarray, *, pre_cast: bool = False) -> np.ndarray:
    """quantized_gemm (contraction/gemm.py:95-121): f16 a [m,k], b [k,n], residual [m,n]; f32 bias
    and output_scale [n]; int8 output. The f32 accumulator is the exact sum rounded once to f32 (the
    products of f16 values are exact in float64, and so are their sums at these sizes); the rest
    runs in f32 steps as the definition writes them: maximum(acc + bias, 0) propagating NaN, plus
    the residual, IEEE division by the scale, minimum(maximum(v, -128), 127), then truncation toward
    zero. NaN, an illegal cast input, gives 0. With pre_cast, returns the f32 value before the cast."""
    acc = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        v = acc + bias.astype(np.float32)[None, :]
        v = np.where(np.isnan(v), v, np.maximum(v, np.float32(0)))
        v = v + residual.astype(np.float32)
        v = v / output_scale.astype(np.float32)[None, :]
        v = np.minimum(np.maximum(v, np.float32(-128)), np.float32(127))
        if pre_cast:
            return v
        return np.where(np.isnan(v), 0, np.trunc(v)).astype(np.int8)


def attention_varlen_fwd(q: np.ndarray, k: np.ndarray, v: np.ndarray, cu_seqlens: np.ndarray, scale: float,
                         causal: bool, *, head_group: int = 1, workers: int | None = None) -> np.ndarray:
    """Packed sequences (flash_varlen_attention_fwd, streaming/attention.py:839-877; with heads,
    flash_varlen_gqa_prefill, :880-924): rows cu_seqlens[s] .. cu_seqlens[s+1] of q [U,HQ,D] (or
    [U,D]), k [U,HK,D], v [U,HK,DV] form sequence s, which attends within itself exactly as one
    batch entry of attention_fwd whose row positions start at 0 (I.ragged over the offsets; causal
    compares absolute positions of the same sequence, so relative positions give the same pairs).
    Rows outside every sequence are left 0. Returns float16 like q."""
    squeeze = q.ndim == 2
    if squeeze:
        q, k, v = q[:, None, :], k[:, None, :], v[:, None, :]
    o = np.zeros((q.shape[0], q.shape[1], v.shape[2]), q.dtype)
    for s in range(cu_seqlens.shape[0] - 1):
        lo, hi = int(cu_seqlens[s]), int(cu_seqlens[s + 1])
        if hi <= lo:
            continue
        part = [np.ascontiguousarray(t[lo:hi].transpose(1, 0, 2))[None] for t in (q, k, v)]
        o[lo:hi] = attention_fwd(*part, scale, causal, head_group=head_group, workers=workers)[0].transpose(1, 0, 2)
    return o[:, 0, :] if squeeze else o


def attention_bias_fwd(q: np.ndarray, k: np.ndarray, v: np.ndarray, bias: np.ndarray, scale: float, *,
                       chunk: int = 64, workers: int | None = None) -> np.ndarray:
    """flash_attention_bias_fwd: q [B,H,Q,D], k [B,H,K,D], v [B,H,K,DV] float16, bias [B,H,K] float32;
    returns o [B,H,Q,DV] float16."""
    batch, heads, sq, d = q.shape
    sk, dv = k.shape[2], v.shape[3]
    o = np.empty((batch, heads, sq, dv), np.float16)
    strides = (ctypes.c_int64 * 16)(*(s // 2 for t in (q, k, v, o) for s in t.strides))
    bias_strides = (ctypes.c_int64 * 3)(*(s // 4 for s in bias.strides))
    lib().oracle_attention_bias_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(bias), _ptr(o), batch, heads, sq, sk, d, dv,
                                    strides, bias_strides, float(np.float32(scale)), chunk,
                                    workers or default_workers())
    return o


def mla_prefill(q, qpe, k, kpe, v, scale: float, *, chunk: int = 64, workers: int | None = None) -> np.ndarray:
    """mla_prefill: f16 q [B,H,Q,D], qpe [B,H,Q,P], k [B,HK,K,D], kpe [B,1,K,P], v [B,HK,K,D];
    returns output [B,H,Q,D] f16 (causal, key head = head // (H / HK))."""
    q, qpe, k, kpe, v = (np.ascontiguousarray(a, np.float16) for a in (q, qpe, k, kpe, v))
    batch, heads, sq, d = q.shape
    kv_heads, sk, pdim = k.shape[1], k.shape[2], qpe.shape[3]
    o = np.empty((batch, heads, sq, d), np.float16)
    status = lib().oracle_mla_prefill(_ptr(q), _ptr(qpe), _ptr(k), _ptr(kpe), _ptr(v), _ptr(o), batch, heads, kv_heads,
                                      sq, sk, d, pdim, float(np.float32(scale)), chunk, workers or default_workers())
    if status:
        raise ValueError(f"oracle_mla_prefill rejected the call ({status})")
    return o


def attention_fwd_f16(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, causal: bool, *,
                      chunk: int = 64, workers: int | None = None) -> np.ndarray:
    """q [B,H,Q,D], k [B,H,K,D], v [B,H,K,DV] float16; returns o [B,H,Q,DV] float16."""
    batch, heads, sq, d = q.shape
    sk, dv = k.shape[2], v.shape[3]
    o = np.empty((batch, heads, sq, dv), np.float16)
    strides = (ctypes.c_int64 * 16)(*(s // 2 for t in (q, k, v, o) for s in t.strides))
    lib().oracle_attention_fwd_f16(_ptr(q), _ptr(k), _ptr(v), _ptr(o), batch, heads, sq, sk, d, dv, strides,
                                   float(np.float32(scale)), int(causal), chunk, workers or default_workers())
    return o


def _elem_strides(*arrays):
    return [st // a.itemsize for a in arrays for st in a.strides]


def attention_bwd_delta(o: np.ndarray, dout: np.ndarray, *, workers: int | None = None) -> np.ndarray:
    """attention_backward_delta: o, dout float16 [B,H,Q,D]; returns delta float32 [B,H,Q]."""
    batch, heads, sq, d = o.shape
    delta = np.empty((batch, heads, sq), np.float32)
    strides = (ctypes.c_int64 * 11)(*_elem_strides(o, dout, delta))
    lib().oracle_attention_bwd_delta(_ptr(o), _ptr(dout), _ptr(delta), batch, heads, sq, d, strides,
                                     workers or default_workers())
    return delta


def attention_bwd_dq(q, k, v, dout, lse, delta, scale: float, causal: bool, *, head_group: int = 1,
                     chunk: int = 64, workers: int | None = None) -> np.ndarray:
    """attention_backward_dq: q/dout [B,HQ,Q,D], k/v [B,HK,K,D] float16; lse/delta [B,HQ,Q] float32."""
    batch, heads, sq, d = q.shape
    sk = k.shape[2]
    dq = np.empty(q.shape, np.float16)
    strides = (ctypes.c_int64 * 26)(*_elem_strides(q, k, v, dout, lse, delta, dq))
    status = lib().oracle_attention_bwd_dq(_ptr(q), _ptr(k), _ptr(v), _ptr(dout), _ptr(lse), _ptr(delta), _ptr(dq),
                                           batch, heads, head_group, sq, sk, d, strides, float(np.float32(scale)),
                                           int(causal), chunk, workers or default_workers())
    if status:
        raise ValueError(f"oracle_attention_bwd_dq rejected the call ({status})")
    return dq


def attention_bwd_dkdv(q, k, v, dout, lse, delta, scale: float, causal: bool, *, head_group: int = 1,
                       chunk: int = 64, workers: int | None = None) -> tuple[np.ndarray, np.ndarray]:
    """attention_backward_dkdv: returns (grad_k, grad_v) float16 [B,HK,K,D]."""
    batch, heads, sq, d = q.shape
    sk = k.shape[2]
    dk = np.empty(k.shape, np.float16)
    dv = np.empty(v.shape, np.float16)
    strides = (ctypes.c_int64 * 30)(*_elem_strides(q, k, v, dout, lse, delta, dk, dv))
    status = lib().oracle_attention_bwd_dkdv(_ptr(q), _ptr(k), _ptr(v), _ptr(dout), _ptr(lse), _ptr(delta),
                                             _ptr(dk), _ptr(dv), batch, heads, head_group, sq, sk, d, strides,
                                             float(np.float32(scale)), int(causal), chunk,
                                             workers or default_workers())
    if status:
        raise ValueError(f"oracle_attention_bwd_dkdv rejected the call ({status})")
    return dk, dv


def paged_decode_partials(q, key_cache, value_cache, page_offsets, page_indices, lengths, split_offsets,
                          scale: float, *, page_size: int, head_group: int, splits: int, chunk: int = 64,
                          workers: int | None = None):
    """paged_gqa_decode_partials: returns (partial_lse [B,HQ,SPLITS] f32, partial_output [B,HQ,SPLITS,DV] f32)."""
    q, kc, vc = (np.ascontiguousarray(a, np.float16) for a in (q, key_cache, value_cache))
    po, pi, ln, so = (np.ascontiguousarray(a, np.int32) for a in (page_offsets, page_indices, lengths,
                                                                   split_offsets))
    batch, heads, d = q.shape
    ps, kv_heads, dv = kc.shape[1], kc.shape[2], vc.shape[3]
    lse = np.empty((batch, heads, splits), np.float32)
    out = np.empty((batch, heads, splits, dv), np.float32)
    status = lib().oracle_paged_decode_partials(_ptr(q), _ptr(kc), _ptr(vc), _ptr(po), _ptr(pi), _ptr(ln), _ptr(so),
                                                _ptr(lse), _ptr(out), batch, heads, d, ps, kv_heads, dv, page_size,
                                                head_group, splits, float(np.float32(scale)), chunk,
                                                workers or default_workers())
    if status:
        raise ValueError(f"oracle_paged_decode_partials rejected the call ({status})")
    return lse, out


def grouped_decode_partials(q_bits, k_bits, v_bits, scale: float, *, parts: int, split_size: int, chunk: int = 64,
                            workers: int | None = None):
    """grouped_flash_decode_partials: bf16 bit patterns q [B,HQ,1,D], k [B,HK,K,D], v [B,HK,K,DV];
    returns (partial_lse [B,HQ,P] f32, partial_output [B,HQ,P,DV] bf16 bits)."""
    q, k, v = (np.ascontiguousarray(a, np.uint16) for a in (q_bits, k_bits, v_bits))
    batch, heads, _, d = q.shape
    kv_heads, keys, dv = k.shape[1], k.shape[2], v.shape[3]
    lse = np.empty((batch, heads, parts), np.float32)
    out = np.empty((batch, heads, parts, dv), np.uint16)
    status = lib().oracle_grouped_decode_partials(_ptr(q), _ptr(k), _ptr(v), _ptr(lse), _ptr(out), batch, heads,
                                                  kv_heads, keys, d, dv, parts, split_size, float(np.float32(scale)),
                                                  chunk, workers or default_workers())
    if status:
        raise ValueError(f"oracle_grouped_decode_partials rejected the call ({status})")
    return lse, out


def continuous_gqa_decode(q, k, v, valid_mask, scale: float, *, chunk: int = 64, workers: int | None = None):
    """continuous_gqa_decode: f16 q [B,HQ,D], k [B,K,HK,D], v [B,K,HK,DV], u8 valid_mask [B,K,HK];
    returns output [B,HQ,DV] f16."""
    q, k, v = (np.ascontiguousarray(a, np.float16) for a in (q, k, v))
    mask = np.ascontiguousarray(valid_mask, np.uint8)
    batch, heads, d = q.shape
    keys, kv_heads, dv = k.shape[1], k.shape[2], v.shape[3]
    out = np.empty((batch, heads, dv), np.float16)
    status = lib().oracle_continuous_gqa_decode(_ptr(q), _ptr(k), _ptr(v), _ptr(mask), _ptr(out), batch, heads,
                                                kv_heads, keys, d, dv, float(np.float32(scale)), chunk,
                                                workers or default_workers())
    if status:
        raise ValueError(f"oracle_continuous_gqa_decode rejected the call ({status})")
    return out


def varlen_decode_sink(q, k, v, cu_seqlens, sink, scale: float, *, max_blocks: int, workers: int | None = None):
    """varlen_gqa_decode_with_sink_logits: f16 q [B,HQ,D], k [U,HK,D], v [U,HK,DV], i32 cu [B+1],
    f32 sink [HQ]; returns (output [B,HQ,DV] f16, block_logits [B,HQ,max_blocks] f32)."""
    q, k, v = (np.ascontiguousarray(a, np.float16) for a in (q, k, v))
    cu = np.ascontiguousarray(cu_seqlens, np.int32)
    sink = np.ascontiguousarray(sink, np.float32)
    sequences, heads, d = q.shape
    kv_heads, dv = k.shape[1], v.shape[2]
    out = np.empty((sequences, heads, dv), np.float16)
    logits = np.empty((sequences, heads, max_blocks), np.float32)
    status = lib().oracle_varlen_decode_sink(_ptr(q), _ptr(k), _ptr(v), _ptr(cu), _ptr(sink), _ptr(out), _ptr(logits),
                                             sequences, heads, kv_heads, d, dv, max_blocks, float(np.float32(scale)),
                                             workers or default_workers())
    if status:
        raise ValueError(f"oracle_varlen_decode_sink rejected the call ({status})")
    return out, logits


def splitk_reduce_f32_to_f16(partial, partial_lse, *, workers: int | None = None) -> np.ndarray:
    """splitk_attention_f32_to_f16_reduce: partial [B,H,S,D] f32, lse [B,H,S] f32 -> [B,H,D] f16."""
    partial = np.ascontiguousarray(partial, np.float32)
    lse = np.ascontiguousarray(partial_lse, np.float32)
    batch, heads, splits, d = partial.shape
    out = np.empty((batch, heads, d), np.float16)
    lib().oracle_splitk_reduce_f32_to_f16(_ptr(partial), _ptr(lse), _ptr(out), batch, heads, splits, d,
                                          workers or default_workers())
    return out


def csr_spmm(offsets: np.ndarray, columns: np.ndarray, values: np.ndarray, dense: np.ndarray, *,
             workers: int | None = None) -> np.ndarray:
    """csr_spmm: out [rows, features] f32, each feature folded over the row's nonzeros in order."""
    offsets = np.ascontiguousarray(offsets, np.int32)
    columns = np.ascontiguousarray(columns, np.int32)
    values = np.ascontiguousarray(values, np.float32)
    dense = np.ascontiguousarray(dense, np.float32)
    rows, features = offsets.shape[0] - 1, dense.shape[1]
    out = np.empty((rows, features), np.float32)
    lib().oracle_csr_spmm_f32(_ptr(offsets), _ptr(columns), _ptr(values), _ptr(dense), _ptr(out), rows, features,
                              features, features, workers or default_workers())
    return out


def csr_spmv(offsets: np.ndarray, columns: np.ndarray, values: np.ndarray, x: np.ndarray, *,
             workers: int | None = None) -> np.ndarray:
    offsets = np.ascontiguousarray(offsets, np.int32)
    columns = np.ascontiguousarray(columns, np.int32)
    values = np.ascontiguousarray(values, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    rows = offsets.shape[0] - 1
    y = np.empty(rows, np.float32)
    lib().oracle_csr_spmv_f32(_ptr(offsets), _ptr(columns), _ptr(values), _ptr(x), _ptr(y), rows,
                              workers or default_workers())
    return y
