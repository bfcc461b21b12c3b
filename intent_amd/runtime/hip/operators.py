"""Definitions the hip provider recognises, and how each is launched.

A definition is recognised by its name plus its runtime signature (access kind,
dtype and rank of every parameter, constexpr names). The signature check stops a
same-named definition with a different contract from being routed to a kernel.
Recognised definitions (reference file:line of the semantics each kernel follows):

  stable_softmax          normalization/softmax.py:23-36   intent_hip_softmax_fwd (f32)
  stable_softmax_f16      normalization/softmax.py:39-51   intent_hip_softmax_fwd (f16)
  chunked_softmax_bf16    normalization/softmax.py:54-66   intent_hip_softmax_fwd (bf16)
  softmax_backward        backward/softmax.py:9-25         intent_hip_softmax_bwd (f32)
  softmax_backward_f16    f16-storage variant of the same  intent_hip_softmax_bwd (f16)
  gemm_f32                contraction/gemm.py:15-27        intent_hip_gemm_f32 (transpose_b 0)
  linear_f32              contraction/gemm.py:30-38        intent_hip_gemm_f32 (transpose_b 1)
  gemm_i8                 contraction/gemm.py:41-51        intent_hip_gemm_i8
  gemm                    contraction/gemm.py:54-73        intent_hip_gemm (f16, ACTIVATION)
  quantized_gemm          contraction/gemm.py:95-121       intent_hip_quantized_gemm
  bf16_gemm               contraction/gemm.py:76-92        intent_hip_gemm_bf16
  flash_attention_fwd     streaming/attention.py:428-466   intent_hip_attention_fwd_f16
  flash_gqa_attention_fwd streaming/attention.py:469-507   intent_hip_attention_fwd (f16, HEAD_GROUP)
  flash_attention_bf16_fwd streaming/attention.py:510-553  intent_hip_attention_fwd (bf16, HEAD_GROUP)
  flash_attention_bias_fwd streaming/attention.py:800-836  intent_hip_attention_bias_fwd
  mla_prefill             streaming/attention.py:756-798   intent_hip_mla_prefill (HEAD_GROUP, causal)
  flash_varlen_attention_fwd streaming/attention.py:839-877 intent_hip_attention_varlen_fwd (one head, CAUSAL)
  flash_varlen_gqa_prefill streaming/attention.py:880-924  intent_hip_attention_varlen_fwd (HEAD_GROUP, causal)
  csr_spmv                sparse/csr_spmv.py:11-29         intent_hip_csr_spmv_f32
  attention_backward_delta backward/attention.py:17-34     intent_hip_attention_bwd_delta
  attention_backward_dkdv backward/attention.py:87-137     intent_hip_attention_bwd_dkdv
  attention_backward_dq   backward/attention.py:171-211    intent_hip_attention_bwd_dq
  paged_gqa_decode_partials streaming/paged_attention.py:77-165  intent_hip_paged_decode_partials
  splitk_attention_f32_to_f16_reduce streaming/splitk_reduce.py:129-155  intent_hip_splitk_reduce_f32_to_f16
  grouped_flash_decode_partials streaming/attention.py:556-627  intent_hip_grouped_decode_partials
  continuous_gqa_decode   streaming/attention.py:629-670   intent_hip_continuous_gqa_decode
  varlen_gqa_decode_with_sink_logits streaming/attention.py:672-754  intent_hip_varlen_decode_sink
  csr_spmm                sparse/csr_spmm.py:11-33         intent_hip_csr_spmm_f32

(paths relative to python/intent/examples/kernels/ in the reference).

Layout handling: kernels read rows with unit inner stride. An input whose inner
stride is not 1 is copied into a contiguous device buffer at every launch (on
the launch stream, so the copy sees the values current at launch time); an Out
buffer with a non-unit inner stride receives the result through a contiguous
buffer copied back after the kernel.
"""
from __future__ import annotations

import contextlib
import contextvars
from dataclasses import dataclass, field
from typing import Callable

from ...diagnostics import CompilationStageError
from .library import (BF16, F16, F32, STATIC_SCRATCH_BYTES, OP_ATTENTION_BWD_DELTA, OP_ATTENTION_BWD_DKDV, OP_ATTENTION_BWD_DQ,
                      OP_ATTENTION_FWD, OP_ATTENTION_FWD_F16, OP_ATTENTION_BIAS, OP_ATTENTION_VARLEN, OP_MLA_PREFILL, OP_CSR_SPMV_F32, OP_GEMM, OP_GEMM_BF16, OP_GEMM_F32, OP_GEMM_I8, OP_QUANTIZED_GEMM,
                      OP_CSR_SPMM_F32, OP_CONTINUOUS_DECODE, OP_GROUPED_DECODE_PARTIALS, OP_PAGED_DECODE_PARTIALS, OP_VARLEN_DECODE, OP_SOFTMAX_BWD, OP_SOFTMAX_FWD, OP_SPLITK_REDUCE)


@dataclass
class Launch:
    """A bound native call: `run(stream)` returns the ABI status."""

    entry: str
    run: Callable[[int], int]
    keep: tuple = ()
    before: tuple = ()            # callables run on the launch stream before the kernel
    after: tuple = ()             # callables run on the launch stream after the kernel
    configuration: tuple = ()
    resources: Callable[[], dict | None] = field(default=lambda: None)
    candidates: tuple = ()        # (row, eligible, reasons) of the definition's tuning family, table order


@dataclass(frozen=True)
class OperatorSpec:
    name: str
    signature: tuple              # per runtime parameter: ("view", access, dtype, rank) | ("scalar", dtype)
    constexprs: tuple[str, ...]
    plan: Callable
    inplace_safe: bool = False    # an Out may be exactly one of the inputs (same address and strides)
    derived: tuple = ()           # (symbol, source symbol, offset): extent(symbol) = extent(source) + offset

    @property
    def entry_point(self) -> str:
        """The C-ABI function (include/intent_hip.h) a launch of this definition calls."""
        return ENTRY_POINTS[self.name]


IN, OUT = 0, 1


def _view(access, dtype, rank):
    return ("view", access, dtype, rank)


# ------------------------------------------------------------------------------ workspace policy
# The target's backend_options["workspace"]: "prepare" lets a plan allocate device memory once per
# prepared call (staging copies, SpMV plan, split partial sums); "static" forbids it.
_WORKSPACE = contextvars.ContextVar("intent_hip_workspace", default="prepare")


@contextlib.contextmanager
def workspace_policy(policy: str):
    """Plans made inside this block follow `policy` ("prepare" or "static")."""
    token = _WORKSPACE.set(policy)
    try:
        yield
    finally:
        _WORKSPACE.reset(token)


def _static_workspace() -> bool:
    return _WORKSPACE.get() == "static"


# The program's compile options numerics: "source" keeps every low-precision cast where the
# definition puts it; "relaxed_normalization" lets a plan pick a kernel that applies the
# normalized-summary rewrite.
_NUMERICS = contextvars.ContextVar("intent_hip_numerics", default="source")


@contextlib.contextmanager
def numerics_policy(numerics: str):
    token = _NUMERICS.set(numerics)
    try:
        yield
    finally:
        _NUMERICS.reset(token)


def _relaxed_normalization() -> bool:
    return _NUMERICS.get() == "relaxed_normalization"


# The program's rows of its tuning family (runtime/hip/tuning.py), in table order.
_TUNING = contextvars.ContextVar("intent_hip_tuning", default=None)


@contextlib.contextmanager
def tuning_policy(rows):
    token = _TUNING.set(rows)
    try:
        yield
    finally:
        _TUNING.reset(token)


def _split_choice(family: str, split_bytes: int) -> tuple[int, tuple]:
    """The first eligible row of `family` (columns: split) and every row's assessment. split = 1
    needs a grid small enough to split (split_bytes > 0: the workspace it takes) and a workspace
    policy that allows one; split = 0 is always eligible."""
    from .tuning import DEFAULT_FAMILIES

    rows = _TUNING.get() or DEFAULT_FAMILIES[family]
    candidates, chosen = [], None
    for row in rows:
        reasons = []
        if row[0] == 1:
            if _static_workspace():
                reasons.append("backend_options workspace='static' allows no workspace")
            if split_bytes <= 0:
                reasons.append("nothing to split: the grid fills the device or the walk is too short")
        candidates.append((row, not reasons, tuple(reasons)))
        if not reasons and chosen is None:
            chosen = row[0]
    if chosen is None:
        raise CompilationStageError("provider_configuration",
                                    f"no row of tuning family {family} is eligible for this call: "
                                    + "; ".join(f"{list(r)}: {', '.join(why)}" for r, _, why in candidates))
    return chosen, tuple(candidates)


# ------------------------------------------------------------------------------ layout helpers
def _aligned(tensor, vector: int) -> bool:
    """Unit inner stride, outer strides multiples of `vector` elements, 16-byte aligned start."""
    if tensor.numel() == 0 or tensor.dim() == 0:
        return True
    if tensor.stride(-1) != 1 and tensor.shape[-1] > 1:
        return False
    if vector > 1:
        if tensor.data_ptr() % 16:
            return False
        if any(s % vector for s, e in zip(tensor.stride()[:-1], tensor.shape[:-1]) if e > 1):
            return False
    return True


def _readable(tensor, keep, before, vector: int = 1):
    """A tensor with the contents of `tensor` at launch time whose layout the kernel takes
    (unit inner stride; with `vector`, also aligned for 16-byte loads)."""
    if _aligned(tensor, vector):
        return tensor
    _refuse_staging(tensor, vector)
    staged = tensor.new_empty(tensor.shape)
    keep.append(staged)
    before.append(lambda: staged.copy_(tensor))
    return staged


def _writable(tensor, keep, after, vector: int = 1):
    if _aligned(tensor, vector):
        return tensor
    _refuse_staging(tensor, vector)
    staged = tensor.new_empty(tensor.shape)
    keep.append(staged)
    after.append(lambda: tensor.copy_(staged))
    return staged


def _refuse_staging(tensor, vector: int) -> None:
    if _static_workspace():
        need = "unit inner stride" + (f", outer strides in multiples of {vector} and a 16-byte aligned start"
                                      if vector > 1 else "")
        raise ValueError(f"with backend_options workspace='static' the provider does not stage views; this "
                         f"kernel needs {need}, got strides {tuple(tensor.stride())}")


# ------------------------------------------------------------------------------ attention head dimensions
# The attention kernels are built for key and value head dimensions of 64 and 128. Any other width up
# to 128 (the reference declares D and DV symbolic, streaming/attention.py:428-553) runs on the next of
# the two through zero-padded copies refreshed at each launch: zero dimensions add exact zeros to
# every score's sum and give output columns that are dropped, so results equal the unpadded ones.
_KERNEL_WIDTHS = (64, 128)


def _kernel_width(extent: int, name: str) -> int:
    for width in _KERNEL_WIDTHS:
        if extent <= width:
            return width
    raise CompilationStageError("provider_configuration",
                                f"{name} = {extent}: the hip attention kernels take head dimensions up to "
                                f"{_KERNEL_WIDTHS[-1]}")


def _padded_in(tensor, width, keep, before):
    """`tensor` with its last dimension extended to `width` by zeros; the copy runs at each launch."""
    _refuse_staging(tensor, 8)
    staged = tensor.new_zeros(tuple(tensor.shape[:-1]) + (width,))
    head = staged[..., :tensor.shape[-1]]
    keep.append(staged)
    before.append(lambda: head.copy_(tensor))
    return staged


def _padded_out(tensor, width, keep, after):
    """A buffer of last dimension `width` whose first columns are copied into `tensor` after a launch."""
    _refuse_staging(tensor, 8)
    staged = tensor.new_empty(tuple(tensor.shape[:-1]) + (width,))
    head = staged[..., :tensor.shape[-1]]
    keep.append(staged)
    after.append(lambda: tensor.copy_(head))
    return staged


def _attention_views(q, k, v, o, keep, before, after):
    """q, k, v and o as an attention kernel reads them, and the kernel's (d, dv): unit inner stride,
    16-byte aligned rows, head dimensions padded to 64 or 128 where they are not."""
    d, dv = q.shape[-1], v.shape[-1]
    kd, kdv = _kernel_width(d, "d"), _kernel_width(dv, "dv")
    if kd != d:
        qk, kk = _padded_in(q, kd, keep, before), _padded_in(k, kd, keep, before)
    else:
        qk, kk = _readable(q, keep, before, 8), _readable(k, keep, before, 8)
    if kdv != dv:
        vk, ok = _padded_in(v, kdv, keep, before), _padded_out(o, kdv, keep, after)
    else:
        vk, ok = _readable(v, keep, before, 8), _writable(o, keep, after, 8)
    return qk, kk, vk, ok, kd, kdv


def _row_stride(tensor):
    rows, cols = tensor.shape
    return tensor.stride(0) if rows > 1 else cols


# ------------------------------------------------------------------------------ softmax
def _softmax_fwd(dtype_code):
    def plan(lib, bound, constexprs, device):
        x, y = bound.arguments
        keep, before, after = [x, y], [], []
        xk, yk = _readable(x, keep, before), _writable(y, keep, after)
        rows, cols = x.shape
        fn = lib.fn["softmax_fwd"]
        args = (dtype_code, xk.data_ptr(), yk.data_ptr(), rows, cols, _row_stride(xk), _row_stride(yk))
        return Launch("intent_hip_softmax_fwd", lambda stream: fn(*args, stream), tuple(keep), tuple(before),
                      tuple(after), (("rows", rows), ("cols", cols)),
                      lambda: lib.kernel_resources(OP_SOFTMAX_FWD, dtype_code, rows, cols))
    return plan


def _softmax_bwd(dtype_code):
    def plan(lib, bound, constexprs, device):
        p, dy, dx = bound.arguments
        keep, before, after = [p, dy, dx], [], []
        pk, gk, dk = _readable(p, keep, before), _readable(dy, keep, before), _writable(dx, keep, after)
        rows, cols = p.shape
        fn = lib.fn["softmax_bwd"]
        args = (dtype_code, pk.data_ptr(), gk.data_ptr(), dk.data_ptr(), rows, cols, _row_stride(pk),
                _row_stride(gk), _row_stride(dk))
        return Launch("intent_hip_softmax_bwd", lambda stream: fn(*args, stream), tuple(keep), tuple(before),
                      tuple(after), (("rows", rows), ("cols", cols)),
                      lambda: lib.kernel_resources(OP_SOFTMAX_BWD, dtype_code, rows, cols))
    return plan


# ------------------------------------------------------------------------------ GEMM
def _gemm_bf16(lib, bound, constexprs, device):
    a, b, c = bound.arguments
    keep, before, after = [a, b, c], [], []
    ak, bk, ck = _readable(a, keep, before), _readable(b, keep, before), _writable(c, keep, after)
    m, k = a.shape
    n = b.shape[1]
    fn = lib.fn["gemm_bf16"]
    args = (ak.data_ptr(), bk.data_ptr(), ck.data_ptr(), m, n, k, _row_stride(ak), _row_stride(bk),
            _row_stride(ck))
    return Launch("intent_hip_gemm_bf16", lambda stream: fn(*args, stream), tuple(keep), tuple(before),
                  tuple(after), (("m", m), ("n", n), ("k", k)),
                  lambda: lib.kernel_resources(OP_GEMM_BF16, BF16, m, n))


def _activation_code(value) -> int:
    """ACTIVATION constexpr (an Activation enum member, gemm.py:10-12) -> ABI code."""
    code = getattr(value, "value", value)
    if code not in (0, 1):
        raise CompilationStageError("provider_configuration",
                                    f"the hip gemm supports ACTIVATION NONE (0) or RELU (1), got {value!r}")
    return int(code)


def _gemm16(dtype_code):
    def plan(lib, bound, constexprs, device):
        a, b, c = bound.arguments
        activation = _activation_code(constexprs.get("ACTIVATION", 0))
        keep, before, after = [a, b, c], [], []
        ak, bk, ck = _readable(a, keep, before), _readable(b, keep, before), _writable(c, keep, after)
        m, k = a.shape
        n = b.shape[1]
        fn = lib.fn["gemm"]
        args = (dtype_code, activation, ak.data_ptr(), bk.data_ptr(), ck.data_ptr(), m, n, k, _row_stride(ak),
                _row_stride(bk), _row_stride(ck))
        return Launch("intent_hip_gemm", lambda stream: fn(*args, stream), tuple(keep), tuple(before),
                      tuple(after), (("m", m), ("n", n), ("k", k), ("activation", activation)),
                      lambda: lib.kernel_resources(OP_GEMM, dtype_code, m, n))
    return plan


def _gemm_f32(transpose_b: bool):
    def plan(lib, bound, constexprs, device):
        a, b, c = bound.arguments
        keep, before, after = [a, b, c], [], []
        ak, bk, ck = _readable(a, keep, before), _readable(b, keep, before), _writable(c, keep, after)
        m, k = a.shape
        n = b.shape[0] if transpose_b else b.shape[1]
        fn = lib.fn["gemm_f32"]
        args = (ak.data_ptr(), bk.data_ptr(), ck.data_ptr(), m, n, k, _row_stride(ak), _row_stride(bk),
                _row_stride(ck), int(transpose_b))
        return Launch("intent_hip_gemm_f32", lambda stream: fn(*args, stream), tuple(keep), tuple(before),
                      tuple(after), (("m", m), ("n", n), ("k", k), ("transpose_b", transpose_b)),
                      lambda: lib.kernel_resources(OP_GEMM_F32, F32, m, n))
    return plan


def _gemm_i8(lib, bound, constexprs, device):
    a, b, bias, c = bound.arguments
    keep, before, after = [a, b, bias, c], [], []
    ak, bk, biask, ck = (_readable(a, keep, before), _readable(b, keep, before), _readable(bias, keep, before),
                         _writable(c, keep, after))
    m, k = a.shape
    n = b.shape[1]
    fn = lib.fn["gemm_i8"]
    args = (ak.data_ptr(), bk.data_ptr(), biask.data_ptr(), ck.data_ptr(), m, n, k, _row_stride(ak), _row_stride(bk),
            _row_stride(ck))
    return Launch("intent_hip_gemm_i8", lambda stream: fn(*args, stream), tuple(keep), tuple(before), tuple(after),
                  (("m", m), ("n", n), ("k", k)), lambda: lib.kernel_resources(OP_GEMM_I8, 0, m, n))


def _quantized_gemm(lib, bound, constexprs, device):
    a, b, bias, residual, scale, out = bound.arguments
    keep, before, after = [a, b, bias, residual, scale, out], [], []
    ak, bk = _readable(a, keep, before), _readable(b, keep, before)
    biask, rk, sk = _readable(bias, keep, before), _readable(residual, keep, before), _readable(scale, keep, before)
    ok = _writable(out, keep, after)
    m, k = a.shape
    n = b.shape[1]
    fn = lib.fn["quantized_gemm"]
    args = (ak.data_ptr(), bk.data_ptr(), biask.data_ptr(), rk.data_ptr(), sk.data_ptr(), ok.data_ptr(), m, n, k,
            _row_stride(ak), _row_stride(bk), _row_stride(rk), _row_stride(ok))
    return Launch("intent_hip_quantized_gemm", lambda stream: fn(*args, stream), tuple(keep), tuple(before),
                  tuple(after), (("m", m), ("n", n), ("k", k)), lambda: lib.kernel_resources(OP_QUANTIZED_GEMM, 0, m, n))


# ------------------------------------------------------------------------------ attention
def _attention_launch(lib, dtype_code, q, k, v, o, scale, group, causal, entry, device):
    """The batched attention forward (head_group query heads per key head). A grid too small to fill
    the device splits each query block's keys over workgroups through a workspace (tuning family
    hip.attention_forward; with workspace='static' or the unsplit row the launch stays unsplit)."""
    import ctypes

    import torch

    keep, before, after = [q, k, v, o], [], []
    qk, kk, vk, ok, d, dv = _attention_views(q, k, v, o, keep, before, after)
    batch, q_heads, sq = q.shape[:3]
    sk = k.shape[2]
    strides = (ctypes.c_int64 * 16)(*(s for t in (qk, kk, vk, ok) for s in t.stride()))
    keep.append(strides)
    size = ctypes.c_size_t(0)
    lib.check(lib.fn["attention_fwd_workspace_bytes"](batch, q_heads, sq, sk, dv, ctypes.byref(size)),
              "provider_preparation")
    split, candidates = _split_choice("hip.attention_forward", size.value)
    config = (("batch", batch), ("q_heads", q_heads), ("head_group", group), ("sq", sq), ("sk", sk), ("d", d),
              ("dv", dv), ("causal", causal), ("split", split))
    resources = lambda: lib.kernel_resources(OP_ATTENTION_FWD, dtype_code, sq, d | (dv << 16))  # noqa: E731
    if split:
        workspace = torch.empty(size.value, dtype=torch.uint8, device=device)
        keep.append(workspace)
        fn = lib.fn["attention_fwd_ws"]
        args = (dtype_code, qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), ok.data_ptr(), batch, q_heads, group, sq,
                sk, d, dv, strides, float(scale), int(causal), workspace.data_ptr(), size.value)
        return Launch("intent_hip_attention_fwd_ws", lambda stream: fn(*args, stream), tuple(keep), tuple(before),
                      tuple(after), config, resources, candidates)
    if entry == "intent_hip_attention_fwd_f16":
        fn = lib.fn["attention_fwd_f16"]
        args = (qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), ok.data_ptr(), batch, q_heads, sq, sk, d, dv, strides,
                float(scale), int(causal))
    else:
        fn = lib.fn["attention_fwd"]
        args = (dtype_code, qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), ok.data_ptr(), batch, q_heads, group, sq,
                sk, d, dv, strides, float(scale), int(causal))
    return Launch(entry, lambda stream: fn(*args, stream), tuple(keep), tuple(before), tuple(after), config,
                  resources if entry != "intent_hip_attention_fwd_f16"
                  else (lambda: lib.kernel_resources(OP_ATTENTION_FWD_F16, F16, sq, d | (dv << 16))), candidates)


def _attention_f16(lib, bound, constexprs, device):
    q, k, v, o, scale = bound.arguments
    return _attention_launch(lib, F16, q, k, v, o, scale, 1, bool(constexprs["CAUSAL"]),
                             "intent_hip_attention_fwd_f16", device)


def _attention_grouped(dtype_code):
    """flash_gqa_attention_fwd (f16) / flash_attention_bf16_fwd (bf16): key head = query head //
    HEAD_GROUP (attention.py:485, 528)."""
    def plan(lib, bound, constexprs, device):
        q, k, v, o, scale = bound.arguments
        group = constexprs["HEAD_GROUP"]
        if isinstance(group, bool) or not isinstance(group, int) or group < 1:
            raise CompilationStageError("provider_configuration", f"HEAD_GROUP must be a positive int, got {group!r}")
        if k.shape[1] * group != q.shape[1]:
            raise ValueError(f"query heads ({q.shape[1]}) must equal key/value heads ({k.shape[1]}) * HEAD_GROUP "
                             f"({group})")
        return _attention_launch(lib, dtype_code, q, k, v, o, scale, group, bool(constexprs["CAUSAL"]),
                                 "intent_hip_attention_fwd", device)
    return plan


def _attention_bias(lib, bound, constexprs, device):
    """flash_attention_bias_fwd: scores (q . k) scale + bias[b, h, key] over every key, no mask
    (attention.py:800-836, :328-366)."""
    import ctypes

    q, k, v, bias, o, scale = bound.arguments
    batch, heads, sq = q.shape[:3]
    sk = k.shape[2]
    if tuple(bias.shape) != (batch, heads, sk):
        raise ValueError(f"bias must be [B, H, K] = {(batch, heads, sk)}, got {tuple(bias.shape)}")
    keep, before, after = [q, k, v, bias, o], [], []
    qk, kk, vk, ok, d, dv = _attention_views(q, k, v, o, keep, before, after)
    bk = _readable(bias, keep, before)
    strides = (ctypes.c_int64 * 16)(*(s for t in (qk, kk, vk, ok) for s in t.stride()))
    bias_strides = (ctypes.c_int64 * 3)(*bk.stride())
    keep += [strides, bias_strides]
    fn = lib.fn["attention_bias_fwd"]
    args = (qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), bk.data_ptr(), ok.data_ptr(), batch, heads, sq, sk, d, dv,
            strides, bias_strides, float(scale))
    return Launch("intent_hip_attention_bias_fwd", lambda stream: fn(*args, stream), tuple(keep), tuple(before),
                  tuple(after), (("batch", batch), ("heads", heads), ("sq", sq), ("sk", sk), ("d", d), ("dv", dv)),
                  lambda: lib.kernel_resources(OP_ATTENTION_BIAS, F16, sq, d | (dv << 16)))


def _mla_prefill(lib, bound, constexprs, device):
    """mla_prefill: causal latent attention, scores (q . k + qpe . kpe) scale (attention.py:756-798)."""
    import ctypes

    import torch

    q, qpe, k, kpe, v, o, scale = bound.arguments
    group = _head_group(constexprs)
    batch, heads, sq, d = q.shape
    sk, p = k.shape[2], qpe.shape[3]
    if k.shape[1] * group != heads or v.shape[1] != k.shape[1]:
        raise ValueError(f"query heads ({heads}) must equal key/value heads ({k.shape[1]}) * HEAD_GROUP ({group})")
    keep, before, after = [q, qpe, k, kpe, v, o], [], []
    views = [_readable(t, keep, before, 8) for t in (q, qpe, k, kpe, v)] + [_writable(o, keep, after, 8)]
    strides = _strides(*views)
    keep.append(strides)
    # Small grids split the keys over workgroups through a workspace (tuning family
    # hip.latent_prefill; with workspace='static' or the unsplit row the launch stays unsplit).
    size = ctypes.c_size_t(0)
    lib.check(lib.fn["mla_prefill_workspace_bytes"](batch, heads, sq, sk, d, ctypes.byref(size)), "provider_preparation")
    split, candidates = _split_choice("hip.latent_prefill", size.value)
    workspace = None
    if split:
        workspace = torch.empty(size.value, dtype=torch.uint8, device=device)
        keep.append(workspace)
    fn = lib.fn["mla_prefill"]
    args = (*(t.data_ptr() for t in views), batch, heads, group, sq, sk, d, p, strides, float(scale),
            workspace.data_ptr() if workspace is not None else None, size.value if workspace is not None else 0)
    return Launch("intent_hip_mla_prefill", lambda stream: fn(*args, stream), tuple(keep), tuple(before),
                  tuple(after), (("batch", batch), ("heads", heads), ("head_group", group), ("sq", sq), ("sk", sk),
                                 ("d", d), ("p", p), ("split", split)),
                  lambda: lib.kernel_resources(OP_MLA_PREFILL, F16, sq, d | (p << 16)), candidates)


def _head_group(constexprs) -> int:
    group = constexprs["HEAD_GROUP"]
    if isinstance(group, bool) or not isinstance(group, int) or group < 1:
        raise CompilationStageError("provider_configuration", f"HEAD_GROUP must be a positive int, got {group!r}")
    return group


def _attention_varlen(grouped: bool):
    """flash_varlen_attention_fwd (q [U,D], one head, CAUSAL) / flash_varlen_gqa_prefill (q [U,HQ,D],
    key head = query head // HEAD_GROUP, causal): packed sequences delimited by cu_seqlens
    (attention.py:839-924). The offsets stay on the device: the kernel's own pre-pass lists the
    work items into a workspace allocated here, once per prepared call."""
    def plan(lib, bound, constexprs, device):
        import ctypes

        import torch

        q, k, v, lengths, cu, o, scale = bound.arguments
        if grouped:
            group, causal = _head_group(constexprs), True
            total, q_heads, d = q.shape
            if k.shape[1] * group != q_heads or v.shape[1] != k.shape[1]:
                raise ValueError(f"query heads ({q_heads}) must equal key/value heads ({k.shape[1]}) * HEAD_GROUP "
                                 f"({group})")
            dv = v.shape[2]
        else:
            group, causal = 1, bool(constexprs["CAUSAL"])
            (total, d), q_heads, dv = q.shape, 1, v.shape[1]
        sequences = lengths.shape[0]
        if cu.shape[0] != sequences + 1:
            raise ValueError(f"cu_seqlens needs sequence_lengths.shape[0] + 1 = {sequences + 1} entries, "
                             f"got {cu.shape[0]}")
        if k.shape[0] != total or v.shape[0] != total:
            raise ValueError("q, k and v must hold the same packed rows")
        if _static_workspace():
            raise CompilationStageError(
                "provider_preparation", "packed-sequence attention lists its work items in a workspace; "
                "backend_options workspace='static' has none for it, use workspace='prepare'")
        keep, before, after = [q, k, v, lengths, cu, o], [], []
        qk, kk, vk, ok, d, dv = _attention_views(q, k, v, o, keep, before, after)
        cuk = _readable(cu, keep, before)

        def row_head_inner(t):
            return (t.stride(0), t.stride(1), t.stride(2)) if t.dim() == 3 else (t.stride(0), 0, t.stride(1))

        strides = (ctypes.c_int64 * 12)(*(x for t in (qk, kk, vk, ok) for x in row_head_inner(t)))
        size = ctypes.c_size_t(0)
        lib.check(lib.fn["attention_varlen_workspace_bytes"](sequences, total, ctypes.byref(size)),
                  "provider_preparation")
        workspace = torch.empty(max(size.value, 1), dtype=torch.uint8, device=device)
        keep += [strides, workspace]
        fn = lib.fn["attention_varlen_fwd"]
        args = (F16, qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), cuk.data_ptr(), ok.data_ptr(), sequences, total,
                q_heads, group, d, dv, strides, float(scale), int(causal), workspace.data_ptr(), size.value)
        return Launch("intent_hip_attention_varlen_fwd", lambda stream: fn(*args, stream), tuple(keep),
                      tuple(before), tuple(after),
                      (("sequences", sequences), ("total", total), ("q_heads", q_heads), ("head_group", group),
                       ("d", d), ("dv", dv), ("causal", causal), ("workspace_bytes", size.value)),
                      lambda: lib.kernel_resources(OP_ATTENTION_VARLEN, F16, total, d | (dv << 16)))
    return plan


# ------------------------------------------------------------------------------ attention backward
def _strides(*tensors):
    import ctypes

    values = [st for t in tensors for st in t.stride()]
    return (ctypes.c_int64 * len(values))(*values)


def _attention_bwd_delta(lib, bound, constexprs, device):
    o, dout, delta = bound.arguments
    keep, before, after = [o, dout, delta], [], []
    ok, gk = _readable(o, keep, before, 8), _readable(dout, keep, before, 8)
    batch, heads, sq, d = o.shape
    strides = _strides(ok, gk, delta)
    keep.append(strides)
    fn = lib.fn["attention_bwd_delta"]
    args = (ok.data_ptr(), gk.data_ptr(), delta.data_ptr(), batch, heads, sq, d, strides)
    return Launch("intent_hip_attention_bwd_delta", lambda stream: fn(*args, stream), tuple(keep), tuple(before),
                  tuple(after), (("batch", batch), ("heads", heads), ("sq", sq), ("d", d)),
                  lambda: lib.kernel_resources(OP_ATTENTION_BWD_DELTA, F16, sq, d))


def _backward_group(q, k, constexprs):
    group = constexprs["HEAD_GROUP"]
    if isinstance(group, bool) or not isinstance(group, int) or group < 1:
        raise CompilationStageError("provider_configuration", f"HEAD_GROUP must be a positive int, got {group!r}")
    if k.shape[1] * group != q.shape[1]:
        raise ValueError(f"query heads ({q.shape[1]}) must equal key/value heads ({k.shape[1]}) * HEAD_GROUP "
                         f"({group})")
    return group


def _attention_bwd(kind):
    """attention_backward_dq (kind "dq") / attention_backward_dkdv (kind "dkdv"); lse and delta are
    read through their own strides, 4-D operands with unit inner stride (staged otherwise)."""
    def plan(lib, bound, constexprs, device):
        if kind == "dq":
            q, k, v, dout, lse, delta, out, scale = bound.arguments
            outs = (out,)
        else:
            q, k, v, dout, lse, delta, grad_k, grad_v, scale = bound.arguments
            outs = (grad_k, grad_v)
        group = _backward_group(q, k, constexprs)
        causal = bool(constexprs["CAUSAL"])
        keep, before, after = [q, k, v, dout, lse, delta, *outs], [], []
        ins = [_readable(t, keep, before, 8) for t in (q, k, v, dout)]
        staged_outs = [_writable(t, keep, after, 8) for t in outs]
        batch, q_heads, sq, d = q.shape
        sk = k.shape[2]
        strides = _strides(*ins, lse, delta, *staged_outs)
        keep.append(strides)
        args = (*(t.data_ptr() for t in ins), lse.data_ptr(), delta.data_ptr(),
                *(t.data_ptr() for t in staged_outs), batch, q_heads, group, sq, sk, d, strides, float(scale),
                int(causal))
        configuration = (("batch", batch), ("q_heads", q_heads), ("head_group", group), ("sq", sq), ("sk", sk),
                         ("d", d), ("causal", causal))
        # Small grids split their work over more workgroups; the f32 partial sums need a
        # workspace, allocated here once per prepared call.
        import ctypes

        import torch

        # (tuning family hip.attention_backward: split = 0 runs the unsplit kernels)
        size = ctypes.c_size_t(0)
        lib.check(lib.fn[f"attention_bwd_{kind}_workspace_bytes"](batch, q_heads, group, sq, sk, d,
                                                                 ctypes.byref(size)), "provider_preparation")
        split, candidates = _split_choice("hip.attention_backward", size.value)
        workspace = torch.empty(size.value, dtype=torch.uint8, device=device) if split else None
        if workspace is not None:
            keep.append(workspace)
        fn = lib.fn[f"attention_bwd_{kind}_ws"]
        args = (*args, workspace.data_ptr() if workspace is not None else None,
                size.value if workspace is not None else 0)
        configuration += (("split", split), ("workspace_bytes", size.value if workspace is not None else 0))
        op = OP_ATTENTION_BWD_DQ if kind == "dq" else OP_ATTENTION_BWD_DKDV
        # The kernel variant depends on the rows of the call: batch x query heads x queries for dQ,
        # batch x key heads x keys for dK/dV.
        rows = batch * q_heads * sq if kind == "dq" else batch * (q_heads // group) * sk
        return Launch(f"intent_hip_attention_bwd_{kind}", lambda stream: fn(*args, stream), tuple(keep),
                      tuple(before), tuple(after), configuration,
                      lambda: lib.kernel_resources(op, F16, rows, d), candidates)
    return plan


# ------------------------------------------------------------------------------ paged decode
def _positive_constexpr(constexprs, name):
    value = constexprs[name]
    if isinstance(value, bool) or not isinstance(value, int) or value < 1:
        raise CompilationStageError("provider_configuration", f"{name} must be a positive int, got {value!r}")
    return value


def _paged_decode_partials(lib, bound, constexprs, device):
    """paged_gqa_decode_partials: one workgroup per (job, key head). The page tables are read as
    given; positions and physical pages outside their arrays are clamped by the kernel."""
    (q, key_cache, value_cache, page_offsets, page_indices, lengths, split_offsets, partial_lse, partial_output,
     scale) = bound.arguments
    page_size = _positive_constexpr(constexprs, "PAGE_SIZE")
    group = _positive_constexpr(constexprs, "HEAD_GROUP")
    splits = _positive_constexpr(constexprs, "SPLITS")
    batch, q_heads, d = q.shape
    pages, ps, kv_heads, dv = value_cache.shape
    if page_offsets.shape[0] != batch + 1:
        raise ValueError(f"page_offsets must hold batch + 1 = {batch + 1} entries, got {page_offsets.shape[0]}")
    if split_offsets.shape[0] != batch * splits + 1:
        raise ValueError(f"split_offsets must hold batch * SPLITS + 1 = {batch * splits + 1} entries, "
                         f"got {split_offsets.shape[0]}")
    if kv_heads * group != q_heads:
        raise ValueError(f"query heads ({q_heads}) must equal key/value heads ({kv_heads}) * HEAD_GROUP ({group})")
    keep = [q, key_cache, value_cache, page_offsets, page_indices, lengths, split_offsets, partial_lse,
            partial_output]
    before, after = [], []
    qk = _readable(q, keep, before)
    kk, vk = _readable(key_cache, keep, before, 8), _readable(value_cache, keep, before, 8)
    tables = [_readable(t, keep, before) for t in (page_offsets, page_indices, lengths, split_offsets)]
    ok = _writable(partial_output, keep, after)
    strides = _strides(qk, kk, vk, partial_lse, ok)
    keep.append(strides)
    fn = lib.fn["paged_decode_partials"]
    args = (qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), *(t.data_ptr() for t in tables), partial_lse.data_ptr(),
            ok.data_ptr(), batch, q_heads, d, pages, ps, kv_heads, dv, page_indices.shape[0], page_size, group,
            splits, strides, float(scale))
    return Launch("intent_hip_paged_decode_partials", lambda stream: fn(*args, stream), tuple(keep), tuple(before),
                  tuple(after),
                  (("batch", batch), ("q_heads", q_heads), ("kv_heads", kv_heads), ("head_group", group),
                   ("d", d), ("pages", pages), ("ps", ps), ("page_size", page_size), ("splits", splits)),
                  lambda: lib.kernel_resources(OP_PAGED_DECODE_PARTIALS, F16, group, d))


def _grouped_decode_partials(lib, bound, constexprs, device):
    """grouped_flash_decode_partials: one workgroup per (batch, part, key head) over the bf16 caches."""
    q, k, v, partial_lse, partial_output, scale = bound.arguments
    group = _positive_constexpr(constexprs, "HEAD_GROUP")
    parts = _positive_constexpr(constexprs, "P")
    split = _positive_constexpr(constexprs, "SPLIT_SIZE")
    batch, q_heads, _, d = q.shape
    kv_heads, keys, dv = k.shape[1], k.shape[2], v.shape[3]
    if partial_lse.shape[2] != parts:
        raise ValueError(f"partial_lse holds {partial_lse.shape[2]} parts, P is {parts}")
    if kv_heads * group != q_heads:
        raise ValueError(f"query heads ({q_heads}) must equal key/value heads ({kv_heads}) * HEAD_GROUP ({group})")
    keep, before, after = [q, k, v, partial_lse, partial_output], [], []
    qk, kk, vk = _readable(q, keep, before), _readable(k, keep, before, 8), _readable(v, keep, before, 8)
    lk, ok = _writable(partial_lse, keep, after), _writable(partial_output, keep, after)
    strides = _strides(qk, kk, vk, lk, ok)
    keep.append(strides)
    fn = lib.fn["grouped_decode_partials"]
    args = (qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), lk.data_ptr(), ok.data_ptr(), batch, q_heads, kv_heads, group,
            keys, d, dv, parts, split, strides, float(scale))
    return Launch("intent_hip_grouped_decode_partials", lambda stream: fn(*args, stream), tuple(keep), tuple(before),
                  tuple(after), (("batch", batch), ("q_heads", q_heads), ("kv_heads", kv_heads), ("keys", keys),
                                 ("d", d), ("parts", parts), ("split_size", split)),
                  lambda: lib.kernel_resources(OP_GROUPED_DECODE_PARTIALS, BF16, group, d))


def _decode_workspace(name):
    if _static_workspace():
        raise CompilationStageError(
            "provider_preparation", f"{name} merges split states through a workspace; backend_options "
            "workspace='static' has none for it, use workspace='prepare'")


def _continuous_decode(lib, bound, constexprs, device):
    """continuous_gqa_decode: the keys split over (batch, split, key head) workgroups whose states
    merge in a second kernel, through a workspace allocated here."""
    import ctypes

    import torch

    q, k, v, mask, output, scale = bound.arguments
    group = _positive_constexpr(constexprs, "HEAD_GROUP")
    batch, q_heads, d = q.shape
    keys, kv_heads, dv = k.shape[1], k.shape[2], v.shape[3]
    if kv_heads * group != q_heads:
        raise ValueError(f"query heads ({q_heads}) must equal key/value heads ({kv_heads}) * HEAD_GROUP ({group})")
    _decode_workspace("continuous_gqa_decode")
    keep, before, after = [q, k, v, mask, output], [], []
    qk, kk, vk = _readable(q, keep, before), _readable(k, keep, before, 8), _readable(v, keep, before, 8)
    mk, ok = _readable(mask, keep, before), _writable(output, keep, after)
    strides = _strides(qk, kk, vk, mk, ok)
    size = ctypes.c_size_t(0)
    lib.check(lib.fn["dense_decode_workspace_bytes"](batch, q_heads, kv_heads, keys, dv, ctypes.byref(size)),
              "provider_preparation")
    workspace = torch.empty(max(size.value, 1), dtype=torch.uint8, device=device)
    keep += [strides, workspace]
    fn = lib.fn["continuous_gqa_decode"]
    args = (qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), mk.data_ptr(), ok.data_ptr(), batch, q_heads, kv_heads, group,
            keys, d, dv, strides, float(scale), workspace.data_ptr(), size.value)
    return Launch("intent_hip_continuous_gqa_decode", lambda stream: fn(*args, stream), tuple(keep), tuple(before),
                  tuple(after), (("batch", batch), ("q_heads", q_heads), ("kv_heads", kv_heads), ("keys", keys),
                                 ("d", d), ("workspace_bytes", size.value)),
                  lambda: lib.kernel_resources(OP_CONTINUOUS_DECODE, F16, group, d))


def _varlen_decode(lib, bound, constexprs, device):
    """varlen_gqa_decode_with_sink_logits: packed sequences split over (sequence, split, key head)
    workgroups; the merge adds the sink and turns the block maxima (kept in block_logits) into
    block logits. The offsets stay on the device."""
    import ctypes

    import torch

    q, k, v, cu, sink, output, block_logits, scale = bound.arguments
    group = _positive_constexpr(constexprs, "HEAD_GROUP")
    max_blocks = _positive_constexpr(constexprs, "MAX_BLOCKS")
    sequences, q_heads, d = q.shape
    rows, kv_heads, dv = k.shape[0], k.shape[1], v.shape[2]
    if kv_heads * group != q_heads:
        raise ValueError(f"query heads ({q_heads}) must equal key/value heads ({kv_heads}) * HEAD_GROUP ({group})")
    if cu.shape[0] != sequences + 1:
        raise ValueError(f"cu_seqlens needs q.shape[0] + 1 = {sequences + 1} entries, got {cu.shape[0]}")
    if max_blocks > block_logits.shape[2]:
        raise ValueError(f"MAX_BLOCKS ({max_blocks}) exceeds the {block_logits.shape[2]} block_logits columns")
    _decode_workspace("varlen_gqa_decode_with_sink_logits")
    keep, before, after = [q, k, v, cu, sink, output, block_logits], [], []
    qk, kk, vk = _readable(q, keep, before), _readable(k, keep, before, 8), _readable(v, keep, before, 8)
    cuk, sk = _readable(cu, keep, before), _readable(sink, keep, before)
    ok, bk = _writable(output, keep, after), _writable(block_logits, keep, after)
    strides = _strides(qk, kk, vk, ok, bk)
    size = ctypes.c_size_t(0)
    lib.check(lib.fn["varlen_decode_workspace_bytes"](sequences, q_heads, kv_heads, max_blocks, dv,
                                                      ctypes.byref(size)), "provider_preparation")
    workspace = torch.empty(max(size.value, 1), dtype=torch.uint8, device=device)
    keep += [strides, workspace]
    fn = lib.fn["varlen_decode_sink"]
    args = (qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), cuk.data_ptr(), sk.data_ptr(), ok.data_ptr(), bk.data_ptr(),
            sequences, rows, q_heads, kv_heads, group, d, dv, max_blocks, strides, float(scale),
            workspace.data_ptr(), size.value)
    return Launch("intent_hip_varlen_decode_sink", lambda stream: fn(*args, stream), tuple(keep), tuple(before),
                  tuple(after), (("sequences", sequences), ("rows", rows), ("q_heads", q_heads),
                                 ("kv_heads", kv_heads), ("d", d), ("max_blocks", max_blocks),
                                 ("workspace_bytes", size.value)),
                  lambda: lib.kernel_resources(OP_VARLEN_DECODE, F16, group, d))


def _splitk_reduce(lib, bound, constexprs, device):
    partial, lse, output = bound.arguments
    keep, before, after = [partial, lse, output], [], []
    pk, outk = _readable(partial, keep, before), _writable(output, keep, after)
    batch, heads, splits, d = partial.shape
    strides = _strides(pk, lse, outk)
    keep.append(strides)
    fn = lib.fn["splitk_reduce_f32_to_f16"]
    args = (pk.data_ptr(), lse.data_ptr(), outk.data_ptr(), batch, heads, splits, d, strides)
    return Launch("intent_hip_splitk_reduce_f32_to_f16", lambda stream: fn(*args, stream), tuple(keep),
                  tuple(before), tuple(after),
                  (("batch", batch), ("heads", heads), ("splits", splits), ("d", d)),
                  lambda: lib.kernel_resources(OP_SPLITK_REDUCE, F32, batch * heads, d))


# ------------------------------------------------------------------------------ SpMV
def _csr_spmv(lib, bound, constexprs, device):
    import ctypes

    import torch

    offsets, columns, values, vector, output = bound.arguments
    rows = offsets.shape[0] - 1
    if rows < 0 or output.shape[0] != rows:
        raise ValueError("csr_spmv requires row_offsets.shape[0] == output.shape[0] + 1")
    if columns.shape[0] != values.shape[0]:
        raise ValueError("csr_spmv requires column_indices and values of equal length")
    keep, before, after = [offsets, columns, values, vector, output], [], []
    ok, ck, vk, xk, yk = (_readable(offsets, keep, before), _readable(columns, keep, before),
                          _readable(values, keep, before), _readable(vector, keep, before),
                          _writable(output, keep, after))
    nnz, cols = values.shape[0], vector.shape[0]
    size = ctypes.c_size_t(0)
    lib.check(lib.fn["csr_spmv_workspace_bytes"](rows, nnz, ctypes.byref(size)), "provider_preparation")
    pointers = (ok.data_ptr(), ck.data_ptr(), vk.data_ptr(), xk.data_ptr(), yk.data_ptr(), rows, cols, nnz)
    facts = (("rows", rows), ("cols", cols), ("nnz", nnz), ("workspace_bytes", size.value))
    if _static_workspace():
        if size.value > STATIC_SCRATCH_BYTES:
            raise CompilationStageError(
                "provider_preparation", f"csr_spmv of {rows} rows and {nnz} nonzeros needs {size.value} workspace "
                f"bytes, beyond the {STATIC_SCRATCH_BYTES}-byte static scratch; use workspace='prepare'")
        fn, entry = lib.fn["csr_spmv_f32_static"], "intent_hip_csr_spmv_f32_static"
        args = pointers
        facts += (("workspace", "static"),)
    else:
        workspace = torch.empty(max(size.value, 1), dtype=torch.uint8, device=device)
        keep.append(workspace)
        fn, entry = lib.fn["csr_spmv_f32"], "intent_hip_csr_spmv_f32"
        args = (*pointers, workspace.data_ptr(), size.value)
    return Launch(entry, lambda stream: fn(*args, stream), tuple(keep), tuple(before), tuple(after), facts,
                  lambda: lib.kernel_resources(OP_CSR_SPMV_F32, F32, rows, nnz))


def _csr_spmm(lib, bound, constexprs, device):
    """csr_spmm: rows read through their own strides (unit inner stride required, staged otherwise)."""
    offsets, columns, values, dense, output = bound.arguments
    rows = offsets.shape[0] - 1
    if rows < 0 or output.shape[0] != rows:
        raise ValueError("csr_spmm requires row_offsets.shape[0] == output.shape[0] + 1")
    if columns.shape[0] != values.shape[0]:
        raise ValueError("csr_spmm requires column_indices and values of equal length")
    if dense.shape[1] != output.shape[1]:
        raise ValueError("csr_spmm requires dense and output of equal feature width")
    keep, before, after = [offsets, columns, values, dense, output], [], []
    ok, ck, vk = (_readable(offsets, keep, before), _readable(columns, keep, before), _readable(values, keep, before))
    dk, outk = _readable(dense, keep, before), _writable(output, keep, after)
    nnz, cols, features = values.shape[0], dense.shape[0], dense.shape[1]
    fn = lib.fn["csr_spmm_f32"]
    args = (ok.data_ptr(), ck.data_ptr(), vk.data_ptr(), dk.data_ptr(), outk.data_ptr(), rows, cols, nnz, features,
            _row_stride(dk) if cols else features, _row_stride(outk) if rows else features)
    return Launch("intent_hip_csr_spmm_f32", lambda stream: fn(*args, stream), tuple(keep), tuple(before),
                  tuple(after), (("rows", rows), ("cols", cols), ("nnz", nnz), ("features", features)),
                  lambda: lib.kernel_resources(OP_CSR_SPMM_F32, F32, rows, features))


_SPECS = (
    OperatorSpec("stable_softmax", (_view(IN, "f32", 2), _view(OUT, "f32", 2)), (), _softmax_fwd(F32), True),
    OperatorSpec("stable_softmax_f16", (_view(IN, "f16", 2), _view(OUT, "f16", 2)), (), _softmax_fwd(F16), True),
    OperatorSpec("chunked_softmax_bf16", (_view(IN, "bf16", 2), _view(OUT, "bf16", 2)), (), _softmax_fwd(BF16),
                 True),
    OperatorSpec("softmax_backward", (_view(IN, "f32", 2), _view(IN, "f32", 2), _view(OUT, "f32", 2)), (),
                 _softmax_bwd(F32), True),
    OperatorSpec("softmax_backward_f16", (_view(IN, "f16", 2), _view(IN, "f16", 2), _view(OUT, "f16", 2)), (),
                 _softmax_bwd(F16), True),
    OperatorSpec("gemm_f32", (_view(IN, "f32", 2), _view(IN, "f32", 2), _view(OUT, "f32", 2)), (),
                 _gemm_f32(False)),
    OperatorSpec("linear_f32", (_view(IN, "f32", 2), _view(IN, "f32", 2), _view(OUT, "f32", 2)), (),
                 _gemm_f32(True)),
    OperatorSpec("gemm_i8", (_view(IN, "i8", 2), _view(IN, "i8", 2), _view(IN, "i32", 1), _view(OUT, "i32", 2)), (),
                 _gemm_i8),
    OperatorSpec("gemm", (_view(IN, "f16", 2), _view(IN, "f16", 2), _view(OUT, "f16", 2)), ("ACTIVATION",),
                 _gemm16(F16)),
    OperatorSpec("quantized_gemm", (_view(IN, "f16", 2), _view(IN, "f16", 2), _view(IN, "f32", 1), _view(IN, "f16", 2),
                                    _view(IN, "f32", 1), _view(OUT, "i8", 2)), (), _quantized_gemm),
    OperatorSpec("bf16_gemm", (_view(IN, "bf16", 2), _view(IN, "bf16", 2), _view(OUT, "bf16", 2)), (),
                 _gemm_bf16),
    OperatorSpec("flash_attention_fwd", (_view(IN, "f16", 4), _view(IN, "f16", 4), _view(IN, "f16", 4),
                                         _view(OUT, "f16", 4), ("scalar", "f32")), ("CAUSAL",), _attention_f16),
    OperatorSpec("flash_gqa_attention_fwd", (_view(IN, "f16", 4), _view(IN, "f16", 4), _view(IN, "f16", 4),
                                             _view(OUT, "f16", 4), ("scalar", "f32")), ("HEAD_GROUP", "CAUSAL"),
                 _attention_grouped(F16)),
    OperatorSpec("flash_attention_bf16_fwd", (_view(IN, "bf16", 4), _view(IN, "bf16", 4), _view(IN, "bf16", 4),
                                              _view(OUT, "bf16", 4), ("scalar", "f32")), ("HEAD_GROUP", "CAUSAL"),
                 _attention_grouped(BF16)),
    OperatorSpec("mla_prefill", (_view(IN, "f16", 4), _view(IN, "f16", 4), _view(IN, "f16", 4), _view(IN, "f16", 4),
                                 _view(IN, "f16", 4), _view(OUT, "f16", 4), ("scalar", "f32")), ("HEAD_GROUP",),
                 _mla_prefill),
    OperatorSpec("flash_attention_bias_fwd", (_view(IN, "f16", 4), _view(IN, "f16", 4), _view(IN, "f16", 4),
                                              _view(IN, "f32", 3), _view(OUT, "f16", 4), ("scalar", "f32")), (),
                 _attention_bias),
    OperatorSpec("flash_varlen_attention_fwd",
                 (_view(IN, "f16", 2), _view(IN, "f16", 2), _view(IN, "f16", 2), _view(IN, "i32", 1),
                  _view(IN, "i32", 1), _view(OUT, "f16", 2), ("scalar", "f32")), ("CAUSAL",),
                 _attention_varlen(False)),
    OperatorSpec("flash_varlen_gqa_prefill",
                 (_view(IN, "f16", 3), _view(IN, "f16", 3), _view(IN, "f16", 3), _view(IN, "i32", 1),
                  _view(IN, "i32", 1), _view(OUT, "f16", 3), ("scalar", "f32")), ("HEAD_GROUP",),
                 _attention_varlen(True)),
    OperatorSpec("attention_backward_delta", (_view(IN, "f16", 4), _view(IN, "f16", 4), _view(OUT, "f32", 3)), (),
                 _attention_bwd_delta),
    OperatorSpec("attention_backward_dkdv",
                 (_view(IN, "f16", 4), _view(IN, "f16", 4), _view(IN, "f16", 4), _view(IN, "f16", 4),
                  _view(IN, "f32", 3), _view(IN, "f32", 3), _view(OUT, "f16", 4), _view(OUT, "f16", 4),
                  ("scalar", "f32")), ("HEAD_GROUP", "CAUSAL"), _attention_bwd("dkdv")),
    OperatorSpec("attention_backward_dq",
                 (_view(IN, "f16", 4), _view(IN, "f16", 4), _view(IN, "f16", 4), _view(IN, "f16", 4),
                  _view(IN, "f32", 3), _view(IN, "f32", 3), _view(OUT, "f16", 4), ("scalar", "f32")),
                 ("HEAD_GROUP", "CAUSAL"), _attention_bwd("dq")),
    OperatorSpec("paged_gqa_decode_partials",
                 (_view(IN, "f16", 3), _view(IN, "f16", 4), _view(IN, "f16", 4), _view(IN, "i32", 1),
                  _view(IN, "i32", 1), _view(IN, "i32", 1), _view(IN, "i32", 1), _view(OUT, "f32", 3),
                  _view(OUT, "f32", 4), ("scalar", "f32")), ("PAGE_SIZE", "HEAD_GROUP", "SPLITS"),
                 _paged_decode_partials),
    OperatorSpec("grouped_flash_decode_partials",
                 (_view(IN, "bf16", 4), _view(IN, "bf16", 4), _view(IN, "bf16", 4), _view(OUT, "f32", 3),
                  _view(OUT, "bf16", 4), ("scalar", "f32")), ("HEAD_GROUP", "P", "SPLIT_SIZE"),
                 _grouped_decode_partials),
    OperatorSpec("continuous_gqa_decode",
                 (_view(IN, "f16", 3), _view(IN, "f16", 4), _view(IN, "f16", 4), _view(IN, "u8", 3),
                  _view(OUT, "f16", 3), ("scalar", "f32")), ("HEAD_GROUP",), _continuous_decode),
    OperatorSpec("varlen_gqa_decode_with_sink_logits",
                 (_view(IN, "f16", 3), _view(IN, "f16", 3), _view(IN, "f16", 3), _view(IN, "i32", 1),
                  _view(IN, "f32", 1), _view(OUT, "f16", 3), _view(OUT, "f32", 3), ("scalar", "f32")),
                 ("HEAD_GROUP", "MAX_BLOCKS"), _varlen_decode),
    OperatorSpec("splitk_attention_f32_to_f16_reduce", (_view(IN, "f32", 4), _view(IN, "f32", 3),
                                                        _view(OUT, "f16", 3)), (), _splitk_reduce),
    OperatorSpec("csr_spmm", (_view(IN, "i32", 1), _view(IN, "i32", 1), _view(IN, "f32", 1), _view(IN, "f32", 2),
                              _view(OUT, "f32", 2)), (), _csr_spmm, derived=(("R", "R1", -1),)),
    OperatorSpec("csr_spmv", (_view(IN, "i32", 1), _view(IN, "i32", 1), _view(IN, "f32", 1), _view(IN, "f32", 1),
                              _view(OUT, "f32", 1)), (), _csr_spmv, derived=(("R", "R1", -1),)),
)

SPECS = {spec.name: spec for spec in _SPECS}

ENTRY_POINTS = {
    "stable_softmax": "intent_hip_softmax_fwd", "stable_softmax_f16": "intent_hip_softmax_fwd",
    "chunked_softmax_bf16": "intent_hip_softmax_fwd", "softmax_backward": "intent_hip_softmax_bwd",
    "softmax_backward_f16": "intent_hip_softmax_bwd", "gemm_f32": "intent_hip_gemm_f32",
    "linear_f32": "intent_hip_gemm_f32", "gemm_i8": "intent_hip_gemm_i8", "gemm": "intent_hip_gemm",
    "quantized_gemm": "intent_hip_quantized_gemm", "bf16_gemm": "intent_hip_gemm_bf16",
    "flash_attention_fwd": "intent_hip_attention_fwd_f16", "flash_gqa_attention_fwd": "intent_hip_attention_fwd",
    "flash_attention_bf16_fwd": "intent_hip_attention_fwd", "mla_prefill": "intent_hip_mla_prefill",
    "flash_attention_bias_fwd": "intent_hip_attention_bias_fwd",
    "flash_varlen_attention_fwd": "intent_hip_attention_varlen_fwd",
    "flash_varlen_gqa_prefill": "intent_hip_attention_varlen_fwd",
    "attention_backward_delta": "intent_hip_attention_bwd_delta",
    "attention_backward_dkdv": "intent_hip_attention_bwd_dkdv", "attention_backward_dq": "intent_hip_attention_bwd_dq",
    "paged_gqa_decode_partials": "intent_hip_paged_decode_partials",
    "grouped_flash_decode_partials": "intent_hip_grouped_decode_partials",
    "continuous_gqa_decode": "intent_hip_continuous_gqa_decode",
    "varlen_gqa_decode_with_sink_logits": "intent_hip_varlen_decode_sink",
    "splitk_attention_f32_to_f16_reduce": "intent_hip_splitk_reduce_f32_to_f16",
    "csr_spmm": "intent_hip_csr_spmm_f32", "csr_spmv": "intent_hip_csr_spmv_f32",
}
assert set(ENTRY_POINTS) == set(SPECS)


def signature_of(interface) -> tuple:
    from ..interface import ViewParameter

    return tuple(("view", int(p.access), p.dtype.name, p.rank) if isinstance(p, ViewParameter)
                 else ("scalar", p.dtype.name) for p in interface.parameters)


def recognize(definition, interface, constexpr_names: tuple[str, ...]) -> OperatorSpec:
    name = getattr(definition, "__name__", None)
    spec = SPECS.get(name)
    if spec is None:
        raise CompilationStageError(
            "provider_recognition", f"the hip provider has no kernel for definition {name!r}; "
            f"supported: {', '.join(sorted(SPECS))}")
    if signature_of(interface) != spec.signature or tuple(constexpr_names) != spec.constexprs:
        raise CompilationStageError(
            "provider_recognition", f"definition {name!r} does not have the signature the hip kernel implements: "
            f"expected {spec.signature} with constexprs {spec.constexprs}, got {signature_of(interface)} "
            f"with constexprs {tuple(constexpr_names)}")
    return spec


def recognize_saved(name: str, signature: tuple, constexpr_names: tuple[str, ...]) -> OperatorSpec:
    """Recognition of a saved program (no definition object): by name, signature and constexprs."""
    spec = SPECS.get(name)
    if spec is None or tuple(signature) != spec.signature or tuple(constexpr_names) != spec.constexprs:
        raise CompilationStageError("provider_recognition",
                                    f"saved program {name!r} does not match a kernel of this hip provider")
    return spec
