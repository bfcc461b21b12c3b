"""Dense GEMM definitions (interface of the reference's
`python/intent/examples/kernels/contraction/gemm.py:10-121`): gemm_f32, linear_f32, gemm_i8 (int8
operands, int32 accumulator and bias), the f16 `gemm` with its ACTIVATION constexpr, bf16_gemm,
and quantized_gemm (f16 operands, int8 output through a bias, ReLU, residual and scale)."""
import intent_amd as intent
import intent_amd.language as I

# The reference's example extents (contraction/gemm.py:5-7), kept as module constants for callers
# that import them; the definitions below take any extents.
M = 4096
K = 4096
N = 14336


class Activation(I.Enum):
    """Epilogue activation of `gemm` (gemm.py:10-12)."""

    NONE = 0
    RELU = 1


@intent.kernel
def gemm_f32(
    a: I.In[I.f32, ("M", "K")],
    b: I.In[I.f32, ("K", "N")],
    c: I.Out[I.f32, ("M", "N")],
):
    M, K = a.shape
    _, N = b.shape
    m, n, k = I.domain(0, M), I.domain(0, N), I.domain(0, K)
    c[m, n] = I.matmul(a[m, k], b[k, n], acc_dtype=I.f32)


@intent.kernel
def linear_f32(
    x: I.In[I.f32, ("M", "K")],
    weight: I.In[I.f32, ("N", "K")],
    output: I.Out[I.f32, ("M", "N")],
):
    m, n, k = I.domain(0, x.shape[0]), I.domain(0, weight.shape[0]), I.domain(0, x.shape[1])
    output[m, n] = I.matmul(x[m, k], weight[n, k], transpose_rhs=True, acc_dtype=I.f32)


@intent.kernel
def gemm_i8(
    a: I.In[I.i8, ("M", "K")],
    b: I.In[I.i8, ("K", "N")],
    bias: I.In[I.i32, ("N",)],
    c: I.Out[I.i32, ("M", "N")],
):
    m, n, k = I.domain(0, a.shape[0]), I.domain(0, b.shape[1]), I.domain(0, a.shape[1])
    c[m, n] = I.matmul(a[m, k], b[k, n], acc_dtype=I.i32) + bias[n]


@intent.kernel
def gemm(
    a: I.In[I.f16, ("M", "K")],
    b: I.In[I.f16, ("K", "N")],
    c: I.Out[I.f16, ("M", "N")],
    ACTIVATION: I.Constexpr[Activation],
):
    M, K = a.shape
    _, N = b.shape
    m, n, k = I.domain(0, M), I.domain(0, N), I.domain(0, K)
    accumulator = I.matmul(a[m, k], b[k, n], acc_dtype=I.f32)
    if ACTIVATION == Activation.RELU:
        accumulator = I.maximum(accumulator, 0.0)
    c[m, n] = I.cast(accumulator, I.f16)


@intent.kernel
def bf16_gemm(
    a: I.In[I.bf16, ("M", "K")],
    b: I.In[I.bf16, ("K", "N")],
    c: I.Out[I.bf16, ("M", "N")],
):
    M, K = a.shape
    _, N = b.shape
    m, n, k = I.domain(0, M), I.domain(0, N), I.domain(0, K)
    c[m, n] = I.cast(I.matmul(a[m, k], b[k, n], acc_dtype=I.f32), I.bf16)


@intent.kernel
def quantized_gemm(
    a: I.In[I.f16, ("M", "K")],
    b: I.In[I.f16, ("K", "N")],
    bias: I.In[I.f32, ("N",)],
    residual: I.In[I.f16, ("M", "N")],
    output_scale: I.In[I.f32, ("N",)],
    output: I.Out[I.i8, ("M", "N")],
):
    m, n, k = I.domain(0, a.shape[0]), I.domain(0, b.shape[1]), I.domain(0, a.shape[1])
    summed = I.matmul(a[m, k], b[k, n], acc_dtype=I.f32)
    rectified = I.maximum(summed + bias[n], 0.0) + I.cast(residual[m, n], I.f32)
    output[m, n] = I.cast(I.minimum(I.maximum(rectified / output_scale[n], -128.0), 127.0), I.i8)
