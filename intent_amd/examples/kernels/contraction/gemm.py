"""Dense GEMM definitions (interface of the reference's
`python/intent/examples/kernels/contraction/gemm.py:76-92`)."""
import intent_amd as intent
import intent_amd.language as I


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
