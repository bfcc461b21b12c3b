"""CPU oracle of the hip provider — TEST INFRASTRUCTURE ONLY.

Only tests/, `__graft_entry__.smoke()` and bench.py's CPU-baseline leg may use
this package; `intent_amd` never imports it.

Parity status of each function (how it is pinned; see tests/test_oracle.py):
  softmax_fwd  f32/f16/bf16  pinned: golden vectors (numpy float64 closed form), torch float64
                              softmax, invariants (row sum, shift invariance), exact special
                              cases (constant rows, one-hot, -inf entries, NaN rows).
  softmax_bwd  f32/f16       pinned: golden vectors, torch.autograd float64 JVP, exact zero for
                              constant dy, row-sum invariant.
  gemm_bf16                  pinned: golden vectors, exact small-integer products (bit-exact),
                              identity/permutation matrices, torch float64 matmul.
  gemm16 (f16, relu; bf16)   pinned: golden vectors (numpy float64 of the rounded operands),
                              exact small-integer products, ReLU against numpy on the exact
                              results, NaN propagation and +0 for negative sums, equality with
                              gemm_bf16 for bf16 operands.
  gemm_f32 / linear          pinned: golden vectors (numpy float64), exact small-integer
                              products, linear(x, W) == gemm(x, W^T) bit for bit, identity.
  attention_fwd (f16/bf16,   pinned: golden vectors (float64 grouped-head attention), grouped heads
    head_group)               equal to the ungrouped function on repeated K/V (bit for bit),
                              bf16 first causal row = v[0], f16 path equal to attention_fwd_f16.
  attention_fwd_f16          pinned: golden vectors (float64 causal softmax attention), exact
                              first causal row (= v[0]), Q = 0 prefix means, chunk-size
                              independence within tolerance, torch SDPA float32.
  csr_spmv_f32               pinned: golden vectors (scipy float64), bit-exact probes (ones ->
                              row lengths; one-hot x -> a column; small integers), strict
                              left-fold restatement in numpy.
  half/bf16 conversions      pinned: exhaustive against numpy float16 / torch bfloat16.
"""
from .oracle import *  # noqa: F401,F403
