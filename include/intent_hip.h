/*
 * intent_hip.h — C ABI of libintent_hip.so, the native side of the `hip` provider.
 *
 * The reference has no native ABI for these operators: each one is a Triton
 * kernel generated at run time and launched from Python
 * (python/intent/runtime/triton/program.py:291-389, launched by
 * python/intent/runtime/block/program.py:66-82). Every entry point below replaces
 * that launch for one `intent.examples` definition; the definition it serves is
 * cited on each declaration.
 *
 * Conventions (all entry points):
 *   - return an int status: INTENT_HIP_OK (0) or one of the codes below;
 *     intent_hip_status_string() names a code, intent_hip_last_error() gives the
 *     calling thread's detail message of the last failure;
 *   - every pointer is a device pointer owned by the caller; extents and strides are
 *     in elements; the innermost stride of every tensor is 1;
 *   - the launch is asynchronous on `stream` (a hipStream_t; NULL = default stream);
 *     nothing is allocated, nothing is synchronised;
 *   - calls are stateless and thread-safe.
 */
#ifndef INTENT_HIP_H
#define INTENT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define INTENT_HIP_ABI_VERSION 17

enum IntentHipStatus {
  INTENT_HIP_OK = 0,
  INTENT_HIP_ERR_INVALID_ARGUMENT = 1, /* bad extent, stride, alignment or dtype code */
  INTENT_HIP_ERR_UNSUPPORTED = 2,      /* valid request this build does not implement */
  INTENT_HIP_ERR_LAUNCH = 3,           /* the HIP runtime rejected the launch */
  INTENT_HIP_ERR_DEVICE = 4,           /* device query failed */
  INTENT_HIP_ERR_WORKSPACE = 5         /* workspace missing or too small */
};

enum IntentHipDtype { INTENT_HIP_F32 = 0, INTENT_HIP_F16 = 1, INTENT_HIP_BF16 = 2 };

/* Operator codes for intent_hip_kernel_resources(). */
enum IntentHipOperator {
  INTENT_HIP_OP_SOFTMAX_FWD = 0,
  INTENT_HIP_OP_SOFTMAX_BWD = 1,
  INTENT_HIP_OP_GEMM_BF16 = 2,
  INTENT_HIP_OP_ATTENTION_FWD_F16 = 3,
  INTENT_HIP_OP_CSR_SPMV_F32 = 4,
  INTENT_HIP_OP_GEMM = 5,              /* dtype F16 or BF16 */
  INTENT_HIP_OP_GEMM_F32 = 6,
  INTENT_HIP_OP_ATTENTION_FWD = 7,     /* dtype F16 or BF16; for both forward ops cols = d, or d | dv << 16 */
  INTENT_HIP_OP_ATTENTION_BWD_DELTA = 8, /* cols = head dimension */
  INTENT_HIP_OP_ATTENTION_BWD_DQ = 9,    /* rows = batch * query heads * queries, cols = head dimension */
  INTENT_HIP_OP_ATTENTION_BWD_DKDV = 10, /* rows = batch * key heads * keys, cols = head dimension */
  INTENT_HIP_OP_PAGED_DECODE_PARTIALS = 11, /* rows = HEAD_GROUP, cols = head dimension */
  INTENT_HIP_OP_SPLITK_REDUCE = 12,
  INTENT_HIP_OP_CSR_SPMM_F32 = 13,        /* cols = features */
  INTENT_HIP_OP_ATTENTION_VARLEN = 14,    /* packed sequences; dtype F16 or BF16, cols = d | dv << 16 */
  INTENT_HIP_OP_GEMM_I8 = 15,
  INTENT_HIP_OP_QUANTIZED_GEMM = 16,
  INTENT_HIP_OP_ATTENTION_BIAS = 17,      /* f16; cols = d | dv << 16 */
  INTENT_HIP_OP_GROUPED_DECODE_PARTIALS = 18, /* rows = HEAD_GROUP, cols = head dimension */
  INTENT_HIP_OP_CONTINUOUS_DECODE = 19,   /* rows = HEAD_GROUP, cols = head dimension */
  INTENT_HIP_OP_VARLEN_DECODE = 20,       /* rows = HEAD_GROUP, cols = head dimension */
  INTENT_HIP_OP_DECODE_MERGE = 21,        /* cols = head dimension */
  INTENT_HIP_OP_MLA_PREFILL = 22          /* cols = D | P << 16 */
};

/* Epilogue activations of intent_hip_gemm (the Activation enum of contraction/gemm.py:10-12). */
enum IntentHipActivation { INTENT_HIP_ACT_NONE = 0, INTENT_HIP_ACT_RELU = 1 };

struct IntentHipDeviceInfo {
  char arch[64];               /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int32_t compute_units;
  int32_t wavefront_size;
  int64_t lds_per_workgroup;   /* bytes */
  int64_t global_memory_bytes;
  int32_t clock_khz;
  int32_t memory_clock_khz;
  int32_t memory_bus_width;    /* bits */
  int32_t l2_bytes;
};

struct IntentHipKernelResources {
  char kernel[128];            /* name of the kernel the selected variant launches */
  int32_t vgprs;               /* architectural + accumulation VGPRs per lane, when reported */
  int32_t lds_bytes;           /* static LDS per workgroup */
  int32_t scratch_bytes;       /* private (spill) bytes per lane */
  int32_t max_threads_per_block;
  int32_t block_threads;       /* threads per workgroup of the launch */
};

int intent_hip_abi_version(void);
const char *intent_hip_status_string(int status);
const char *intent_hip_last_error(void);

int intent_hip_device_count(int *count);
/* Replaces the CUDA driver queries of python/intent/targets/nvidia/device.py:6 (target facts). */
int intent_hip_device_info(int device, struct IntentHipDeviceInfo *out);

/* Facts of the kernel a call with these extents would launch (observation,
 * python/intent/runtime/diagnostics.py:23-145; python/intent/runtime/triton/cuda.py:46-57). */
int intent_hip_kernel_resources(int op, int dtype, int64_t rows, int64_t cols,
                                struct IntentHipKernelResources *out);

/* Row softmax forward, y[r,:] = softmax(x[r,:]).
 * dtype F32: stable_softmax            (python/intent/examples/kernels/normalization/softmax.py:23-36)
 *            y = exp(x - max) * (1 / sum)
 * dtype F16: stable_softmax_f16        (softmax.py:39-51)   y = f16(exp(x - max) / sum), f32 math
 * dtype BF16: chunked_softmax_bf16     (softmax.py:54-66)   y = bf16(exp(x - max) / sum), f32 math
 * max is maximum_num (a one-sided NaN is ignored; softmax.py:12-20). */
int intent_hip_softmax_fwd(int dtype, const void *x, void *y, int64_t rows, int64_t cols,
                           int64_t x_row_stride, int64_t y_row_stride, void *stream);

/* Row softmax backward, dx = p * (dy - sum(p * dy)), f32 accumulation.
 * dtype F32: softmax_backward (python/intent/examples/kernels/backward/softmax.py:9-25);
 * dtype F16: softmax_backward_f16, the f16-storage variant of the same body. */
int intent_hip_softmax_bwd(int dtype, const void *p, const void *dy, void *dx, int64_t rows,
                           int64_t cols, int64_t p_row_stride, int64_t dy_row_stride,
                           int64_t dx_row_stride, void *stream);

/* C = bf16(A @ B), fp32 accumulation; A [m,k], B [k,n], C [m,n], row strides lda/ldb/ldc.
 * bf16_gemm (python/intent/examples/kernels/contraction/gemm.py:76-92). */
int intent_hip_gemm_bf16(const void *a, const void *b, void *c, int64_t m, int64_t n, int64_t k,
                         int64_t lda, int64_t ldb, int64_t ldc, void *stream);

/* C = T(act(A @ B)), fp32 accumulation, T the operand type (dtype F16 or BF16).
 * dtype F16: gemm (python/intent/examples/kernels/contraction/gemm.py:54-73) with the
 *            ACTIVATION constexpr: NONE, or RELU = maximum(acc, 0.0) before the cast
 *            (NaN propagates, types-numerics-and-effects.en.md:117);
 * dtype BF16: bf16_gemm (gemm.py:76-92) with activation NONE (RELU is also accepted).
 * Casts round to nearest even. A [m,k], B [k,n], C [m,n], row strides lda/ldb/ldc. */
int intent_hip_gemm(int dtype, int activation, const void *a, const void *b, void *c, int64_t m,
                    int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc, void *stream);

/* f32 GEMM with f32 accumulation (no TF32).
 * transpose_b = 0: gemm_f32   (gemm.py:15-27), C = A @ B,   B [k,n];
 * transpose_b = 1: linear_f32 (gemm.py:30-38), C = A @ B^T, B [n,k] (the weight).
 * ldb is B's row stride in either layout. */
int intent_hip_gemm_f32(const float *a, const float *b, float *c, int64_t m, int64_t n, int64_t k,
                        int64_t lda, int64_t ldb, int64_t ldc, int transpose_b, void *stream);

/* f16 GEMM with f32 accumulation and a quantizing epilogue, int8 output:
 * quantized_gemm (python/intent/examples/kernels/contraction/gemm.py:95-121). Per element, each
 * step an f32 operation: v = maximum(acc + bias[n], 0) (NaN propagates), v += residual[i][n],
 * v = v / output_scale[n] (IEEE division), v = minimum(maximum(v, -128), 127), out = i8(v)
 * truncating toward zero (NaN, an illegal cast input, gives 0). a [m,k], b [k,n], residual [m,n]
 * f16; bias, output_scale [n] f32; out [m,n] int8; row strides lda/ldb/ldr/ldo in elements. */
int intent_hip_quantized_gemm(const void *a, const void *b, const float *bias, const void *residual,
                              const float *output_scale, void *out, int64_t m, int64_t n, int64_t k,
                              int64_t lda, int64_t ldb, int64_t ldr, int64_t ldo, void *stream);

/* int8 GEMM with int32 accumulation and bias, C = A @ B + bias:
 * gemm_i8 (python/intent/examples/kernels/contraction/gemm.py:41-51). A [m,k] and B [k,n] int8,
 * bias [n] and C [m,n] int32, row strides lda/ldb/ldc in elements. int32 sums wrap on overflow;
 * the result is exact, so every shape gives the same bits. */
int intent_hip_gemm_i8(const void *a, const void *b, const int32_t *bias, int32_t *c, int64_t m,
                       int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc, void *stream);

/* Fused attention forward, f16 in/out, f32 softmax in the exp2 domain.
 * flash_attention_fwd (python/intent/examples/kernels/streaming/attention.py:428-466) with
 * summarize_attention_chunk_f16 (:152-191), merge_attention_summaries (:82-114) and
 * normalize_attention_summary (:417-425): keys folded in 64-key chunks, each chunk's weights
 * rounded to f16 against that chunk's own maximum before P @ V, chunks merged with exp2 factors.
 * q [b,h,sq,d], k [b,h,sk,d], v [b,h,sk,dv], o [b,h,sq,dv]; strides[16] holds the four
 * element strides of q, k, v, o in that order (the last of each must be 1).
 * causal: key j is valid for query i iff i >= j (absolute indices). d and dv are each 64 or 128
 * (the Python provider serves other widths up to 128 by zero-padding to these). */
int intent_hip_attention_fwd_f16(const void *q, const void *k, const void *v, void *o,
                                 int64_t batch, int64_t heads, int64_t sq, int64_t sk, int64_t d,
                                 int64_t dv, const int64_t strides[16], float scale, int causal,
                                 void *stream);

/* Fused attention forward with grouped key/value heads: q [b,hq,sq,d], k [b,hk,sk,d],
 * v [b,hk,sk,dv], o [b,hq,sq,dv] with hq = q_heads = hk * head_group; query head h reads key/value
 * head h / head_group. Same algebra as intent_hip_attention_fwd_f16, in the element type:
 * dtype F16:  flash_gqa_attention_fwd   (streaming/attention.py:469-507; HEAD_GROUP and CAUSAL
 *             constexprs), and flash_attention_fwd with head_group 1;
 * dtype BF16: flash_attention_bf16_fwd  (attention.py:510-553) with
 *             summarize_attention_chunk_bf16 (:193-237): P rounded to bf16 before P @ V, output
 *             cast to bf16. */
int intent_hip_attention_fwd(int dtype, const void *q, const void *k, const void *v, void *o,
                             int64_t batch, int64_t q_heads, int64_t head_group, int64_t sq,
                             int64_t sk, int64_t d, int64_t dv, const int64_t strides[16],
                             float scale, int causal, void *stream);

/* intent_hip_attention_fwd with a key split for small grids, the same three definitions (no
 * counterpart call in the reference: its Triton launch has no workspace; the split changes only the
 * association of the f32 merge of chunk summaries, merge_attention_summaries :82-114). When the
 * grid of 256-query blocks holds fewer than 256 workgroups, each block's key tiles are divided over
 * up to 8 workgroups, each writing its unnormalised state (maximum, denominator, O) to `workspace`,
 * and a second kernel merges the splits in order with exp2 factors. The workspace must hold
 * intent_hip_attention_fwd_workspace_bytes (0: nothing to split) and be 256-byte aligned; with a
 * null or smaller workspace the launch is unsplit, as intent_hip_attention_fwd. */
int intent_hip_attention_fwd_workspace_bytes(int64_t batch, int64_t q_heads, int64_t sq, int64_t sk,
                                             int64_t dv, size_t *bytes);
int intent_hip_attention_fwd_ws(int dtype, const void *q, const void *k, const void *v, void *o,
                                int64_t batch, int64_t q_heads, int64_t head_group, int64_t sq,
                                int64_t sk, int64_t d, int64_t dv, const int64_t strides[16],
                                float scale, int causal, void *workspace, size_t workspace_bytes,
                                void *stream);

/* Latent attention prefill: mla_prefill (streaming/attention.py:756-798, scores of
 * summarize_mla_chunk :368-415): s = (q . k + qpe . kpe) scale log2 e with the causal rule
 * key <= query, weights rounded to f16 before P @ V. q [b,h,sq,d], qpe [b,h,sq,p], k [b,hk,sk,d],
 * kpe [b,1,sk,p] (one position row per key, shared by every head), v [b,hk,sk,d], o [b,h,sq,d],
 * all f16; key head = h / head_group. d in {64, 128}, p = 64.
 * strides[24]: q, qpe, k, kpe, v, o, each (batch, head, row, col), col stride 1.
 * When batch * heads * ceil(sq / 256) leaves CUs idle, the keys of each query block are split
 * over workgroups whose states a second kernel merges; that needs a workspace (256-byte aligned)
 * of intent_hip_mla_prefill_workspace_bytes(...) bytes, 0 when no split applies. A null or
 * smaller workspace gives the unsplit launch. */
int intent_hip_mla_prefill_workspace_bytes(int64_t batch, int64_t heads, int64_t sq, int64_t sk,
                                           int64_t d, size_t *bytes);
int intent_hip_mla_prefill(const void *q, const void *qpe, const void *k, const void *kpe, const void *v,
                           void *o, int64_t batch, int64_t heads, int64_t head_group, int64_t sq,
                           int64_t sk, int64_t d, int64_t p, const int64_t strides[24], float scale,
                           void *workspace, size_t workspace_bytes, void *stream);

/* Attention forward with an additive per-key bias: flash_attention_bias_fwd
 * (streaming/attention.py:800-836, scores of summarize_biased_attention_chunk :328-366):
 * o[b,h,i,:] = sum_j softmax_j((q_i . k_j) scale + bias[b,h,j]) v[b,h,j,:], every key valid, no
 * causal mask. q, k, v, o f16 as in intent_hip_attention_fwd_f16 (strides[16]); bias f32 at
 * bias + b bias_strides[0] + h bias_strides[1] + j bias_strides[2], bias_strides[2] = 1, 4-byte
 * aligned. A bias of -inf removes its key (weight 0); a row whose keys are all removed is 0 (the
 * reference returns NaN for a query whose fold chunk is entirely -inf). */
int intent_hip_attention_bias_fwd(const void *q, const void *k, const void *v, const float *bias,
                                  void *o, int64_t batch, int64_t heads, int64_t sq, int64_t sk,
                                  int64_t d, int64_t dv, const int64_t strides[16],
                                  const int64_t bias_strides[3], float scale, void *stream);

/* Fused attention forward over packed sequences: rows cu_seqlens[s] .. cu_seqlens[s+1] of
 * q [total,hq,d], k [total,hk,d], v [total,hk,dv] and o [total,hq,dv] form sequence s; each
 * sequence attends within itself (with `causal`, key row <= query row), with the algebra of
 * intent_hip_attention_fwd.
 *   flash_varlen_attention_fwd (streaming/attention.py:839-877): hq = hk = 1, CAUSAL constexpr;
 *   flash_varlen_gqa_prefill   (streaming/attention.py:880-924): key head = query head /
 *                              head_group, causal.
 * strides[12]: (row, head, inner) element strides of q, k, v, o; inner must be 1. The offsets are
 * read on the device (clamped into [0, total]): a one-workgroup kernel lists the
 * (sequence, query block) work items into the workspace, whose size
 * intent_hip_attention_varlen_workspace_bytes gives. dtype F16 or BF16; d, dv in {64, 128}. */
int intent_hip_attention_varlen_workspace_bytes(int64_t sequences, int64_t total, size_t *bytes);
int intent_hip_attention_varlen_fwd(int dtype, const void *q, const void *k, const void *v,
                                    const int32_t *cu_seqlens, void *o, int64_t sequences, int64_t total,
                                    int64_t q_heads, int64_t head_group, int64_t d, int64_t dv,
                                    const int64_t strides[12], float scale, int causal, void *workspace,
                                    size_t workspace_bytes, void *stream);

/* Attention backward, f16 storage with f32 arithmetic, head dimension d = 64 or 128
 * (python/intent/examples/kernels/backward/attention.py; the three kernels of
 * programs/attention_backward.py:1-41). Shapes: q, dout, dq [b,hq,sq,d]; k, v, dk, dv [b,hk,sk,d]
 * with hq = q_heads = hk * head_group; lse, delta [b,hq,sq] f32; lse is the natural log of the
 * forward's softmax denominator. Every 4-D operand has unit inner stride.
 *
 * delta = sum_d o * dout: attention_backward_delta (:17-34). strides[11]: o[4], dout[4], delta[3]. */
int intent_hip_attention_bwd_delta(const void *o, const void *dout, float *delta, int64_t batch,
                                   int64_t heads, int64_t sq, int64_t d, const int64_t strides[11],
                                   void *stream);

/* dq = f16(scale * sum_k f16(p * (dout.v - delta)) k), p = exp2(q.k * scale * log2e - lse * log2e),
 * causal validity q >= k: attention_backward_dq (:171-211) with summarize_query_gradients
 * (:140-163). strides[26]: q, k, v, dout (4 each), lse[3], delta[3], dq[4]. */
int intent_hip_attention_bwd_dq(const void *q, const void *k, const void *v, const void *dout,
                                const float *lse, const float *delta, void *dq, int64_t batch,
                                int64_t q_heads, int64_t head_group, int64_t sq, int64_t sk, int64_t d,
                                const int64_t strides[26], float scale, int causal, void *stream);

/* The same with a caller-owned device workspace. When the call has fewer than 256 * 256 rows
 * (batch * q_heads * sq) and the grid above would hold fewer than 256 workgroups
 * (batch * q_heads * ceil(sq / 128)), the key tiles of each query block are divided into up to 8
 * ranges (enough for about 512 workgroups) with a workgroup each, which write unscaled f32 partial sums to the workspace
 * ([splits][batch * q_heads][sq][d]); a second kernel folds them in range order, scales and
 * casts. intent_hip_attention_bwd_dq_workspace_bytes gives the size (0 when the split is not
 * taken; the workspace may then be NULL, and a NULL workspace always selects the unsplit kernel).
 * The workspace must be 16-byte aligned. No counterpart in the reference: the reference's single
 * kernel launch (backward/attention.py:171-211) has no workspace. */
int intent_hip_attention_bwd_dq_workspace_bytes(int64_t batch, int64_t q_heads, int64_t head_group,
                                                int64_t sq, int64_t sk, int64_t d, size_t *bytes);
int intent_hip_attention_bwd_dq_ws(const void *q, const void *k, const void *v, const void *dout,
                                   const float *lse, const float *delta, void *dq, int64_t batch,
                                   int64_t q_heads, int64_t head_group, int64_t sq, int64_t sk, int64_t d,
                                   const int64_t strides[26], float scale, int causal, void *workspace,
                                   size_t workspace_bytes, void *stream);

/* dk = f16(scale * sum_q f16(ds) q), dv = f16(sum_q f16(p) dout), summed over the head_group query
 * heads of each key head: attention_backward_dkdv (:87-137) with summarize_key_value_gradients
 * (:47-79). strides[30]: q, k, v, dout (4 each), lse[3], delta[3], dk[4], dv[4]. */
int intent_hip_attention_bwd_dkdv(const void *q, const void *k, const void *v, const void *dout,
                                  const float *lse, const float *delta, void *dk, void *dv,
                                  int64_t batch, int64_t q_heads, int64_t head_group, int64_t sq,
                                  int64_t sk, int64_t d, const int64_t strides[30], float scale,
                                  int causal, void *stream);

/* The same with a caller-owned device workspace. When the grid above would hold fewer than 256
 * workgroups (batch * kv_heads * ceil(sk / 128)), each query head of the group, and each of up to
 * 8 ranges of its query tiles (qsplits, enough for about 512 workgroups), gets its own workgroups, which write unscaled f32
 * partial sums to the workspace ([2][head_group * qsplits][batch][kv_heads][sk][d]: dK, then dV);
 * a second kernel folds them in (head, range) order, scales dK and casts. With head_group == 1
 * the split is taken only when qsplits > 1. intent_hip_attention_bwd_dkdv_workspace_bytes gives
 * the size (0 when the split is not taken; the workspace may then be NULL, and a NULL workspace
 * always selects the unsplit kernel). The workspace must be 16-byte aligned. No counterpart in
 * the reference: the reference's single kernel launch (backward/attention.py:87-137) has no
 * workspace. */
int intent_hip_attention_bwd_dkdv_workspace_bytes(int64_t batch, int64_t q_heads, int64_t head_group,
                                                  int64_t sq, int64_t sk, int64_t d, size_t *bytes);
int intent_hip_attention_bwd_dkdv_ws(const void *q, const void *k, const void *v, const void *dout,
                                     const float *lse, const float *delta, void *dk, void *dv,
                                     int64_t batch, int64_t q_heads, int64_t head_group, int64_t sq,
                                     int64_t sk, int64_t d, const int64_t strides[30], float scale,
                                     int causal, void *workspace, size_t workspace_bytes, void *stream);

/* Paged grouped-query decode attention over one page range per (batch, split): f16 q, caches,
 * f32 partial results. paged_gqa_decode_partials
 * (python/intent/examples/kernels/streaming/paged_attention.py:77-165) with
 * summarize_masked_attention_chunk (streaming/attention.py:250-285); launched first by
 * PagedDecode (programs/composition.py:95-122).
 * Shapes: q [batch, q_heads, d]; key_cache [pages, ps, kv_heads, d]; value_cache
 * [pages, ps, kv_heads, dv]; page_offsets [batch + 1], lengths [batch], split_offsets
 * [batch * splits + 1], page_indices [positions] (i32); partial_lse [batch, q_heads, splits] and
 * partial_output [batch, q_heads, splits, dv] (f32). q_heads = kv_heads * head_group,
 * head_group 1..16, d = dv = 64 or 128; page_size is the PAGE_SIZE constexpr (logical tokens per
 * page). Job j = b * splits + s covers page positions split_offsets[j] .. split_offsets[j+1];
 * a token is active while its logical index is below lengths[b]. partial_lse is base 2
 * (max + ln(den) * log2 e, -inf for an empty job); partial_output = acc / den (0 for an empty
 * job). Out-of-range page positions and physical pages are clamped, never dereferenced.
 * strides[18]: q[3], key_cache[4], value_cache[4], partial_lse[3], partial_output[4]. */
int intent_hip_paged_decode_partials(const void *q, const void *key_cache, const void *value_cache,
                                     const int32_t *page_offsets, const int32_t *page_indices,
                                     const int32_t *lengths, const int32_t *split_offsets,
                                     float *partial_lse, float *partial_output, int64_t batch,
                                     int64_t q_heads, int64_t d, int64_t pages, int64_t ps,
                                     int64_t kv_heads, int64_t dv, int64_t positions, int64_t page_size,
                                     int64_t head_group, int64_t splits, const int64_t strides[18],
                                     float scale, void *stream);

/* Split-K merge: out[b,h,:] = f16(sum_s w_s partial[b,h,s,:] * rcp(sum_s w_s)),
 * w_s = exp(lse[b,h,s] - max_s lse[b,h,s]) with the natural exponential, as
 * splitk_attention_f32_to_f16_reduce (streaming/splitk_reduce.py:129-155) writes it; launched
 * second by PagedDecode (programs/composition.py:95-122). partial f32 [batch, heads, splits, d],
 * lse f32 [batch, heads, splits], out f16 [batch, heads, d].
 * strides[10]: partial[4], lse[3], out[3]. */
int intent_hip_splitk_reduce_f32_to_f16(const float *partial, const float *lse, void *out, int64_t batch,
                                        int64_t heads, int64_t splits, int64_t d, const int64_t strides[10],
                                        void *stream);

/* Grouped-query decode partials over dense bf16 caches: grouped_flash_decode_partials
 * (streaming/attention.py:556-627) with summarize_attention_chunk_bf16 (:195-237). q
 * [batch, q_heads, 1, d], k [batch, kv_heads, keys, d], v [batch, kv_heads, keys, dv] (bf16);
 * part p of (b, key head) covers keys p * split_size .. + split_size below `keys`. Weights are
 * rounded to bf16 before P @ V. partial_lse f32 [batch, q_heads, parts] (max + ln(den) log2 e,
 * -inf for a part with no key), partial_output bf16 [batch, q_heads, parts, dv] (acc / den, 0 for
 * a part with no key). q_heads = kv_heads * head_group, head_group 1..16, d = dv = 64 or 128.
 * strides[19]: q[4], k[4], v[4], partial_lse[3], partial_output[4]. */
int intent_hip_grouped_decode_partials(const void *q, const void *k, const void *v, float *partial_lse,
                                       void *partial_output, int64_t batch, int64_t q_heads,
                                       int64_t kv_heads, int64_t head_group, int64_t keys, int64_t d,
                                       int64_t dv, int64_t parts, int64_t split_size,
                                       const int64_t strides[19], float scale, void *stream);

/* Decode over a dense f16 cache with a validity mask: continuous_gqa_decode
 * (streaming/attention.py:629-670) with summarize_masked_attention_chunk (:250-285). q
 * [batch, q_heads, d], k [batch, keys, kv_heads, d], v [batch, keys, kv_heads, dv], valid_mask u8
 * [batch, keys, kv_heads] (key j of head kh admitted where nonzero), output f16
 * [batch, q_heads, dv] (0 for a query with no admitted key). The keys are split over workgroups
 * whose states merge in a second kernel; the workspace (256-byte aligned) holds
 * intent_hip_dense_decode_workspace_bytes(batch, q_heads, kv_heads, keys, dv) bytes.
 * strides[17]: q[3], k[4], v[4], valid_mask[3], output[3]. */
int intent_hip_dense_decode_workspace_bytes(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t keys,
                                            int64_t dv, size_t *bytes);
int intent_hip_continuous_gqa_decode(const void *q, const void *k, const void *v, const uint8_t *valid_mask,
                                     void *out, int64_t batch, int64_t q_heads, int64_t kv_heads,
                                     int64_t head_group, int64_t keys, int64_t d, int64_t dv,
                                     const int64_t strides[17], float scale, void *workspace,
                                     size_t workspace_bytes, void *stream);

/* Decode over packed f16 sequences with a per-head sink and block logits:
 * varlen_gqa_decode_with_sink_logits (streaming/attention.py:672-754). q [sequences, q_heads, d],
 * k [rows, kv_heads, d], v [rows, kv_heads, dv]; sequence b is rows cu_seqlens[b] .. [b + 1]
 * (offsets clamped into [0, rows]), of which the first 64 * max_blocks keys are attended, in
 * 64-key blocks. With M the largest block maximum (exp2 domain) and den the merged denominator,
 * output = acc / (den + sink[h]) (f16; 0 for an empty sequence) and block_logits[b, h, j] =
 * exp2(max_j - M) / (den + sink[h]) for j < ceil(length / 64), else 0 (f32). The workspace
 * (256-byte aligned) holds intent_hip_varlen_decode_workspace_bytes(sequences, q_heads, kv_heads,
 * max_blocks, dv) bytes. strides[15]: q[3], k[3], v[3], output[3], block_logits[3]. */
int intent_hip_varlen_decode_workspace_bytes(int64_t sequences, int64_t q_heads, int64_t kv_heads,
                                             int64_t max_blocks, int64_t dv, size_t *bytes);
int intent_hip_varlen_decode_sink(const void *q, const void *k, const void *v, const int32_t *cu_seqlens,
                                  const float *sink, void *out, float *block_logits, int64_t sequences,
                                  int64_t rows, int64_t q_heads, int64_t kv_heads, int64_t head_group,
                                  int64_t d, int64_t dv, int64_t max_blocks, const int64_t strides[15],
                                  float scale, void *workspace, size_t workspace_bytes, void *stream);

/* CSR SpMV y = A x, f32 values, i32 indices.
 * csr_spmv (python/intent/examples/kernels/sparse/csr_spmv.py:11-29), with dynamic extents. Row r
 * covers the absolute positions [row_offsets[r], row_offsets[r + 1]) of column_indices and values
 * (nnz entries each), so the offsets may start above 0 and end below nnz.
 * The workspace (device memory, caller-owned, 256-byte aligned) must hold
 * intent_hip_csr_spmv_workspace_bytes(rows, nnz): at most about 1.13 bytes per nonzero. */
int intent_hip_csr_spmv_workspace_bytes(int64_t rows, int64_t nnz, size_t *bytes);
int intent_hip_csr_spmv_f32(const int32_t *row_offsets, const int32_t *column_indices,
                            const float *values, const float *x, float *y, int64_t rows,
                            int64_t cols, int64_t nnz, void *workspace, size_t workspace_bytes,
                            void *stream);

/* CSR SpMV with no workspace argument and no allocation: the workspace is a static device array of
 * INTENT_HIP_STATIC_SCRATCH_BYTES inside the library (one per GPU, held until the process ends).
 * No counterpart in the reference; it is for callers that cannot allocate device memory (code
 * under graph capture, serving loops, harnesses that forbid hipMalloc). Same results as
 * intent_hip_csr_spmv_f32 (the same kernels). Returns INTENT_HIP_ERR_WORKSPACE when
 * intent_hip_csr_spmv_workspace_bytes(rows, nnz) exceeds the static array. Unlike the other entry
 * points it is not stateless: calls that overlap on one GPU share the array and race. */
#define INTENT_HIP_STATIC_SCRATCH_BYTES (32u << 20)
int intent_hip_csr_spmv_f32_static(const int32_t *row_offsets, const int32_t *column_indices,
                                   const float *values, const float *x, float *y, int64_t rows,
                                   int64_t cols, int64_t nnz, void *stream);

/* CSR SpMM out = A dense, f32 values and features, i32 indices.
 * csr_spmm (python/intent/examples/kernels/sparse/csr_spmm.py:11-33), with dynamic extents:
 * row_offsets [rows + 1], column_indices and values [nnz], dense [cols, features] with row stride
 * ldd, out [rows, features] with row stride ldo. Each output element is the left fold over the
 * row's nonzeros in order, acc = acc + values[nz] * dense[col, f] with the product rounded before
 * the add. Columns outside [0, cols) read row cols - 1; offsets are clamped to [0, nnz]. */
int intent_hip_csr_spmm_f32(const int32_t *row_offsets, const int32_t *column_indices,
                            const float *values, const float *dense, float *out, int64_t rows,
                            int64_t cols, int64_t nnz, int64_t features, int64_t ldd, int64_t ldo,
                            void *stream);

/* Measurement probe (no counterpart in the reference): the box's own MFMA ceiling, reported by the
 * benchmark beside the published peak, as the measurement protocol asks for an MFMA
 * microbenchmark on the same box. `blocks` workgroups of 4 waves (two workgroups per CU give two
 * waves per SIMD), each wave issuing `iterations` rounds of 8 independent
 * v_mfma_f32_32x32x16_{f16,bf16} on register operands; dtype F16 or BF16. varied = 0: every MFMA
 * multiplies the same two operands; varied = 1: each chain has its own operands with pseudo-random
 * mantissas, switching as many multiplier bits as real data. Operand values lie in [0.5, 1).
 * Work: blocks * 4 * iterations * 8 * 32768 FLOP. out: blocks * 4 floats (one sum per wave, so
 * the work cannot be dropped). */
int intent_hip_mfma_probe(int dtype, int varied, int64_t blocks, int64_t iterations, float *out,
                          void *stream);

#ifdef __cplusplus
}
#endif

#endif /* INTENT_HIP_H */
