/*
 * tokengate_hip.h — C ABI of the MI355X (gfx950) key-bias attention and gate-path kernels.
 *
 * Every entry point takes raw device pointers, element strides and sizes, and a HIP stream.
 * Nothing here allocates device memory unless stated: the caller owns every input, output
 * and workspace buffer.  Work is enqueued on `stream` and runs asynchronously; no entry point
 * synchronises the host.  A nonzero return value is an error code; tg_last_error() gives the
 * message (thread-local, valid until the next call on the same thread).
 *
 * Tensor conventions (all strides in ELEMENTS, the head_dim axis always contiguous):
 *   q   (B, Sq, H,   D) bf16        k, v (B, Sk, Hkv, D) bf16
 *   out (B, Sq, H,   D) bf16        lse  (B, H, Sq) fp32, contiguous, natural log
 *   bias_raw (B, H, Sk) fp32, last axis contiguous, in raw-score units: the logit of query i
 *   and key j is softmax_scale * (q_i . k_j + bias_raw[b, h, j]).
 * Varlen tensors drop the batch axis and stack sequences along the row axis:
 *   q (total, H, D), k/v (total, Hkv, D), cu_seqlens int32 (num_seqs + 1) on the device,
 *   bias_raw (num_seqs, H, max_seqlen) indexed by each key's position inside its own sequence,
 *   lse (H, total) fp32.
 * Only bf16 with head_dim 128 is supported (the reference build's restriction,
 * kernels/fa2bias/keybias.patch:18 and :94).
 */
#ifndef TOKENGATE_HIP_H
#define TOKENGATE_HIP_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI stamp: 2 = key bias available on the variable-length entry points.
 * Replaces the BUILD_INFO.json "abi" field read by require_varlen()
 * (kernels/fa2bias/site_path.py:7-8, kernels/fa2bias/keybias.py:29-37). */
int tg_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char *tg_last_error(void);

/* Dense key-bias attention forward.
 * Replaces ext().fwd(q, k, v, None, bias_raw, 0.0, scale, causal, -1, -1, 0.0, False, None)
 * (kernels/fa2bias/keybias.py:40-44; patched mha_fwd, keybias.patch:7-28, 65-83, 279-332).
 * bias_raw may be NULL (plain causal/non-causal attention, the Phase-1 "flash" call).
 * Causal masking aligns the last query with the last key (key j visible to query i iff
 * j <= i + Sk - Sq).  Rows that see no key get out = 0 and lse = +inf. */
int tg_keybias_fwd(const void *q, const void *k, const void *v, const float *bias_raw,
                   void *out, float *lse,
                   int32_t batch, int32_t seqlen_q, int32_t seqlen_k,
                   int32_t num_heads, int32_t num_heads_k, int32_t head_dim,
                   int64_t q_batch_stride, int64_t q_row_stride, int64_t q_head_stride,
                   int64_t k_batch_stride, int64_t k_row_stride, int64_t k_head_stride,
                   int64_t v_batch_stride, int64_t v_row_stride, int64_t v_head_stride,
                   int64_t o_batch_stride, int64_t o_row_stride, int64_t o_head_stride,
                   int64_t bias_batch_stride, int64_t bias_head_stride,
                   float softmax_scale, int32_t causal, hipStream_t stream);

/* Variable-length key-bias attention forward (one causal attention per packed sequence).
 * Replaces ext().varlen_fwd(q, k, v, None, cu, cu, None, None, None, bias_raw, max, max, 0.0,
 * scale, False, causal, -1, -1, 0.0, False, None) (kernels/fa2bias/keybias.py:90-100; varlen
 * bias enabled by kernels/fa2bias/build.py:58-78).  cu_seqlens serves both q and k. */
int tg_keybias_varlen_fwd(const void *q, const void *k, const void *v, const float *bias_raw,
                          void *out, float *lse, const int32_t *cu_seqlens,
                          int32_t num_seqs, int32_t max_seqlen, int32_t total,
                          int32_t num_heads, int32_t num_heads_k, int32_t head_dim,
                          int64_t q_row_stride, int64_t q_head_stride,
                          int64_t k_row_stride, int64_t k_head_stride,
                          int64_t v_row_stride, int64_t v_head_stride,
                          int64_t o_row_stride, int64_t o_head_stride,
                          int64_t bias_seq_stride, int64_t bias_head_stride,
                          float softmax_scale, int32_t causal, hipStream_t stream);

/* Dense key-bias attention backward.
 * Replaces ext().bwd(dout, q, k, v, out, lse, None, None, None, bias_raw, 0.0, scale, causal,
 * -1, -1, 0.0, False, None, None) -> (dq, dk, dv, softmax_d, dbias) (kernels/fa2bias/keybias.py:52-63;
 * patched mha_bwd and the dBias reduction, keybias.patch:87-129, 219-271).
 * Outputs (caller-allocated, fully overwritten): dq like q, dk/dv like k/v (summed over the query
 * heads of each KV head), softmax_d (B, H, Sq) fp32 = rowsum(dout * out), and, when bias_raw is
 * given, dbias (B, H, Sk) fp32 = softmax_scale * sum_i dS[i, j] (the gradient with respect to
 * bias_raw).  Deterministic: no atomics.
 * strides: 28 int64 on the host, in elements:
 *   q, k, v, out, dout, dq, dk, dv as (batch, row, head) triples, then bias (batch, head) and
 *   dbias (batch, head). */
int tg_keybias_bwd(const void *dout, const void *q, const void *k, const void *v, const void *out,
                   const float *lse, const float *bias_raw, void *dq, void *dk, void *dv, float *dbias,
                   float *softmax_d, int32_t batch, int32_t seqlen_q, int32_t seqlen_k,
                   int32_t num_heads, int32_t num_heads_k, int32_t head_dim,
                   const int64_t *strides, float softmax_scale, int32_t causal, hipStream_t stream);

/* Variable-length backward (kernels/fa2bias/keybias.py:103-115).  lse and softmax_d are (H, total);
 * bias_raw and dbias are (num_seqs, H, max_seqlen).
 * strides: 20 int64 on the host: q, k, v, out, dout, dq, dk, dv as (row, head) pairs, then bias
 * (seq, head) and dbias (seq, head). */
int tg_keybias_varlen_bwd(const void *dout, const void *q, const void *k, const void *v, const void *out,
                          const float *lse, const float *bias_raw, void *dq, void *dk, void *dv,
                          float *dbias, float *softmax_d, const int32_t *cu_seqlens,
                          int32_t num_seqs, int32_t max_seqlen, int32_t total,
                          int32_t num_heads, int32_t num_heads_k, int32_t head_dim,
                          const int64_t *strides, float softmax_scale, int32_t causal, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TOKENGATE_HIP_H */
