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
 * j <= i + Sk - Sq).  Rows that see no key get out = 0 and lse = +inf.
 * workspace: caller-allocated device memory of tg_keybias_fwd_workspace_size() bytes (16-byte
 * aligned) for the key-range split of launches too small to fill the GPU, like the split-KV
 * accumulators the reference's mha_fwd allocates for itself (softmax_lse_accum / out_accum in
 * flash-attn's set_params_splitkv); NULL, or fewer bytes, runs without the split.  Contents need
 * no initialisation; calls that share one workspace must be stream-ordered. */
int tg_keybias_fwd(const void *q, const void *k, const void *v, const float *bias_raw,
                   void *out, float *lse,
                   int32_t batch, int32_t seqlen_q, int32_t seqlen_k,
                   int32_t num_heads, int32_t num_heads_k, int32_t head_dim,
                   int64_t q_batch_stride, int64_t q_row_stride, int64_t q_head_stride,
                   int64_t k_batch_stride, int64_t k_row_stride, int64_t k_head_stride,
                   int64_t v_batch_stride, int64_t v_row_stride, int64_t v_head_stride,
                   int64_t o_batch_stride, int64_t o_row_stride, int64_t o_head_stride,
                   int64_t bias_batch_stride, int64_t bias_head_stride,
                   float softmax_scale, int32_t causal,
                   void *workspace, int64_t workspace_bytes, hipStream_t stream);

/* Workspace bytes tg_keybias_fwd uses for these sizes on the current device (0: no split). */
int64_t tg_keybias_fwd_workspace_size(int32_t batch, int32_t seqlen_q, int32_t seqlen_k,
                                      int32_t num_heads, int32_t num_heads_k, int32_t causal);

/* tg_keybias_fwd for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the reference, whose
 * mha_fwd allocates its split-KV accumulators itself.  Same arguments and results as
 * tg_keybias_fwd; the key-range split's partials live in a static 24 MiB device array of the
 * library (one per device, held until the process ends; a split needs at most CUs x 73,728 bytes,
 * 18 MiB on MI355X) instead of a caller workspace.  Calls no hipMalloc / hipFree.  Returns an
 * error, before launching anything, if a launch would need more than the static size.  All calls
 * on one device share that array: calls that overlap on one device (different streams, or
 * graphs replayed concurrently) race; calls ordered on one stream do not.  Its contents need no
 * initialisation (every partial a launch reads is written by that launch). */
int tg_keybias_fwd_noalloc(const void *q, const void *k, const void *v, const float *bias_raw,
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
 * bias enabled by kernels/fa2bias/build.py:58-78).  cu_seqlens serves both q and k.
 * workspace: as for tg_keybias_fwd, sized by tg_keybias_varlen_fwd_workspace_size(). */
int tg_keybias_varlen_fwd(const void *q, const void *k, const void *v, const float *bias_raw,
                          void *out, float *lse, const int32_t *cu_seqlens,
                          int32_t num_seqs, int32_t max_seqlen, int32_t total,
                          int32_t num_heads, int32_t num_heads_k, int32_t head_dim,
                          int64_t q_row_stride, int64_t q_head_stride,
                          int64_t k_row_stride, int64_t k_head_stride,
                          int64_t v_row_stride, int64_t v_head_stride,
                          int64_t o_row_stride, int64_t o_head_stride,
                          int64_t bias_seq_stride, int64_t bias_head_stride,
                          float softmax_scale, int32_t causal,
                          void *workspace, int64_t workspace_bytes, hipStream_t stream);

/* Workspace bytes tg_keybias_varlen_fwd uses for these sizes on the current device (0: no split). */
int64_t tg_keybias_varlen_fwd_workspace_size(int32_t num_seqs, int32_t max_seqlen,
                                             int32_t num_heads, int32_t num_heads_k, int32_t causal);

/* Variable-length forward with the keys of each sequence stored apart from its queries: the
 * general form of the same ext().varlen_fwd binding, whose cu_seqlens_k and seqused_k arguments
 * the reference's own call leaves at cu and None (kernels/fa2bias/keybias.py:90-100).  Query rows
 * of sequence b are cu_seqlens_q[b] .. cu_seqlens_q[b + 1] - 1 (at most max_seqlen_q of them);
 * its keys are k / v rows cu_seqlens_k[b] .. cu_seqlens_k[b] + n_b - 1 with n_b = seqused_k[b]
 * (seqused_k NULL: n_b = cu_seqlens_k[b + 1] - cu_seqlens_k[b]), at most max_seqlen_k.  Causal
 * masking is bottom-right aligned (query i of m sees keys j <= i + n_b - m).  bias_raw
 * (num_seqs, H, >= max_seqlen_k) fp32, column j = key j of the sequence.  lse (H, total_q).
 * This is the layout of a KV cache with room for generated tokens after every sequence: the
 * gated prefill's Phase 2 writes its kept rows there and every decode step attends over it for
 * all sequences in one launch (the reference's decode attention over its pruned, padded cache,
 * qwen3_flex_attention.py:978-1117, gate_decode.py:143-235).  workspace: sized by
 * tg_keybias_varlen_kv_fwd_workspace_size(). */
int tg_keybias_varlen_kv_fwd(const void *q, const void *k, const void *v, const float *bias_raw,
                             void *out, float *lse, const int32_t *cu_seqlens_q,
                             const int32_t *cu_seqlens_k, const int32_t *seqused_k, int32_t num_seqs,
                             int32_t max_seqlen_q, int32_t max_seqlen_k, int32_t total_q,
                             int32_t num_heads, int32_t num_heads_k, int32_t head_dim,
                             int64_t q_row_stride, int64_t q_head_stride,
                             int64_t k_row_stride, int64_t k_head_stride,
                             int64_t v_row_stride, int64_t v_head_stride,
                             int64_t o_row_stride, int64_t o_head_stride,
                             int64_t bias_seq_stride, int64_t bias_head_stride,
                             float softmax_scale, int32_t causal,
                             void *workspace, int64_t workspace_bytes, hipStream_t stream);

/* Workspace bytes tg_keybias_varlen_kv_fwd uses for these sizes on the current device. */
int64_t tg_keybias_varlen_kv_fwd_workspace_size(int32_t num_seqs, int32_t max_seqlen_q, int32_t max_seqlen_k,
                                                int32_t num_heads, int32_t num_heads_k, int32_t causal);

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

/* ---- gate path (tokengate/e2e_gate/gate_module/gate_forward.py:1384-1522) ---------------- */

/* Scoring head over packed rows: scores[r] = w2 . silu(W1 x_r + b1) + b2, fp32.
 * x (n_rows, d_in) bf16 with row stride x_row_stride (elements), W1 (d_hidden, d_in) bf16
 * row-major (nn.Linear weight), b1 / w2 fp32 (d_hidden).  d_in = 2048, d_hidden = 256 (the
 * Linear(2048->256) -> SiLU -> Linear(256->1) head).  Stands in for the gate-layer scoring that
 * feeds the selection (gate_branch_hs / E2EGate.forward, gate_forward.py:491-524,
 * e2e_gate_module.py:348-385). */
int tg_gate_score_mlp(const void *x, int64_t n_rows, int64_t x_row_stride, int32_t d_in,
                      int32_t d_hidden, const void *w1, const float *b1, const float *w2, float b2,
                      float *scores, hipStream_t stream);

/* tg_gate_score_mlp with W1 stored k-step major: w1_ktiled (d_in / 32, d_hidden, 32) bf16,
 * element (s, u, j) = W1[u, 32 s + j] (torch: w1.view(256, 64, 32).transpose(0, 1).contiguous()),
 * so that each 32-input step of the weight stream is 16 KiB contiguous instead of 256 rows of
 * 64 bytes 4 KiB apart.  The same results bit for bit; the scoring head's own (synthetic) weight
 * layout, kept by gate.ScoringHead next to the row-major W1.  Stands in for the same gate-layer
 * scoring (gate_forward.py:491-524, e2e_gate_module.py:348-385). */
int tg_gate_score_mlp_ktiled(const void *x, int64_t n_rows, int64_t x_row_stride, int32_t d_in,
                             int32_t d_hidden, const void *w1_ktiled, const float *b1, const float *w2,
                             float b2, float *scores, hipStream_t stream);

/* Order-preserving top-K keep lists, one per sequence (gate_forward.py:1396-1421, _keep_indices
 * :77-81, torch.topk via _select_topk_or_random :84-99).
 * geom: device int32 (num_seqs, 6) rows [row_start, seq_len, art_start, art_end, k_clamped,
 * kept_start]: the sequence's scores are scores[row_start + i], 0 <= i < seq_len; its state span
 * (article) is [art_start, art_end); k_clamped = max(1, min(K, art_end - art_start)) (0 for an
 * empty article); its keep list goes to keep[kept_start ...]: 0..art_start-1, then the article
 * positions of the k_clamped largest scores in ascending position order, then art_end..seq_len-1.
 * Ties at the threshold go to the lower position; -0.0 equals +0.0; NaN ranks above +inf.
 * sumsq (optional, device fp32 per sequence) receives the sum of squared article scores.
 * max_article_len: the largest art_end - art_start, a speed hint only: it picks the register-
 * resident variant for the launch, and any sequence whose article is longer than that variant
 * holds (32768 or 65536 keys) takes the streaming path inside the same launch, so an understated
 * value never truncates a keep list. */
int tg_gate_topk_keep(const float *scores, const int32_t *geom, int32_t num_seqs,
                      int32_t max_article_len, int64_t *keep, float *sumsq, hipStream_t stream);

/* One row stream of the pack: source row r starts at src + r * src_row_stride and consists of
 * n_chunks chunks of chunk_bytes, src_chunk_stride apart (1 chunk for a (rows, ...) contiguous
 * row; Hkv chunks for a head-major cache); destination row j is the chunks back to back at
 * dst + j * dst_row_stride.  Byte units; everything 16-byte aligned. */
typedef struct tg_pack_stream {
  const void *src;
  void *dst;
  int64_t src_row_stride;
  int64_t dst_row_stride;
  int64_t src_chunk_stride;
  int32_t chunk_bytes;
  int32_t n_chunks;
  int64_t dst_seq_gap;   /* rows left free after each sequence's destination rows: kept row j of
                            sequence b goes to destination row j + b * dst_seq_gap (0: back to
                            back) -- a KV cache with room for generated tokens */
} tg_pack_stream;

/* Ragged gather of the kept rows (gate_forward.py:1454-1522: hs_pruned, kept_positions,
 * gate_bias_batched, the below-gate KV index_select), packed back to back in keep order
 * (cu_seqlens layout: sequence b's rows start at geom[b].kept_start).  For kept row j of
 * sequence b, every stream copies source row geom[b].row_start + keep[j] to destination row j;
 * positions_out[j] = keep[j] (int64, optional); bias_out[j] (optional) = the kept row's score
 * bias_src[row_start + keep[j]] scaled by rsqrt(sumsq[b] / n_art + rms_eps) when sumsq is given,
 * on article rows, and 0 on prefix / suffix rows.  A kept position outside [0, seq_len) of its
 * sequence gathers nothing (destination row, positions_out and bias_out entries left as they
 * were).  At most 16 streams. */
int tg_gate_pack(const tg_pack_stream *streams, int32_t n_streams, const int64_t *keep,
                 const int32_t *geom, int32_t num_seqs, int64_t total_kept, int64_t *positions_out,
                 const float *bias_src, const float *sumsq, float rms_eps, float *bias_out,
                 hipStream_t stream);

/* tg_gate_topk_keep then tg_gate_pack, with the keep lists selected by many workgroups per
 * sequence (the reference's per-sample score -> topk -> sort -> cat -> index_select loop,
 * gate_forward.py:1396-1522, for a whole ragged batch); two stream-ordered launches (the
 * selection, then the gather) when n_select_wgs is at most the device's CU count, 512 and
 * chunk_capacity, four above (three selection launches).  Sequence
 * b's state span is cut into chunks of 512 * keys_per_thread scores (keys_per_thread 4, 8, 16 or 32)
 * selected by one workgroup each: wg_start (num_seqs + 1, int32, device) lists them, sequence b
 * owning chunks [wg_start[b], wg_start[b + 1]) (none when its span is empty, at most 64),
 * n_select_wgs = wg_start[num_seqs].  Outputs: keep (total_kept, int64, the same lists as
 * tg_gate_topk_keep), positions_out = keep (optional), bias_out (optional) = the kept state rows'
 * scores times rsqrt(mean of the span's squared scores + rms_eps), 0 on prefix / suffix rows, and
 * every stream's rows gathered as tg_gate_pack does.  workspace:
 * tg_gate_select_pack_workspace_size(seq_capacity, chunk_capacity) bytes (about 90 KB per
 * chunk of capacity up to 512 and 25 KB per chunk beyond, plus 128 KB per sequence: 55 MB for
 * 64 sequences and 512 chunks), 256-byte aligned,
 * zero-filled before its first use, for calls of at most seq_capacity sequences and
 * chunk_capacity chunks (every call on one workspace passes the same capacities: its layout
 * depends on them alone).  Every call leaves its counters zeroed again, so stream-ordered calls
 * reuse it without clearing; calls that overlap on one workspace race.  The 32-bit word at byte
 * offset 8 of the workspace is an error word that stays set until the caller clears it: 1 = a
 * wait timed out, 2 = a chunk's count overran its sequence, 3 = the gather met a kept position
 * outside its sequence (a keep entry left unwritten) and skipped that row.  Nonzero means the keep
 * lists and gathered rows of the calls since it was last cleared are not to be used; no row outside
 * a sequence is ever read or written.  Every wait is bounded (seconds), so every call completes.
 * In the one-launch form the chunk workgroups of a sequence wait for one another: at most one per
 * CU, they are resident together unless other work holds the CUs for longer than the bound (then
 * error 1); in the three-launch form no workgroup waits for one that may not have started. */
int tg_gate_select_pack(const float *scores, const int32_t *geom, const int32_t *wg_start, int32_t num_seqs,
                        int32_t n_select_wgs, int32_t keys_per_thread, const tg_pack_stream *streams,
                        int32_t n_streams, int64_t total_kept, int64_t *keep, int64_t *positions_out,
                        float *bias_out, float rms_eps, void *workspace, int32_t seq_capacity,
                        int32_t chunk_capacity, hipStream_t stream);

/* Workspace bytes of tg_gate_select_pack for these capacities. */
int64_t tg_gate_select_pack_workspace_size(int32_t seq_capacity, int32_t chunk_capacity);

/* Threshold selection (_select_threshold with aggregate, gate_forward.py:102-143,
 * e2e_gate_module.py:387-399: keep the state tokens with sigmoid(agg) >= tau, or the single argmax
 * when none passes; the kept count is sample-dependent).  For the state span of every sequence
 * (geom as for tg_gate_select_pack; its k_clamped / kept_start columns are ignored), with
 * raw = scores[row_start + art_start + j]: inv = fp32(1 / sqrt(fp32(m + rms_eps))), m the span's
 * mean of raw^2 rounded once to fp32; bn = fp32(gain * fp32(raw * inv)); agg = the sum over h in
 * order of fp32(fp32(bn * head_scale[h]) * fp32(1 / n_heads)) (bn * head_scale[0] for one head),
 * every operation a separately rounded fp32 one; head_scale (n_heads <= 64 floats, HOST memory) is
 * softplus(gate_scale) of the first Phase-2 layer.  A token passes when agg >= b_star (the exact
 * fp32 form of sigmoid(agg) >= tau: the least fp32 value whose sigmoid reaches tau; NaN to pass
 * nothing); NaN never passes.  Outputs, at the span's rows of the packed row layout: agg_out and
 * select_out (rows fp32) with select = passing ? 1 : 0 when the sequence has a passing token, else
 * agg; counts[b] = passing tokens (int32); sumsq[b] (optional) = the span's sum of squares.  Top-K
 * of select_out with K_b = max(counts[b], 1) (tg_gate_select_pack) is then exactly the reference's
 * selection. */
int tg_gate_threshold_select(const float *scores, const int32_t *geom, int32_t num_seqs, const float *head_scale,
                             int32_t n_heads, float gain, float rms_eps, float b_star, float *agg_out,
                             float *select_out, int32_t *counts, float *sumsq, hipStream_t stream);

/* ---- decoder ops of the gated prefill (Qwen3 layer, transformers 5.x modeling_qwen3.py) ------
 * Called by this library's prefill around the attention; the reference runs them as eager torch
 * modules inside each decoder layer (qwen3_flex_attention.py:533-544 for q/k norm + RoPE). */

/* Residual add + RMSNorm over rows of `dim` bf16 elements (Qwen3RMSNorm, Qwen3DecoderLayer's
 * input / post-attention norms and the model's final norm).  With residual != NULL:
 * s = bf16(x + residual), written to residual_out when that is non-NULL (it may alias residual);
 * else s = x.  out = bf16(weight * s / sqrt(mean(s^2) + eps)).  dim a multiple of 8, <= 4096;
 * strides in elements, multiples of 8; pointers 16-byte aligned.  out may alias x. */
int tg_rmsnorm(const void *x, int64_t x_row_stride, const void *residual, int64_t residual_row_stride,
               void *residual_out, int64_t residual_out_row_stride, const void *weight, void *out,
               int64_t out_row_stride, int64_t n_rows, int32_t dim, float eps, hipStream_t stream);

/* Per-head q/k RMSNorm + rotary embedding (Qwen3Attention q_norm / k_norm, rotate-half RoPE,
 * qwen3_flex_attention.py:533-544), with the Phase-2 query scale of _phase2_q_bias (:433-473)
 * folded in: per head (attn_scale) and per row (the scaled-softmax ratio r_q, :417-431).
 * qkv rows hold [q heads | k heads | v heads] x head_dim (=128) bf16.  For token t at position
 * positions[t] (int64): angle_i = float(positions[t]) * inv_freq[i] (fp32, i < 64); q head h ->
 * q_out row t (may alias qkv); where q_head_scale / q_row_scale are non-NULL the rotated query,
 * rounded to bf16, is multiplied by s = bf16(q_head_scale[h] * q_row_scale[t]) (a missing factor
 * is 1) and rounded again — the reference's bf16 q * s_eff; k head g -> k_out row c and v head g
 * copied to v_out row c (the layer's KV cache, (rows, num_heads_k, 128)), with c = kv_rows[t]
 * (int32) when kv_rows is non-NULL (a cache with free rows after each sequence), else c = t. */
int tg_qk_norm_rope(const void *qkv, int64_t qkv_row_stride, const int64_t *positions, int64_t n_tokens,
                    int32_t num_heads, int32_t num_heads_k, int32_t head_dim, const void *q_norm_weight,
                    const void *k_norm_weight, float eps, const float *inv_freq, const float *q_head_scale,
                    const float *q_row_scale, void *q_out, int64_t q_row_stride, void *k_out,
                    int64_t k_row_stride, void *v_out, int64_t v_row_stride, const int32_t *kv_rows,
                    hipStream_t stream);

/* out[r, i] = bf16(silu(gate_up[r, i]) * gate_up[r, inter + i]) (Qwen3MLP act_fn(gate) * up on
 * the fused gate/up projection). */
int tg_silu_mul(const void *gate_up, int64_t gate_up_row_stride, int64_t n_rows, int32_t inter,
                void *out, int64_t out_row_stride, hipStream_t stream);

/* The finalized gate's scoring readout on the fused gate/up projection of its MLP branch:
 * scores[r] = bf16(w_row . bf16(bf16(silu(gate_up[r, :inter])) * gate_up[r, inter:])) as fp32 —
 * the branch Qwen3MLP whose down_proj is the absorbed (1, inter) row (gate_branch_hs,
 * gate_forward.py:491-524; build_gate_branch :261-342; load_gate e2e_gate_module.py:497-514), fed
 * z = post_attention_layernorm(a) of the gate layer's attention boundary a.  w_row: inter bf16. */
int tg_gate_branch_readout(const void *gate_up, int64_t gate_up_row_stride, int64_t n_rows, int32_t inter,
                           const void *w_row, float *scores, hipStream_t stream);

/* LM head on the rows that produce the next token (1 to 8 rows): out[b, v] = bf16(sum_d x[b, d] *
 * weight[v, d]) as fp32, accumulated in fp32 — F.linear(x, lm_head).float() on bf16 tensors, as
 * the reference's first-token / decode step computes the logits (gate_forward.py:1559-1562,
 * gate_decode.py:227).
 * weight: (vocab, dim) bf16 row-major (the embedding when tied); dim a multiple of 512. */
int tg_lm_head(const void *x, int64_t x_row_stride, int32_t n_rows, const void *weight, int64_t vocab,
               int32_t dim, float *out, int64_t out_row_stride, hipStream_t stream);

/* Decoder projections of a decode step (1 to 8 rows): out[b, v] = bf16(sum_d x[b, d] * weight[v, d]),
 * accumulated in fp32 and stored as bf16 — F.linear(x, weight) on bf16 tensors, the nn.Linear
 * q/k/v/o and gate/up/down projections of the Qwen3 layers the reference's decode loop calls
 * once per step and layer (gate_decode.py:210-226, inner.layers[li](...)).  The weight is read once
 * from HBM (the step is bound by streaming the layer weights).
 * weight: (n_out, dim) bf16 row-major; dim a multiple of 512; out: bf16 rows of out_row_stride. */
int tg_linear_rows(const void *x, int64_t x_row_stride, int32_t n_rows, const void *weight, int64_t n_out,
                   int32_t dim, void *out, int64_t out_row_stride, hipStream_t stream);

/* tg_linear_rows with the input formed from the previous sublayer's output, one launch instead of
 * two: x = RMSNorm(s) = bf16(norm_weight * s / sqrt(mean(s^2) + eps)) with s = bf16(h + residual)
 * (residual NULL: s = h), the same arithmetic and summation order as tg_rmsnorm; s is also written
 * to residual_out (NULL: not written), which must not be the residual input (every workgroup reads
 * it).  The decode step's input_layernorm -> q/k/v projection, post_attention_layernorm -> gate/up
 * projection and final norm -> LM head (Qwen3DecoderLayer / Qwen3Model.norm / lm_head as the
 * reference's decode loop calls them, gate_decode.py:210-227).  out_fp32: write the bf16 result
 * as fp32 (the logits), else as bf16. */
int tg_linear_rows_norm(const void *h, int64_t h_row_stride, const void *residual, int64_t residual_row_stride,
                        void *residual_out, int64_t residual_out_row_stride, const void *norm_weight, float eps,
                        int32_t n_rows, const void *weight, int64_t n_out, int32_t dim, void *out,
                        int64_t out_row_stride, int32_t out_fp32, hipStream_t stream);

/* tg_linear_rows of the SwiGLU product: x = bf16(silu(g) * u) of the gate/up rows [g | u] (inter
 * values each), as tg_silu_mul computes it — Qwen3MLP's down_proj(act_fn(gate_proj(x)) *
 * up_proj(x)) in the decode step (gate_decode.py:210-226). */
int tg_linear_rows_swiglu(const void *gate_up, int64_t gate_up_row_stride, int32_t n_rows, int32_t inter,
                          const void *weight, int64_t n_out, void *out, int64_t out_row_stride, hipStream_t stream);

/* Greedy next token: out[b] = argmax_v x[b, v] (int64) with torch.argmax's rules (a NaN wins, ties
 * go to the lower index) — the reference's logits.argmax(-1) of the first-token and decode steps
 * (gate_forward.py:1559-1562, gate_decode.py:227).  One launch and no memory clears, so a decode
 * step captured in a graph replays it safely.  x: fp32 rows of x_row_stride (a multiple of 4). */
int tg_argmax_rows(const float *x, int64_t x_row_stride, int32_t n_rows, int64_t n_cols, int64_t *out,
                   hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TOKENGATE_HIP_H */
