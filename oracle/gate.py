"""Oracle: gate-path selection and packing in numpy (TEST INFRASTRUCTURE ONLY).

Restates tokengate/e2e_gate/gate_module/gate_forward.py:
  * K_clamped = max(1, min(K, n_art))                          (:1409-1410)
  * topk over the article scores                               (_select_topk_or_random :84-99;
    torch.topk's tie order is implementation-defined — this library's rule, applied here, is that
    among equal scores the lower position wins; -0.0 equals +0.0; NaN ranks above +inf)
  * keep = cat(arange(s), s + sort(topk), arange(e, seq_len)) (:1417-1421 == _keep_indices :77-81)
  * gathers of hidden / K / V rows at the kept positions       (:1454-1522)
  * gate bias of kept rows: RMS-normalised article score (E2EGate.forward,
    e2e_gate_module.py:348-385, eps 1e-6 :74) on kept article rows, 0 on prefix/suffix rows
    (build_gate_bias_vectorized :968-1036)
and the synthetic scoring head Linear(2048->256) -> SiLU -> Linear(256->1).

The reference's arithmetic chain from score to Phase-2 softmax input, restated with its own
rounding points (the model runs in bf16, the gate's parameters are fp32):
  * b[j, l, h] = fp32(gain * fp32(raw_j * rsqrt(mean_art(raw^2) + eps))) * softplus(gate_scale[l, h])
    in fp32: transformers' Qwen3RMSNorm(1, eps) over the sequence axis (E2EGate._seq_rms_norm_qwen,
    e2e_gate_module.py:299, :342-344, forward :363-385); raw is the branch's bf16 score in fp32
    (gate_forward.py:1399-1405)
  * selection key agg_j = sum_h b[j, 0, h] * (1/H) (aggregate :387-399); the threshold mode keeps
    the tokens with sigmoid(agg_j) >= tau, or the argmax when none passes (_select_threshold,
    gate_forward.py:102-125)
  * stored bias gb = bf16(b) on kept article rows, 0 on prefix / suffix rows
    (build_gate_bias_vectorized, per_layer_gate branch, gate_forward.py:995-1008; model dtype
    :1450, :1462-1466)
  * Phase 2 (_phase2_q_bias / _ssmax_s_eff, qwen3_flex_attention.py:417-473), all in bf16:
    scaled softmax: s_eff[h, q] = bf16(bf16(gamma_h) * bf16(r_q)), q' = bf16(q * s_eff),
    bias' = bf16(gb * bf16(mean_h s_eff[:, key])); per-head temperature: s = bf16(gamma_h),
    q' = bf16(q * s), bias' = bf16(gb * s); gamma = softplus(attn_scale[l]) in fp32
    (attn_scale_eff :302-305, installed per layer by _apply_gate_bias gate_forward.py:647-660)
  * decode (FormDecodeState.step / _decode_scaled_forward, qwen3_flex_attention.py:1090-1101,
    :374-400): the new token's query scale is bf16(fp32(gamma_h * r)), the cached keys keep
    bias' (decode_phase2_layer_tensors :1010-1017), generated keys carry 0
  * the attention kernel receives bias_raw = fp32(bias') / scale (flash_attn_key_bias,
    kernels/fa2bias/keybias.py:86)
Pinned against vectors written by the reference's own functions (tests/golden/gate_chain.npz,
tests/golden/make_gate_chain_vectors.py) and against transformers' Qwen3RMSNorm.
"""
import numpy as np

RMS_EPS = 1e-6


def k_clamped(K, n_art):
    return 0 if n_art <= 0 else max(1, min(int(K), int(n_art)))


def topk_order(scores):
    """Indices of `scores` ordered best-first: larger score first, NaN above everything, equal
    scores (incl. -0.0 == +0.0) by ascending index."""
    s = np.asarray(scores, dtype=np.float64)
    nan = np.isnan(s)
    key = np.where(nan, 0.0, -s)
    return np.lexsort((np.arange(len(s)), key, ~nan))


def select_topk(scores, K):
    """Article-relative indices of the kept tokens, ascending (sort(topk(scores, K_c)))."""
    kc = k_clamped(K, len(scores))
    return np.sort(topk_order(scores)[:kc])


def keep_indices(scores_art, K, art_start, art_end, seq_len):
    topk = select_topk(scores_art, K)
    return np.concatenate([np.arange(art_start), art_start + topk, np.arange(art_end, seq_len)]).astype(np.int64)


def bf16(x):
    """float32 values rounded to the nearest bfloat16 (ties to even), returned as float32."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    r = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(a), a, r).astype(np.float32)


def softplus32(x):
    """torch.nn.functional.softplus in fp32 (beta 1, threshold 20), correctly rounded."""
    x = np.asarray(x, dtype=np.float32)
    return np.where(x > 20, x, np.log1p(np.exp(x.astype(np.float64)))).astype(np.float32)


def seq_rms_norm(raw, eps=RMS_EPS, gain=1.0):
    """Qwen3RMSNorm(1, eps) applied over the sequence axis, fp32: gain * (x * rsqrt(mean(x^2) +
    eps)) with x the article's fp32 scores (E2EGate._seq_rms_norm_qwen).  The mean is the
    correctly rounded fp32 mean (torch's summation order can move its last bit)."""
    x = np.asarray(raw, dtype=np.float32)
    if x.size == 0:
        return x.copy()
    var = np.float32(np.mean(np.square(x.astype(np.float64))))
    inv = np.float32(1.0 / np.sqrt(np.float64(np.float32(var + np.float32(eps)))))
    return (np.float32(gain) * (x * inv).astype(np.float32)).astype(np.float32)


def gate_bias(scores_art, keep, art_start, art_end, eps=RMS_EPS, gain=1.0):
    """Per kept row: the RMS-normalised score (seq_rms_norm, fp32) on article rows, 0 on
    prefix/suffix rows."""
    keep = np.asarray(keep)
    bn = seq_rms_norm(scores_art, eps, gain)
    out = np.zeros(len(keep), dtype=np.float32)
    art = (keep >= art_start) & (keep < art_end)
    out[art] = bn[keep[art] - art_start]
    return out


def gate_bias_layers(scores_art, gate_scale, eps=RMS_EPS, gain=1.0):
    """E2EGate.forward: (n_art, L2, H) fp32 = seq_rms_norm(scores) * softplus(gate_scale[l, h])."""
    bn = seq_rms_norm(scores_art, eps, gain)
    return (bn[:, None, None] * softplus32(gate_scale)[None]).astype(np.float32)


def aggregate(b):
    """E2EGate.aggregate: the first Phase-2 layer's slot, summed over heads with weights 1/H
    (fp32, heads added in order)."""
    b0 = np.asarray(b, dtype=np.float32)[:, 0, :]
    H = b0.shape[1]
    if H == 1:
        return b0[:, 0].copy()
    w = np.float32(1.0 / H)
    acc = np.zeros(b0.shape[0], dtype=np.float32)
    for h in range(H):
        acc = (acc + (b0[:, h] * w).astype(np.float32)).astype(np.float32)
    return acc


def kept_bias_layers(b, keep, art_start, art_end):
    """build_gate_bias_vectorized (per_layer_gate) stored in bf16: (n_kept, L2, H), the kept
    article rows' b, 0 on prefix / suffix rows."""
    b = np.asarray(b, dtype=np.float32)
    keep = np.asarray(keep)
    out = np.zeros((len(keep),) + b.shape[1:], dtype=np.float32)
    art = (keep >= art_start) & (keep < art_end)
    out[art] = b[keep[art] - art_start]
    return bf16(out)


def phase2_query_scale(temp, ratio=None):
    """Phase-2 query multiplier s (H, n) for one layer (bf16 values): scaled softmax
    bf16(bf16(gamma_h) * bf16(r_q)); per-head temperature bf16(gamma_h) ((H, 1)).  temp: fp32
    softplus(attn_scale[l]) (H,); ratio: fp32 r of the query rows (n,) or None."""
    g = bf16(temp)
    if ratio is None:
        return g[:, None]
    return bf16(g[:, None] * bf16(ratio)[None, :])


def phase2_bias(gb, temp, ratio=None):
    """Phase-2 key bias bias' (n, H) (bf16 values, logit units) for one layer from the stored
    bias gb (n, H): scaled softmax bf16(gb * bf16(mean_h s_eff[h, key])) with s_eff at the key's
    own ratio; per-head temperature bf16(gb * bf16(gamma_h)); no temperature: gb."""
    gb = np.asarray(gb, dtype=np.float32)
    if temp is None:
        return gb.copy()
    s = phase2_query_scale(temp, ratio)                       # (H, n) or (H, 1)
    if ratio is None:
        return bf16(gb * s[:, 0][None, :])
    H = s.shape[0]
    sb = bf16((s.astype(np.float32).sum(0, dtype=np.float32) / np.float32(H)).astype(np.float32))
    return bf16(gb * sb[:, None])


def phase2_query(q, s):
    """q' = bf16(q * s) for query rows q (H, n, D) (bf16 values) and the multiplier s (H, n|1)."""
    return bf16(np.asarray(q, dtype=np.float32) * np.asarray(s, dtype=np.float32)[:, :, None])


def decode_query_scale(temp, r):
    """The decode token's query multiplier bf16(fp32(gamma_h * r)) (H,) (FormDecodeState.step)."""
    return bf16((np.asarray(temp, dtype=np.float32) * np.float32(r)).astype(np.float32))


def selection_values(scores_art, gate_scale, eps=RMS_EPS, gain=1.0):
    """The selection value agg_j of every state token (aggregate of E2EGate.forward's bias,
    e2e_gate_module.py:363-399): the value _select_indices compares (gate_forward.py:1411-1412)."""
    return aggregate(gate_bias_layers(scores_art, gate_scale, eps, gain))


def argmax_first(x):
    """torch.argmax of a 1-D float tensor: the first maximal entry, a NaN counting as maximal."""
    x = np.asarray(x, dtype=np.float32)
    nan = np.isnan(x)
    if nan.any():
        return int(np.argmax(nan))
    return int(np.argmax(x))


def select_threshold(agg, b_star):
    """_select_threshold (gate_forward.py:102-125): article-relative indices, ascending, of the
    tokens with sigmoid(agg) >= tau, written as agg >= b_star (b_star: the least fp32 value whose
    sigmoid reaches tau; NaN when none does, -inf when all do); NaN never passes; when nothing
    passes, the single argmax."""
    agg = np.asarray(agg, dtype=np.float32)
    with np.errstate(invalid="ignore"):
        idx = np.nonzero(agg >= np.float32(b_star))[0]
    if len(idx) == 0 and len(agg) > 0:
        return np.array([argmax_first(agg)], dtype=np.int64)
    return idx.astype(np.int64)


def threshold_keep_indices(agg, b_star, art_start, art_end, seq_len):
    """keep = [0, s) + s + select_threshold + [e, seq_len) (gate_forward.py:1412-1421)."""
    sel = select_threshold(agg, b_star)
    return np.concatenate([np.arange(art_start), art_start + sel, np.arange(art_end, seq_len)]).astype(np.int64)


def select_and_pack(scores, seqs):
    """seqs: list of (row_start, seq_len, art_start, art_end, K).  Returns the packed keep list
    (int64), kept_start per sequence and the per-sequence K_clamped."""
    keeps, starts, kcs, off = [], [], [], 0
    for (r0, L, s, e, K) in seqs:
        kp = keep_indices(scores[r0 + s:r0 + e], K, s, e, L)
        keeps.append(kp)
        starts.append(off)
        kcs.append(k_clamped(K, e - s))
        off += len(kp)
    return np.concatenate(keeps) if keeps else np.zeros(0, np.int64), starts, kcs


def score_mlp(x, w1, b1, w2, b2):
    """float64 evaluation of w2 . silu(W1 x + b1) + b2 for each row of x."""
    h = np.asarray(x, np.float64) @ np.asarray(w1, np.float64).T + np.asarray(b1, np.float64)
    return (h / (1.0 + np.exp(-h))) @ np.asarray(w2, np.float64) + float(b2)


def ssmax_ratio(kept_positions):
    """r_q = min(1, ln max(m_q, 2) / ln max(p_q + 1, 2)), m_q the 1-based slot, p_q the original
    position (gate_forward.py:574-585)."""
    p = np.asarray(kept_positions, dtype=np.float64)
    m = np.maximum(np.arange(1, p.shape[-1] + 1, dtype=np.float64), 2.0)
    pos = np.maximum(p + 1.0, 2.0)
    return np.minimum(np.log(m) / np.log(pos), 1.0)
