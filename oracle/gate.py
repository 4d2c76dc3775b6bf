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


def gate_bias(scores_art, keep, art_start, art_end, eps=RMS_EPS):
    """Per kept row: RMS-normalised score on article rows, 0 on prefix/suffix rows."""
    s = np.asarray(scores_art, dtype=np.float64)
    inv = 1.0 / np.sqrt(np.mean(s * s) + eps) if len(s) else 0.0
    out = np.zeros(len(keep))
    art = (keep >= art_start) & (keep < art_end)
    out[art] = s[keep[art] - art_start] * inv
    return out


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
