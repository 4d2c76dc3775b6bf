"""Oracle: the reference's own CPU execution of the hot path's two stages, restated in torch on the
host (TEST INFRASTRUCTURE ONLY: the parity tests in tests/ and bench.py's timed CPU baseline).

  sdpa_chunked — the reference's SDPA compatibility prefill, sdpa_causal
                 (tokengate/e2e_gate/attn/sdpa_compat.py:6-37): K / V heads repeated to the query
                 heads (GQA), the query axis cut into chunks of `chunk` rows (128 there), chunk
                 [start, end) attending to keys [0, end) through
                 torch.nn.functional.scaled_dot_product_attention with an additive float mask =
                 the per-key logit bias (broadcast over heads, _bias_bhs of
                 flex_attention_utils.py) where key <= query and -inf above the diagonal; SDPA's
                 default softmax scale 1/sqrt(head_dim).  Layout (B, H, S, D) as there.
  prune        — the reference's per-sample pruning (gate_forward.py:1396-1470, _keep_indices
                 :77-81): K_c = max(1, min(K, n_art)), torch.topk of the state span's scores,
                 torch.sort of the indices, torch.cat(arange(s), s + sorted, arange(e, L)), then
                 index_select of the kept rows of every tensor.

Pinned by tests/test_oracle_cpu_path.py: sdpa_chunked against the float64 numpy oracle
(oracle.attention.keybias_fwd) with bias_raw = bias_logit / scale; prune against
oracle.gate.keep_indices on tie-free scores (torch.topk's order among equal scores is
implementation-defined) and numpy row indexing.
"""
from typing import Optional, Sequence

import torch
import torch.nn.functional as F


def sdpa_chunked(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, bias_logit: Optional[torch.Tensor] = None,
                 chunk: int = 128, rows: Optional[range] = None) -> torch.Tensor:
    """Causal attention of q (B, H, S, D) over k / v (B, Hkv, S, D) with a per-key logit bias
    (B, S) or None.  rows: a range of query rows (whole chunks of the same chunking are the
    reference's own work for those rows); all rows by default.  Returns (B, H, len(rows), D)."""
    B, H, S, D = q.shape
    if k.shape[2] != S or H % k.shape[1]:
        raise ValueError("sdpa_chunked: aligned q / k and a KV head count dividing the query heads")
    g = H // k.shape[1]
    if g > 1:
        k = k.repeat_interleave(g, dim=1)
        v = v.repeat_interleave(g, dim=1)
    bias = bias_logit[:, None, None, :] if bias_logit is not None else None      # (B, 1, 1, S)
    rows = range(S) if rows is None else rows
    outs = []
    for start in range(rows.start, rows.stop, chunk):
        end = min(start + chunk, rows.stop)
        keep = torch.arange(end, device=q.device)[None, :] <= torch.arange(start, end, device=q.device)[:, None]
        mask = torch.zeros(end - start, end, dtype=q.dtype, device=q.device)
        if bias is not None:
            mask = mask + bias[..., :end].to(q.dtype)
        mask = mask.masked_fill(~keep, float("-inf"))
        outs.append(F.scaled_dot_product_attention(q[:, :, start:end], k[:, :, :end], v[:, :, :end],
                                                   attn_mask=mask, dropout_p=0.0))
    return torch.cat(outs, dim=2)


def prune(scores_art: torch.Tensor, K: int, art_start: int, art_end: int, seq_len: int,
          tensors: Sequence[torch.Tensor] = ()):
    """Keep indices (int64) of one sample and the kept rows of every tensor (row axis 0)."""
    n_art = art_end - art_start
    kc = max(1, min(int(K), n_art))
    top = torch.topk(scores_art, kc).indices
    top = torch.sort(top).values
    keep = torch.cat([torch.arange(art_start, dtype=torch.int64), art_start + top,
                      torch.arange(art_end, seq_len, dtype=torch.int64)])
    return keep, [t.index_select(0, keep) for t in tensors]
