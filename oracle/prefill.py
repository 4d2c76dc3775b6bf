"""Oracle: the gated prefill in float32 torch (TEST INFRASTRUCTURE ONLY).

Restates, for a Qwen3-shaped decoder given as float32 weights:
  * one decoder layer — transformers' Qwen3DecoderLayer / Qwen3Attention / Qwen3MLP /
    Qwen3RMSNorm / default RoPE (modeling_qwen3.py; transformers 5.19.0 pinned by the reference's
    uv.lock:3897-3898), with the attention replaced by the key-bias attention the reference
    routes through (qwen3_flex_attention.py:524-659): RMSNorm -> q/k/v projections -> per-head
    q/k RMSNorm -> RoPE (cos/sin of fp32 angles position * inv_freq) -> causal GQA attention with
    an additive per-key logit bias -> o_proj -> residual -> RMSNorm -> down(silu(gate) * up) ->
    residual.  Phase 2's temperature multiplies the query and the bias per head
    (_phase2_q_bias :433-473); in scaled-softmax mode the query is scaled by gamma_h * r_q and the
    bias by mean_h(gamma) * r_k, r = _ssmax_ratio (gate_forward.py:574-585).
  * prefill_batch_for_decode (gate_forward.py:1280-1580) in its own layout: prompts right-padded
    to the longest, layers 0..gate_layer over every position, per-sample scoring and top-K
    (K_clamped, keep = prefix + sorted top-K + suffix), kept rows gathered into a zero-padded
    (B, n_alloc) batch whose pad slots carry a -1e9 bias, layers above the gate on that batch
    with RoPE at the kept original positions, first token = argmax of the LM head at each
    sample's last kept row.
  * the finalized gate's MLP scoring branch (gate_branch_hs, gate_forward.py:491-524): score =
    w_row . (silu(W_gate z) * (W_up z)), z = post_attention_layernorm(a) of the gate layer's
    attention boundary a; with it the oracle still runs the gate layer whole on every row and
    gathers the kept rows afterwards — the unsplit form the split prefill must equal.
Pinned by tests/test_oracle_prefill.py against transformers' own Qwen3DecoderLayer and Qwen3MLP
(same weights, float32, eager attention; the branch as load_gate rebuilds it, a Qwen3MLP with a
(1, I) down_proj, e2e_gate_module.py:497-514) and by padded-vs-per-sequence equivalence.
"""
import math
from typing import List, Optional, Sequence

import numpy as np
import torch
import torch.nn.functional as F

from oracle import attention_torch as oat
from oracle import gate as og


def rms(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    return w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))


def rope_cos_sin(pos: torch.Tensor, inv_freq: torch.Tensor):
    ang = pos.float()[..., None] * inv_freq.float()            # fp32 product, as the rotary table
    emb = torch.cat([ang, ang], dim=-1)
    return emb.cos(), emb.sin()


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], dim=-1)


class Weights:
    """float32 copies of a decoder's weights (any object with the DecoderWeights fields)."""

    def __init__(self, wts, device="cpu"):
        s = wts.shape
        self.shape = s
        f = lambda t: t.detach().float().to(device)
        self.embed = f(wts.embed)
        self.final_norm = f(wts.final_norm)
        self.lm_head = f(wts.lm_head)
        self.inv_freq = f(wts.inv_freq)
        self.layers = []
        for lw in wts.layers:
            q, k, v = torch.split(f(lw.w_qkv), [s.n_heads * s.head_dim, s.n_kv_heads * s.head_dim,
                                                s.n_kv_heads * s.head_dim])
            g, u = torch.split(f(lw.w_gu), [s.d_ff, s.d_ff])
            self.layers.append(dict(ln1=f(lw.ln1), wq=q, wk=k, wv=v, q_norm=f(lw.q_norm), k_norm=f(lw.k_norm),
                                    wo=f(lw.w_o), ln2=f(lw.ln2), wg=g, wu=u, wd=f(lw.w_down)))


def layer(W: Weights, i: int, x: torch.Tensor, pos: torch.Tensor, bias_logit: Optional[torch.Tensor] = None,
          q_temp: Optional[torch.Tensor] = None, q_scale: Optional[torch.Tensor] = None,
          boundary: Optional[list] = None, rows: Optional[torch.Tensor] = None):
    """One decoder layer on a batch x (B, n, d) float32 at positions pos (B, n); bias_logit
    (B, H, n) per-key logit bias or None.  q_temp (H,): a per-head temperature multiplying the
    query and the bias (the fp32 form of the per-head branch of _phase2_q_bias); q_scale
    (B, H, n): a per-(head, row) query multiplier, the bias used as given (the caller passes the
    reference's bf16 Phase-2 values, phase2_tables).  Returns (x_out, k, v) with k/v
    (B, n, Hkv, D) after norm and RoPE; boundary (a list), if given, receives the attention
    residual a = x + o_proj(attn).  rows (int64, optional): evaluate only these query rows (each
    over every key it sees); x_out (and boundary) then hold those rows only."""
    s = W.shape
    L = W.layers[i]
    B, n, _ = x.shape
    H, Hkv, D = s.n_heads, s.n_kv_heads, s.head_dim
    h = rms(x, L["ln1"], s.rms_eps)
    k = (h @ L["wk"].t()).view(B, n, Hkv, D)
    v = (h @ L["wv"].t()).view(B, n, Hkv, D)
    k = rms(k, L["k_norm"], s.rms_eps)
    cos, sin = rope_cos_sin(pos, W.inv_freq)                  # (B, n, D)
    cos, sin = cos[:, :, None, :], sin[:, :, None, :]
    k = k * cos + rotate_half(k) * sin
    if rows is not None:
        rows = torch.as_tensor(rows, dtype=torch.int64, device=x.device)
        h, cos, sin, x = h[:, rows], cos[:, rows], sin[:, rows], x[:, rows]
        if q_scale is not None:
            q_scale = q_scale[:, :, rows]
    nq = h.shape[1]
    q = rms((h @ L["wq"].t()).view(B, nq, H, D), L["q_norm"], s.rms_eps)
    q = q * cos + rotate_half(q) * sin
    scale = 1.0 / math.sqrt(D)
    braw = None
    if bias_logit is not None:
        bl = bias_logit * q_temp[None, :, None] if q_temp is not None else bias_logit
        braw = bl / scale
    if q_temp is not None:
        q = q * q_temp[None, None, :, None]
    if q_scale is not None:
        q = q * q_scale.permute(0, 2, 1)[..., None]
    attn, _ = oat.fwd(q, k, v, braw, scale, causal=True, q_pos=rows)
    x = x + attn.reshape(B, nq, H * D) @ L["wo"].t()
    if boundary is not None:
        boundary.append(x)
    return mlp_half(W, i, x), k, v


def phase2_tables(head, scores_art: np.ndarray, keep: np.ndarray, art_start: int, art_end: int,
                  ratio=None):
    """The reference's Phase-2 constants of one sample (oracle.gate's bf16 chain): per Phase-2
    layer j, the key bias bias'[j] (H, n_kept) in logit units and the query multiplier
    s[j] (H, n_kept), both bf16 values as float32 tensors; s is None without a temperature.

    ratio: the kept rows' scaled-softmax ratio r as fp32 values, or None for the closed form
    (ssmax_ratio, float64) rounded to fp32.  The reference evaluates r with fp32 logs on its own
    device (_ssmax_ratio, gate_forward.py:573-584), so where r lies within an fp32 unit or two of
    a bf16 rounding point its bf16 value depends on that device's logf.  A parity test therefore
    checks a pipeline's r against the closed form to fp32 accuracy and passes it here."""
    gs = head.gate_scale.float().cpu().numpy()
    b = og.gate_bias_layers(scores_art, gs, gain=float(getattr(head, "bias_gain", 1.0)))
    gb = og.kept_bias_layers(b, keep, art_start, art_end)                   # (n, L2, H)
    temp = og.softplus32(head.attn_scale.float().cpu().numpy()) if head.attn_scale is not None else None
    ssmax = bool(getattr(head, "scaled_softmax", False)) and temp is not None
    if ssmax:
        r = (og.ssmax_ratio(keep) if ratio is None else np.asarray(ratio, dtype=np.float64)).astype(np.float32)
    else:
        r = None
    biases, scales = [], []
    for j in range(gb.shape[1]):
        tj = temp[j] if temp is not None else None
        biases.append(torch.from_numpy(og.phase2_bias(gb[:, j, :], tj, r).T.copy()))
        if tj is None:
            scales.append(None)
        else:
            sq = og.phase2_query_scale(tj, r)
            scales.append(torch.from_numpy(np.broadcast_to(sq, (sq.shape[0], len(keep))).copy()))
    return biases, scales


def mlp_half(W: Weights, i: int, a: torch.Tensor) -> torch.Tensor:
    """Layer i's MLP half: a + down(silu(gate) * up)(post_attention_layernorm(a))."""
    L = W.layers[i]
    h = rms(a, L["ln2"], W.shape.rms_eps)
    return a + (F.silu(h @ L["wg"].t()) * (h @ L["wu"].t())) @ L["wd"].t()


def head_scores(head, h: torch.Tensor) -> np.ndarray:
    """The scoring head on rows h (n, d), float64."""
    return og.score_mlp(h.double().numpy(), head.w1.float().cpu().numpy(), head.b1.cpu().numpy(),
                        head.w2.cpu().numpy(), head.b2)


def branch_scores_f32(head, a: torch.Tensor, ln2: torch.Tensor, eps: float) -> torch.Tensor:
    """The finalized gate's scoring branch on boundary rows a (n, d), float32:
    w_row . (silu(W_gate z) * (W_up z)), z = rms(a) * ln2 (gate_branch_hs, absorbed readout)."""
    wg, wu = head.w_gu.float().cpu().chunk(2, 0)
    z = rms(a.float(), ln2.float(), eps)
    return (F.silu(z @ wg.t()) * (z @ wu.t())) @ head.w_row.float().cpu()


def branch_scores(head, a: torch.Tensor, ln2: torch.Tensor, eps: float) -> torch.Tensor:
    """branch_scores_f32 rounded to bf16: the branch's output is the model dtype's
    (gate_forward.py:519-521), and the raw score the gate normalises is that bf16 value."""
    return branch_scores_f32(head, a, ln2, eps).to(torch.bfloat16).float()


def _is_branch(head) -> bool:
    return bool(getattr(head, "split_gate_layer", False))


def gate_scores(W: Weights, head, gate_layer: int, a: torch.Tensor, h: torch.Tensor) -> np.ndarray:
    """Scores of state rows, float64: the branch on the gate layer's boundary rows a, or the
    synthetic head on its output rows h."""
    if _is_branch(head):
        return branch_scores(head, a, W.layers[gate_layer]["ln2"], W.shape.rms_eps).double().numpy()
    return head_scores(head, h)


def prefill(W: Weights, head, ids_list: Sequence[Sequence[int]], art_starts, art_ends, gate_layer: int, K,
            keep_override: Optional[List[np.ndarray]] = None, scores_override: Optional[List[np.ndarray]] = None):
    """The reference's padded-batch prefill.  keep_override / scores_override (per sample) replace
    the oracle's own selection / scores (to compare layouts and numerics on the same keep set).
    Returns dict(first_tokens, logits (B, vocab), keep (list), h_gate (list of (len, d)),
    h_last (B, n_alloc, d), kept_bias (list))."""
    s = W.shape
    B = len(ids_list)
    lens = [len(x) for x in ids_list]
    S = max(lens)
    ids = torch.zeros(B, S, dtype=torch.long)
    for b, x in enumerate(ids_list):
        ids[b, :lens[b]] = torch.as_tensor(list(x), dtype=torch.long)
    x = W.embed[ids]
    pos = torch.arange(S)[None, :].expand(B, S)
    bnd = []
    for i in range(gate_layer + 1):
        x, _, _ = layer(W, i, x, pos, boundary=bnd)
    a = bnd[-1]
    Ks = K if isinstance(K, (list, tuple)) else [K] * B
    keeps, biases, h_gate, scs = [], [], [], []
    for b in range(B):
        st, en = art_starts[b], art_ends[b]
        h_gate.append(x[b, :lens[b]].clone())
        sc = (scores_override[b] if scores_override is not None
              else gate_scores(W, head, gate_layer, a[b, st:en], x[b, st:en]))
        kp = keep_override[b] if keep_override is not None else og.keep_indices(sc, Ks[b], st, en, lens[b])
        keeps.append(np.asarray(kp, dtype=np.int64))
        scs.append(np.asarray(sc, dtype=np.float32))
        biases.append(og.gate_bias(scs[-1], keeps[-1], st, en, gain=float(getattr(head, "bias_gain", 1.0))))
    n_alloc = max(len(k) for k in keeps)
    hp = torch.zeros(B, n_alloc, s.d_model)
    kpos = torch.zeros(B, n_alloc, dtype=torch.long)
    if tuple(head.gate_scale.shape) != (s.n_layers - gate_layer - 1, s.n_heads):
        raise ValueError("gate_scale must be (layers above the gate, heads)")
    L2 = s.n_layers - gate_layer - 1
    # pad slots carry -1e9 (gate_forward.py:1467-1469); their query multiplier is irrelevant
    bl = torch.full((L2, B, s.n_heads, n_alloc), -1e9)
    qs = torch.ones(L2, B, s.n_heads, n_alloc)
    any_scale = False
    for b in range(B):
        kt = torch.as_tensor(keeps[b])
        n = len(kt)
        hp[b, :n] = x[b, kt]
        kpos[b, :n] = kt
        bj, sj = phase2_tables(head, scs[b], keeps[b], art_starts[b], art_ends[b])
        for j in range(L2):
            bl[j, b, :, :n] = bj[j]
            if sj[j] is not None:
                qs[j, b, :, :n] = sj[j]
                any_scale = True
    xx = hp
    for j, i in enumerate(range(gate_layer + 1, s.n_layers)):
        xx, _, _ = layer(W, i, xx, kpos, bias_logit=bl[j], q_scale=qs[j] if any_scale else None)
    last = torch.tensor([len(k) - 1 for k in keeps])
    rows = xx[torch.arange(B), last]
    logits = rms(rows, W.final_norm, s.rms_eps) @ W.lm_head.t()
    return dict(first_tokens=logits.argmax(-1), logits=logits, keep=keeps, h_gate=h_gate, h_last=xx,
                kept_bias=biases)


def layer_with_past(W: Weights, i: int, x: torch.Tensor, pos: torch.Tensor, k_past: torch.Tensor,
                    v_past: torch.Tensor, bias_logit: Optional[torch.Tensor] = None,
                    q_temp: Optional[torch.Tensor] = None):
    """One decoder layer for new rows x (1, n, d) at positions pos (1, n) that attend over cached
    keys / values k_past, v_past (1, m, Hkv, D) and then over themselves causally; bias_logit
    (1, H, m + n) per key (past then new) or None.  Returns (x_out, k_new, v_new)."""
    s = W.shape
    L = W.layers[i]
    _, n, _ = x.shape
    H, Hkv, D = s.n_heads, s.n_kv_heads, s.head_dim
    h = rms(x, L["ln1"], s.rms_eps)
    q = rms((h @ L["wq"].t()).view(1, n, H, D), L["q_norm"], s.rms_eps)
    k = rms((h @ L["wk"].t()).view(1, n, Hkv, D), L["k_norm"], s.rms_eps)
    v = (h @ L["wv"].t()).view(1, n, Hkv, D)
    cos, sin = rope_cos_sin(pos, W.inv_freq)
    cos, sin = cos[:, :, None, :], sin[:, :, None, :]
    q = q * cos + rotate_half(q) * sin
    k = k * cos + rotate_half(k) * sin
    scale = 1.0 / math.sqrt(D)
    braw = None
    if bias_logit is not None:
        bl = bias_logit * q_temp[None, :, None] if q_temp is not None else bias_logit
        braw = bl / scale
    if q_temp is not None:
        q = q * q_temp[None, None, :, None]
    attn, _ = oat.fwd(q, torch.cat([k_past, k], 1), torch.cat([v_past, v], 1), braw, scale, causal=True)
    x = x + attn.reshape(1, n, H * D) @ L["wo"].t()
    h = rms(x, L["ln2"], s.rms_eps)
    x = x + (F.silu(h @ L["wg"].t()) * (h @ L["wu"].t())) @ L["wd"].t()
    return x, k, v


def decode_logits(W: Weights, head, ids: Sequence[int], art_start: int, art_end: int, gate_layer: int,
                  keep: np.ndarray, gen: Sequence[int], prune_below_gate: bool = False):
    """Teacher-forced logits of the reference's decode for one sample (generate_batch,
    gate_decode.py:88-262, default form): the generated tokens, at positions last kept position
    + 1, + 2, ..., go through layers 0..gate_layer attending over the prompt's cache at those
    layers (every prompt row, or only the kept rows with prune_below_gate) and through the layers
    above over the kept rows, where prompt keys keep their gate bias and generated keys carry 0.
    Returns (1 + len(gen), vocab): the logits after the last kept row (the first token) and after
    each generated token."""
    s = W.shape
    L, g = len(ids), len(gen)
    kp = torch.as_tensor(np.asarray(keep, dtype=np.int64))
    nxt = int(kp[-1]) + 1
    gpos = (nxt + torch.arange(g))[None]
    x = W.embed[torch.as_tensor(list(ids), dtype=torch.long)][None]
    xg = W.embed[torch.as_tensor(list(gen), dtype=torch.long)][None]
    pos = torch.arange(L)[None]
    bnd = []
    for i in range(gate_layer + 1):
        xn, k, v = layer(W, i, x, pos, boundary=bnd)
        if prune_below_gate:
            k, v = k[:, kp], v[:, kp]
        if g:
            xg, _, _ = layer_with_past(W, i, xg, gpos, k, v)
        x = xn
    sc = gate_scores(W, head, gate_layer, bnd[-1][0, art_start:art_end], x[0, art_start:art_end])
    biases, scales = phase2_tables(head, np.asarray(sc, dtype=np.float32), np.asarray(keep), art_start, art_end)
    xx = torch.cat([x[0, kp], xg[0]])[None]
    pos2 = torch.cat([kp[None], gpos], 1)
    n_kept, H = len(kp), s.n_heads
    temp = og.softplus32(head.attn_scale.float().cpu().numpy()) if head.attn_scale is not None else None
    ssmax = bool(getattr(head, "scaled_softmax", False)) and temp is not None
    # a generated token's ratio: slot n_kept + 1 + i at position nxt + i (FormDecodeState.step)
    r_gen = og.ssmax_ratio(pos2.numpy())[0, n_kept:].astype(np.float32) if ssmax else None
    for j, i in enumerate(range(gate_layer + 1, s.n_layers)):
        bl = torch.cat([biases[j], torch.zeros(H, g)], 1)[None]            # generated keys: 0
        qs = None
        if scales[j] is not None:
            if ssmax:
                sg = [og.decode_query_scale(temp[j], r_gen[t]) for t in range(g)]
            else:
                sg = [og.phase2_query_scale(temp[j])[:, 0]] * g
            qs = torch.cat([scales[j]] + [torch.from_numpy(np.asarray(v, np.float32))[:, None] for v in sg], 1)[None]
        xx, _, _ = layer(W, i, xx, pos2, bias_logit=bl, q_scale=qs)
    rows = xx[0, len(kp) - 1:]
    return rms(rows, W.final_norm, s.rms_eps) @ W.lm_head.t()
