"""Greedy decode after the gated prefill, over the pruned KV caches.

Follows generate_batch (tokengate/e2e_gate/decode/gate_decode.py:88-262) in its default form:
layers at or below the gate attend over the full prompt cache (prune_below_gate=False) plus the
generated tokens; layers above it attend over the kept rows, which keep their gate bias and
per-head temperature through decode (decode_phase2_form=True, FormDecodeState
qwen3_flex_attention.py:978-1117) while generated tokens carry bias 0; positions continue from
each sequence's last kept original position (+1 per step); generation stops when every row has
produced EOS, and answers are cut at the first EOS (gate_decode.py:241-257).

Cache layout: the prefill run with decode_headroom >= the steps to come leaves every layer's
cache with that many free rows after each sequence (decoder.CacheGap), and the decode appends in
place: each step's new K/V rows are written by the q/k-norm + RoPE kernel straight into row
seg[b] + used[b] of each sequence's segment, and each layer's attention is ONE varlen launch
(tg_keybias_varlen_kv_fwd) with one query row per sequence over its segment's used rows.  A
prefill without enough headroom is re-laid out once (one copy per layer) into that layout.
The per-step counters live on the device, so nothing in a step synchronises with the host, and
every step launches the same kernels with the same arguments: with graph=True the second and
later steps replay one captured HIP graph of the whole step (about 250 launches), whose inputs
and outputs are static device buffers; the first step runs eagerly and warms every kernel and
library handle the capture records.
"""
import math
from dataclasses import dataclass
from typing import List, Optional

import torch

from tokengate_amd.decoder import (CacheGap, DecoderWeights, LayerKV, argmax_rows, h2d, linear_rows, linear_rows_norm,
                                   linear_rows_swiglu, logits_last, qk_norm_rope, rmsnorm, silu_mul,
                                   varlen_kv_attention)
from tokengate_amd.gate import ScoringHead
from tokengate_amd.prefill import PrefillResult


@dataclass
class _Group:
    """Layers that share one cache geometry (at / below the gate, or above it)."""
    seg: List[int]            # host: segment start per sequence
    n0: List[int]             # host: rows per sequence when decoding starts
    gap: int


def _relayout(kv: LayerKV, cu: List[int], gap: int) -> LayerKV:
    """Copy a back-to-back cache (cu layout) into one with `gap` free rows after each sequence."""
    B = len(cu) - 1
    rows = cu[-1] + B * gap
    k = torch.zeros(rows, *kv.k.shape[1:], dtype=kv.k.dtype, device=kv.k.device)
    v = torch.zeros_like(k)
    for b in range(B):
        s = cu[b] + b * gap
        k[s:s + cu[b + 1] - cu[b]] = kv.k[cu[b]:cu[b + 1]]
        v[s:s + cu[b + 1] - cu[b]] = kv.v[cu[b]:cu[b + 1]]
    return LayerKV(k, v)


class DecodeState:
    # most rows per step for which the norms and the SwiGLU product are folded into the projections
    max_fused_rows = 2

    def __init__(self, wts: DecoderWeights, head: ScoringHead, gate_layer: int, pf: PrefillResult,
                 max_new_tokens: int, prune_below_gate: bool = False, graph: bool = False, fused: bool = True):
        shape = wts.shape
        self.wts, self.shape = wts, shape
        dev = wts.device
        B = len(pf.n_kept)
        self.B = B
        self.gate_layer = gate_layer
        L2 = shape.n_layers - gate_layer - 1
        cu_below = pf.cu_prompt if not prune_below_gate else pf.cu_kept
        in_place = pf.decode_headroom >= max_new_tokens and pf.cache_above is not None \
            and pf.cache_below is not None
        gap = pf.decode_headroom if in_place else max_new_tokens
        self.in_place = in_place
        self.kv: List[LayerKV] = []
        for l in range(shape.n_layers):
            if in_place:
                self.kv.append(pf.kv[l])
            else:                      # the prefill left no room: one copy per layer
                self.kv.append(_relayout(pf.kv[l], cu_below if l <= gate_layer else pf.cu_kept, gap))
        groups = []
        for cu in (cu_below, pf.cu_kept):
            groups.append(_Group([cu[b] + b * gap for b in range(B)], [cu[b + 1] - cu[b] for b in range(B)], gap))
        self.groups = groups
        # device state: segment starts and rows used, (2, B) int32 (group 0: at / below the gate)
        hdr = torch.tensor([g.seg for g in groups] + [g.n0 for g in groups], dtype=torch.int32)
        d = h2d(hdr, dev)
        self.seg_dev, self.used = d[:2].contiguous(), d[2:].contiguous()
        self.cap_k = [max(g.n0) + max_new_tokens for g in groups]   # longest key run either group reaches
        # Phase-2 layers: key bias by (sequence, head, key), 0 on generated keys (decode_phase2_layer_tensors,
        # qwen3_flex_attention.py:1010-1017), and the per-head query scale
        if in_place and pf.phase2_bias_seq is not None and pf.phase2_bias_seq.shape[-1] >= self.cap_k[1]:
            self.bias = pf.phase2_bias_seq
        else:
            W = self.cap_k[1]
            self.bias = torch.zeros(L2, B, shape.n_heads, W, dtype=torch.float32, device=dev)
            for b in range(B):
                n = pf.n_kept[b]
                self.bias[:, b, :, :n] = pf.phase2_bias[:, :, pf.cu_kept[b]:pf.cu_kept[b + 1]]
        q_head = head.decode_query_head()
        self.qscale = [q_head[j].contiguous() for j in range(L2)] if q_head is not None else None
        last = torch.tensor([pf.cu_kept[b + 1] - 1 for b in range(B)], dtype=torch.int64)
        self.next_pos = pf.kept_positions.index_select(0, h2d(last, dev)) + 1
        self.ssmax = pf.kept_ratio is not None
        self.n_kept_f = h2d(torch.tensor([float(x) for x in pf.n_kept], dtype=torch.float32), dev)
        self.cu_q = torch.arange(B + 1, dtype=torch.int32, device=dev)
        self.rows_b = torch.arange(B, device=dev)
        self.steps = 0
        self.step_f = torch.zeros((), dtype=torch.float32, device=dev)   # steps taken, on the device
        self.max_new_tokens = max_new_tokens
        self.use_graph = graph
        self.fused = fused
        self._graph = None
        self._tok_in = self._tok_out = None

    @torch.no_grad()
    def step(self, tokens: torch.Tensor) -> torch.Tensor:
        """Appends one token per sequence (tokens (B,) int64) and returns the next greedy tokens."""
        if self.steps >= self.max_new_tokens:
            raise RuntimeError("DecodeState: more steps than max_new_tokens (the caches are full)")
        if not self.use_graph or self.steps == 0:
            out = self._body(tokens)
        else:
            if self._graph is None:
                self._tok_in = tokens.clone()
                self._graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(self._graph):
                    self._tok_out = self._body(self._tok_in)
            self._tok_in.copy_(tokens)
            self._graph.replay()
            out = self._tok_out.clone()
        self.steps += 1
        return out

    def _body(self, tokens: torch.Tensor) -> torch.Tensor:
        """One decode step as device work only (no host synchronisation, no host-side state), so
        that it can be captured and replayed."""
        s, w = self.shape, self.wts
        B = self.B
        dev = tokens.device
        x = torch.nn.functional.embedding(tokens, w.embed)
        # rows beyond max_fused_rows take the separate norm / SwiGLU launches
        fused = self.fused and B <= self.max_fused_rows and s.d_model % 512 == 0 and s.d_ff % 512 == 0
        res = None if fused else x.clone()
        normed = torch.empty_like(x)
        hid = torch.empty_like(x)
        qkv = torch.empty(B, s.qkv_dim, dtype=x.dtype, device=dev)
        att = torch.empty(B, s.n_heads, s.head_dim, dtype=x.dtype, device=dev)
        lse = torch.empty(s.n_heads, B, dtype=torch.float32, device=dev)
        rows = self.seg_dev + self.used          # the new token's cache row in each group, (2, B)
        self.used += 1
        r_dec = None
        if self.ssmax:   # the new token's own ratio: slot n_kept + 1 + step at position next_pos
            m = (self.n_kept_f + 1.0 + self.step_f).clamp(min=2.0)
            p = (self.next_pos.to(torch.float32) + 1.0).clamp(min=2.0)
            r_dec = (torch.log(m) / torch.log(p)).clamp(max=1.0)
        scale = 1.0 / math.sqrt(s.head_dim)
        if fused:
            # each norm is folded into the projection after it, and the SwiGLU product into the down
            # projection; the residual stream alternates between two buffers (a fused norm reads one
            # and writes the other)
            rbuf = [torch.empty_like(x), torch.empty_like(x)]
            cur = 0
        for l in range(s.n_layers):
            lw = w.layers[l]
            g = 0 if l <= self.gate_layer else 1
            j = l - self.gate_layer - 1
            if fused:
                linear_rows_norm(x if l == 0 else hid, lw.ln1, s.rms_eps, lw.w_qkv, residual=None if l == 0 else rbuf[cur],
                                 residual_out=rbuf[1 - cur], out=qkv)
                cur = 1 - cur
            elif l == 0:
                rmsnorm(res, lw.ln1, s.rms_eps, out=normed)
            else:
                rmsnorm(hid, lw.ln1, s.rms_eps, residual=res, residual_out=res, out=normed)
            if not fused:
                linear_rows(normed, lw.w_qkv, out=qkv)
            kv = self.kv[l]
            q = qk_norm_rope(qkv, self.next_pos, lw, s, w.inv_freq, kv.k, kv.v,
                             self.qscale[j] if (g and self.qscale is not None) else None,
                             r_dec if (r_dec is not None and g) else None, kv_rows=rows[g])
            varlen_kv_attention(q, kv.k, kv.v, self.cu_q, self.seg_dev[g], self.used[g], 1, self.cap_k[g], scale,
                                self.bias[j] if g else None, out=att, lse=lse)
            linear_rows(att.view(B, -1), lw.w_o, out=hid)
            if fused:
                gu = linear_rows_norm(hid, lw.ln2, s.rms_eps, lw.w_gu, residual=rbuf[cur], residual_out=rbuf[1 - cur])
                cur = 1 - cur
                linear_rows_swiglu(gu, lw.w_down, out=hid)
            else:
                rmsnorm(hid, lw.ln2, s.rms_eps, residual=res, residual_out=res, out=normed)
                act = silu_mul(linear_rows(normed, lw.w_gu))
                linear_rows(act, lw.w_down, out=hid)
        self.next_pos += 1
        self.step_f += 1.0
        if fused:   # every row produces a token: the final norm folds into the LM head
            logits = linear_rows_norm(hid, w.final_norm, s.rms_eps, w.lm_head, residual=rbuf[cur], out_fp32=True)
        else:
            logits = logits_last(w, hid + res, self.rows_b)
        self.last_logits = logits
        return argmax_rows(logits)
