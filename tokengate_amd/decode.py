"""Greedy decode after the gated prefill, over the pruned KV caches.

Follows generate_batch (tokengate/e2e_gate/decode/gate_decode.py:88-262) in its default form:
layers at or below the gate attend over the full prompt cache (prune_below_gate=False) plus the
generated tokens; layers above it attend over the kept rows, which keep their gate bias and
per-head temperature through decode (decode_phase2_form=True, FormDecodeState
qwen3_flex_attention.py:978-1117) while generated tokens carry bias 0; positions continue from
each sequence's last kept original position (+1 per step); generation stops when every row has
produced EOS, and answers are cut at the first EOS (gate_decode.py:241-257).

Every decode attention is the key-bias forward (tg_keybias_fwd) with one query row over the
sequence's cache segment; the per-token ops are the prefill's fused kernels.  Caches are copied
once, after the first token, into per-sequence segments with room for the generated rows.
"""
import math
from dataclasses import dataclass
from typing import List, Optional

import torch

from tokengate_amd import _lib
from tokengate_amd.decoder import DecoderWeights, h2d, logits_last, qk_norm_rope, rmsnorm, silu_mul
from tokengate_amd.gate import ScoringHead
from tokengate_amd.prefill import PrefillResult


@dataclass
class _LayerCache:
    k: torch.Tensor          # (rows, Hkv, D): sequence b's segment starts at seg[b]
    v: torch.Tensor
    seg: List[int]
    n: List[int]             # valid rows per sequence (grows by one per step)
    bias: Optional[torch.Tensor] = None    # (B, H, cap) fp32 raw units, Phase-2 layers
    qscale: Optional[torch.Tensor] = None  # (H,) fp32


class DecodeState:
    def __init__(self, wts: DecoderWeights, head: ScoringHead, gate_layer: int, pf: PrefillResult,
                 max_new_tokens: int, prune_below_gate: bool = False):
        shape = wts.shape
        self.wts, self.shape = wts, shape
        dev = wts.device
        B = len(pf.n_kept)
        self.B = B
        q_head = head.decode_query_head()
        self.layers: List[_LayerCache] = []
        for l in range(shape.n_layers):
            below = l <= gate_layer
            cu = pf.cu_prompt if (below and not prune_below_gate) else pf.cu_kept
            n = [cu[b + 1] - cu[b] for b in range(B)]
            seg, off = [], 0
            for b in range(B):
                seg.append(off)
                off += n[b] + max_new_tokens
            k = torch.zeros(off, shape.n_kv_heads, shape.head_dim, dtype=torch.bfloat16, device=dev)
            v = torch.zeros_like(k)
            for b in range(B):
                k[seg[b]:seg[b] + n[b]] = pf.kv[l].k[cu[b]:cu[b + 1]]
                v[seg[b]:seg[b] + n[b]] = pf.kv[l].v[cu[b]:cu[b + 1]]
            lc = _LayerCache(k, v, seg, list(n))
            if not below:
                j = l - gate_layer - 1
                cap = max(n) + max_new_tokens
                # kept keys keep their Phase-2 bias (decode_phase2_layer_tensors,
                # qwen3_flex_attention.py:1010-1017); generated keys carry 0
                bias = torch.zeros(B, shape.n_heads, cap, dtype=torch.float32, device=dev)
                for b in range(B):
                    bias[b, :, :n[b]] = pf.phase2_bias[j, :, pf.cu_kept[b]:pf.cu_kept[b + 1]]
                lc.bias = bias
                lc.qscale = q_head[j].contiguous() if q_head is not None else None
            self.layers.append(lc)
        last = torch.tensor([pf.cu_kept[b + 1] - 1 for b in range(B)], dtype=torch.int64)
        self.next_pos = pf.kept_positions.index_select(0, h2d(last, dev)) + 1
        self.gate_layer = gate_layer
        self.ssmax = pf.kept_ratio is not None
        self.n_kept_f = h2d(torch.tensor([float(x) for x in pf.n_kept], dtype=torch.float32), dev)
        self.steps = 0
        # one key-range-split workspace for every attention launch of every step (stream-ordered),
        # sized for the longest cache this state can reach (the planned size grows with the keys)
        longest = max(max(lc.n) for lc in self.layers) + max_new_tokens
        self._ws, ptr, self._ws_bytes = _lib.fwd_workspace("tg_keybias_fwd_workspace_size", dev, 1, 1, longest,
                                                           shape.n_heads, shape.n_kv_heads, 1)
        self._ws_ptr = ptr if self._ws_bytes else None

    def _attend(self, lc: _LayerCache, q: torch.Tensor, out: torch.Tensor) -> None:
        """q (B, H, D) -> out (B, H, D): sequence b attends over its segment's n[b] rows."""
        s = self.shape
        stream = torch.cuda.current_stream(q.device).cuda_stream
        lse = torch.empty(self.B, s.n_heads, 1, dtype=torch.float32, device=q.device)
        scale = 1.0 / math.sqrt(s.head_dim)
        ws_ptr, ws_bytes = self._ws_ptr, self._ws_bytes
        for b in range(self.B):
            kb = lc.k[lc.seg[b]:]
            vb = lc.v[lc.seg[b]:]
            bias = lc.bias[b:b + 1] if lc.bias is not None else None
            _lib.call("tg_keybias_fwd", q[b].data_ptr(), kb.data_ptr(), vb.data_ptr(),
                      bias.data_ptr() if bias is not None else None, out[b].data_ptr(), lse[b].data_ptr(),
                      1, 1, lc.n[b], s.n_heads, s.n_kv_heads, s.head_dim,
                      0, s.n_heads * s.head_dim, s.head_dim, 0, kb.stride(0), kb.stride(1),
                      0, vb.stride(0), vb.stride(1), 0, s.n_heads * s.head_dim, s.head_dim,
                      bias.stride(0) if bias is not None else 0, bias.stride(1) if bias is not None else 0,
                      scale, 1, ws_ptr if ws_bytes else None, ws_bytes, stream)

    @torch.no_grad()
    def step(self, tokens: torch.Tensor) -> torch.Tensor:
        """Appends one token per sequence (tokens (B,) int64) and returns the next greedy tokens."""
        s, w = self.shape, self.wts
        B = self.B
        dev = tokens.device
        x = torch.nn.functional.embedding(tokens, w.embed)
        res = x.clone()
        normed = torch.empty_like(x)
        hid = torch.empty_like(x)
        qkv = torch.empty(B, s.qkv_dim, dtype=x.dtype, device=dev)
        kn = torch.empty(B, s.n_kv_heads, s.head_dim, dtype=x.dtype, device=dev)
        vn = torch.empty_like(kn)
        att = torch.empty(B, s.n_heads, s.head_dim, dtype=x.dtype, device=dev)
        r_dec = None
        if self.ssmax:   # the new token's own ratio: slot n_kept + 1 + step at position next_pos
            m = (self.n_kept_f + 1.0 + self.steps).clamp(min=2.0)
            p = (self.next_pos.to(torch.float32) + 1.0).clamp(min=2.0)
            r_dec = (torch.log(m) / torch.log(p)).clamp(max=1.0)
        for l, lc in enumerate(self.layers):
            lw = w.layers[l]
            if l == 0:
                rmsnorm(res, lw.ln1, s.rms_eps, out=normed)
            else:
                rmsnorm(hid, lw.ln1, s.rms_eps, residual=res, residual_out=res, out=normed)
            torch.matmul(normed, lw.w_qkv.t(), out=qkv)
            q = qk_norm_rope(qkv, self.next_pos, lw, s, w.inv_freq, kn, vn, lc.qscale,
                             r_dec if (r_dec is not None and l > self.gate_layer) else None)
            rows = torch.tensor([lc.seg[b] + lc.n[b] for b in range(B)], dtype=torch.int64)
            rows = h2d(rows, dev)
            lc.k.index_copy_(0, rows, kn)
            lc.v.index_copy_(0, rows, vn)
            for b in range(B):
                lc.n[b] += 1
            qc = q.contiguous()
            self._attend(lc, qc, att)
            torch.matmul(att.view(B, -1), lw.w_o.t(), out=hid)
            rmsnorm(hid, lw.ln2, s.rms_eps, residual=res, residual_out=res, out=normed)
            act = silu_mul(torch.matmul(normed, lw.w_gu.t()))
            torch.matmul(act, lw.w_down.t(), out=hid)
        h = hid + res
        self.next_pos = self.next_pos + 1
        self.steps += 1
        logits = logits_last(w, h, torch.arange(B, device=dev))
        self.last_logits = logits
        return logits.argmax(-1)
