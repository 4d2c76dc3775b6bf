"""Qwen3-shaped decoder stack for the gated prefill, on this package's gfx950 kernels.

The reference runs Qwen3 through transformers' eager modules patched with its attention backends
(qwen3_flex_attention.py:475-659): per layer RMSNorm -> q/k/v projections -> per-head q/k RMSNorm
-> RoPE -> causal (Phase 1) or gate-biased (Phase 2) attention -> o_proj -> residual ->
RMSNorm -> SwiGLU MLP -> residual.  Here a layer is five library GEMMs (fused QKV, O, fused
gate/up, down; hipBLASLt through torch) and four launches of this package's kernels:
tg_rmsnorm (residual add fused), tg_qk_norm_rope (q in place, k/v straight into the layer's KV
cache rows), tg_keybias_varlen_fwd (every sequence of the batch in one launch, cu_seqlens
layout, no padding), tg_silu_mul.  Tokens of all sequences are packed back to back, so Phase 1
runs the ragged batch without the reference's right padding.

Weights are bf16, generated from a seed (no checkpoint): the model is Qwen3-1.7B-shaped
(28 layers, d 2048, 16/8 heads, head_dim 128, FFN 6144, vocab 151936, RoPE theta 1e6, tied
embeddings), which is what the prefill measurements run.
"""
import math
from dataclasses import dataclass, field
from typing import List, Optional

import torch
import torch.nn.functional as F

from tokengate_amd import _lib


@dataclass(frozen=True)
class DecoderShape:
    n_layers: int = 28
    d_model: int = 2048
    n_heads: int = 16
    n_kv_heads: int = 8
    head_dim: int = 128
    d_ff: int = 6144
    vocab: int = 151936
    rms_eps: float = 1e-6
    rope_theta: float = 1e6
    tie_embeddings: bool = True

    @property
    def qkv_dim(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim


QWEN3_1P7B = DecoderShape()


@dataclass
class LayerWeights:
    ln1: torch.Tensor        # (d,) bf16 input_layernorm
    w_qkv: torch.Tensor      # (qkv_dim, d) bf16 = [q_proj; k_proj; v_proj]
    q_norm: torch.Tensor     # (head_dim,) bf16
    k_norm: torch.Tensor     # (head_dim,) bf16
    w_o: torch.Tensor        # (d, H*head_dim) bf16
    ln2: torch.Tensor        # (d,) bf16 post_attention_layernorm
    w_gu: torch.Tensor       # (2*d_ff, d) bf16 = [gate_proj; up_proj]
    w_down: torch.Tensor     # (d, d_ff) bf16


@dataclass
class DecoderWeights:
    shape: DecoderShape
    embed: torch.Tensor      # (vocab, d) bf16
    layers: List[LayerWeights]
    final_norm: torch.Tensor
    lm_head: torch.Tensor    # (vocab, d) bf16 (the embedding when tied)
    inv_freq: torch.Tensor = field(default=None)   # (head_dim/2,) fp32 on the device

    @property
    def device(self) -> torch.device:
        return self.embed.device


def rope_inv_freq(shape: DecoderShape, device) -> torch.Tensor:
    """1 / theta^(2i/D) in fp32, as Qwen3RotaryEmbedding's default initialisation computes it."""
    exps = torch.arange(0, shape.head_dim, 2, dtype=torch.float32) / shape.head_dim
    return (1.0 / (shape.rope_theta ** exps)).to(device)


def random_decoder(shape: DecoderShape = QWEN3_1P7B, seed: int = 0, device="cuda", std: float = 0.02,
                   norm_jitter: float = 0.0) -> DecoderWeights:
    """Seeded random initialisation: linear / embedding weights N(0, std) (the transformers
    initializer_range default), norm weights 1 (+ optional uniform jitter, so tests can see a
    norm weight that is not 1)."""
    g = torch.Generator(device=device).manual_seed(seed)
    bf = torch.bfloat16

    def lin(o, i):
        return (torch.randn(o, i, generator=g, device=device) * std).to(bf)

    def norm(n):
        w = torch.ones(n, device=device)
        if norm_jitter:
            w += (torch.rand(n, generator=g, device=device) - 0.5) * 2 * norm_jitter
        return w.to(bf)

    d, D = shape.d_model, shape.head_dim
    layers = [LayerWeights(norm(d), lin(shape.qkv_dim, d), norm(D), norm(D), lin(d, shape.n_heads * D), norm(d),
                           lin(2 * shape.d_ff, d), lin(d, shape.d_ff)) for _ in range(shape.n_layers)]
    embed = lin(shape.vocab, d)
    lm_head = embed if shape.tie_embeddings else lin(shape.vocab, d)
    return DecoderWeights(shape, embed, layers, norm(d), lm_head, rope_inv_freq(shape, device))


# ---- fused per-token ops -----------------------------------------------------------------------

def h2d(t: torch.Tensor, device) -> torch.Tensor:
    """Asynchronous host -> device copy of a small host tensor (through pinned memory)."""
    if torch.device(device).type != "cuda":
        return t
    return t.pin_memory().to(device, non_blocking=True)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, residual: Optional[torch.Tensor] = None,
            residual_out: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out = RMSNorm(x + residual) (residual_out <- x + residual when given); rows of x are the
    leading axis, last axis contiguous."""
    out = torch.empty_like(x) if out is None else out
    n, d = x.shape
    _lib.call("tg_rmsnorm", x.data_ptr(), x.stride(0),
              residual.data_ptr() if residual is not None else None,
              residual.stride(0) if residual is not None else 0,
              residual_out.data_ptr() if residual_out is not None else None,
              residual_out.stride(0) if residual_out is not None else 0,
              w.data_ptr(), out.data_ptr(), out.stride(0), n, d, float(eps), _stream(x))
    return out


def qk_norm_rope(qkv: torch.Tensor, positions: torch.Tensor, lw: LayerWeights, shape: DecoderShape,
                 inv_freq: torch.Tensor, k_out: torch.Tensor, v_out: torch.Tensor,
                 q_head_scale: Optional[torch.Tensor] = None,
                 q_row_scale: Optional[torch.Tensor] = None,
                 kv_rows: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Normalises and rotates q in place inside qkv (returned as a (T, H, D) view) and writes the
    rotated k and the v rows into k_out / v_out ((rows, Hkv, D) contiguous rows) at row t, or at
    row kv_rows[t] (int32) when given.  With q_head_scale (H,) and / or q_row_scale (T,) fp32 the
    bf16 query is multiplied by bf16(q_head_scale[h] * q_row_scale[t]) and rounded to bf16 again
    (the reference's bf16 q * s_eff)."""
    T = qkv.shape[0]
    H, Hkv, D = shape.n_heads, shape.n_kv_heads, shape.head_dim
    if positions.dtype != torch.int64 or positions.numel() != T:
        raise RuntimeError("qk_norm_rope: positions must be int64 with one entry per token")
    if q_row_scale is not None and (q_row_scale.dtype != torch.float32 or q_row_scale.numel() < T):
        raise RuntimeError("qk_norm_rope: q_row_scale must be fp32 with one entry per token")
    if kv_rows is not None and (kv_rows.dtype != torch.int32 or kv_rows.numel() < T or not kv_rows.is_contiguous()):
        raise RuntimeError("qk_norm_rope: kv_rows must be contiguous int32 with one entry per token")
    _lib.call("tg_qk_norm_rope", qkv.data_ptr(), qkv.stride(0), positions.data_ptr(), T, H, Hkv, D,
              lw.q_norm.data_ptr(), lw.k_norm.data_ptr(), float(shape.rms_eps), inv_freq.data_ptr(),
              q_head_scale.data_ptr() if q_head_scale is not None else None,
              q_row_scale.data_ptr() if q_row_scale is not None else None,
              qkv.data_ptr(), qkv.stride(0), k_out.data_ptr(), k_out.stride(0), v_out.data_ptr(), v_out.stride(0),
              kv_rows.data_ptr() if kv_rows is not None else None, _stream(qkv))
    return qkv[:, :H * D].view(T, H, D) if qkv.is_contiguous() else qkv[:, :H * D].unflatten(1, (H, D))


def silu_mul(gu: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    n, two_i = gu.shape
    inter = two_i // 2
    out = torch.empty(n, inter, dtype=gu.dtype, device=gu.device) if out is None else out
    _lib.call("tg_silu_mul", gu.data_ptr(), gu.stride(0), n, inter, out.data_ptr(), out.stride(0), _stream(gu))
    return out


def varlen_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens: torch.Tensor, max_seqlen: int,
                     scale: float, bias_raw: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                     lse: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal attention of every packed sequence in one launch (tg_keybias_varlen_fwd);
    bias_raw (nseq, H, >= max_seqlen) fp32 in raw-score units (logit bias / scale) or None."""
    T, H, D = q.shape
    Hkv = k.shape[1]
    out = torch.empty(T, H, D, dtype=q.dtype, device=q.device) if out is None else out
    lse = torch.empty(H, T, dtype=torch.float32, device=q.device) if lse is None else lse
    nseq = cu_seqlens.numel() - 1
    if bias_raw is not None and (bias_raw.dtype != torch.float32 or bias_raw.stride(-1) != 1):
        raise RuntimeError("varlen_attention: bias must be fp32 with a contiguous key axis")
    ws, ws_ptr, ws_bytes = _lib.fwd_workspace("tg_keybias_varlen_fwd_workspace_size", q.device, nseq, int(max_seqlen),
                                              H, Hkv, 1)
    _lib.call("tg_keybias_varlen_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(),
              bias_raw.data_ptr() if bias_raw is not None else None, out.data_ptr(), lse.data_ptr(),
              cu_seqlens.data_ptr(), nseq, int(max_seqlen), T, H, Hkv, D,
              q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
              out.stride(0), out.stride(1),
              bias_raw.stride(0) if bias_raw is not None else 0, bias_raw.stride(1) if bias_raw is not None else 0,
              float(scale), 1, ws_ptr, ws_bytes, _stream(q))
    return out


def varlen_kv_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_q: torch.Tensor, kv_cu: torch.Tensor,
                        kv_used: torch.Tensor, max_q: int, max_k: int, scale: float,
                        bias_raw: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                        lse: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal attention of every packed query segment over its own key segment of a cache
    (tg_keybias_varlen_kv_fwd): queries cu_q[b] .. cu_q[b+1]-1 over cache rows kv_cu[b] ..
    kv_cu[b] + kv_used[b] - 1, bottom-right aligned; bias_raw (nseq, H, >= max_k) fp32 with
    column j the sequence's key j."""
    T, H, D = q.shape
    Hkv = k.shape[1]
    out = torch.empty(T, H, D, dtype=q.dtype, device=q.device) if out is None else out
    lse = torch.empty(H, T, dtype=torch.float32, device=q.device) if lse is None else lse
    nseq = cu_q.numel() - 1
    for t in (cu_q, kv_cu, kv_used):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise RuntimeError("varlen_kv_attention: cu_q, kv_cu and kv_used must be contiguous int32")
    if kv_cu.numel() < nseq or kv_used.numel() < nseq:
        raise RuntimeError("varlen_kv_attention: kv_cu / kv_used need an entry per sequence")
    if bias_raw is not None and (bias_raw.dtype != torch.float32 or bias_raw.stride(-1) != 1
                                 or bias_raw.shape[-1] < max_k):
        raise RuntimeError("varlen_kv_attention: bias must be fp32 with a contiguous key axis of >= max_k")
    ws, ws_ptr, ws_bytes = _lib.fwd_workspace("tg_keybias_varlen_kv_fwd_workspace_size", q.device, nseq,
                                              int(max_q), int(max_k), H, Hkv, 1)
    _lib.call("tg_keybias_varlen_kv_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(),
              bias_raw.data_ptr() if bias_raw is not None else None, out.data_ptr(), lse.data_ptr(),
              cu_q.data_ptr(), kv_cu.data_ptr(), kv_used.data_ptr(), nseq, int(max_q), int(max_k), T, H, Hkv, D,
              q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
              out.stride(0), out.stride(1),
              bias_raw.stride(0) if bias_raw is not None else 0, bias_raw.stride(1) if bias_raw is not None else 0,
              float(scale), 1, ws_ptr, ws_bytes, _stream(q))
    return out


# ---- layer runner ------------------------------------------------------------------------------

@dataclass
class CacheGap:
    """KV-cache layout with `gap` free rows after each sequence (room for generated tokens): the
    cache rows of sequence b start at seg[b] = cu[b] + b * gap."""
    gap: int
    seg: List[int]                 # (nseq + 1,) host: segment starts, seg[nseq] = cu[nseq] + nseq * gap
    seg_dev: torch.Tensor          # int32 (nseq + 1,)
    used_dev: torch.Tensor         # int32 (nseq,) rows written per sequence
    rows_dev: torch.Tensor         # int32 (T,) cache row of every packed row
    pad: int = 0                   # rows after the last sequence (mapped past every segment)

    @property
    def rows(self) -> int:
        """Cache rows the layout needs."""
        return self.seg[-1] + self.pad

    @staticmethod
    def build(cu: List[int], gap: int, device, pad_rows: int = 0) -> "CacheGap":
        """pad_rows rows after the last sequence (a bucketed graph's padding) map past every segment."""
        n = len(cu) - 1
        seg = [cu[b] + b * gap for b in range(n + 1)]
        lens = [cu[b + 1] - cu[b] for b in range(n)]
        off = torch.tensor([b * gap for b in range(n)] + [n * gap], dtype=torch.int32)
        reps = torch.tensor(lens + [pad_rows], dtype=torch.int64)
        T = cu[-1] + pad_rows
        rows_h = torch.arange(T, dtype=torch.int32) + torch.repeat_interleave(off, reps, output_size=T)
        packed = torch.cat([torch.tensor(seg, dtype=torch.int32), torch.tensor(lens, dtype=torch.int32), rows_h])
        d = h2d(packed, device)
        return CacheGap(gap, seg, d[:n + 1], d[n + 1:2 * n + 1], d[2 * n + 1:], pad_rows)


@dataclass
class Ragged:
    """Token geometry of a packed batch: rows of sequence b are cu[b] .. cu[b+1]-1.  With `cache`
    the layer's KV rows go to a cache with free rows after each sequence (CacheGap) and attention
    reads its keys there."""
    cu: List[int]
    cu_dev: torch.Tensor       # int32 (nseq + 1,) on the device
    positions: torch.Tensor    # int64 (T,) RoPE position of every row
    max_len: int
    cache: Optional[CacheGap] = None

    @property
    def total(self) -> int:
        return self.cu[-1]

    @property
    def kv_rows(self) -> int:
        """Rows a layer's KV cache needs for this geometry."""
        return self.cache.rows if self.cache is not None else self.total

    @staticmethod
    def from_lengths(lengths: List[int], device) -> "Ragged":
        cu = [0]
        for n in lengths:
            cu.append(cu[-1] + int(n))
        cu_h = torch.tensor(cu, dtype=torch.int64)
        cu_dev = h2d(cu_h.to(torch.int32), device)
        # position of every row = row - first row of its sequence, built on the device
        T = cu[-1]
        lens_d = h2d(torch.tensor([int(n) for n in lengths], dtype=torch.int64), device)
        starts_d = h2d(cu_h[:-1].clone(), device)
        pos = torch.arange(T, dtype=torch.int64, device=device) - torch.repeat_interleave(starts_d, lens_d,
                                                                                           output_size=T)
        return Ragged(cu, cu_dev, pos, max(lengths, default=0))


@dataclass
class LayerKV:
    k: torch.Tensor   # (rows, Hkv, D) bf16: the layer's cache, rows in the ragged layout
    v: torch.Tensor


class Workspace:
    """Activation buffers reused across the layers of one phase (sized for `rows` tokens; the
    MLP intermediates for `mlp_rows`)."""

    def __init__(self, shape: DecoderShape, rows: int, device, mlp_rows: Optional[int] = None):
        bf = torch.bfloat16
        self.rows = rows
        self.mlp_rows = min(rows, mlp_rows or rows)
        d = shape.d_model
        self.residual = torch.empty(rows, d, dtype=bf, device=device)
        self.normed = torch.empty(rows, d, dtype=bf, device=device)
        self.hidden = torch.empty(rows, d, dtype=bf, device=device)
        self.qkv = torch.empty(rows, shape.qkv_dim, dtype=bf, device=device)
        self.attn = torch.empty(rows, shape.n_heads, shape.head_dim, dtype=bf, device=device)
        self.lse = torch.empty(shape.n_heads * rows, dtype=torch.float32, device=device)
        self.gu = torch.empty(self.mlp_rows, 2 * shape.d_ff, dtype=bf, device=device)
        self.act = torch.empty(self.mlp_rows, shape.d_ff, dtype=bf, device=device)


def run_layers(wts: DecoderWeights, layer_ids, x: torch.Tensor, geo: Ragged, ws: Workspace,
               kv: List[Optional[LayerKV]], biases=None, q_scales=None, capture: Optional[list] = None,
               q_row_scale: Optional[torch.Tensor] = None, attn_only_last: bool = False) -> torch.Tensor:
    """Runs decoder layers `layer_ids` over the packed rows x (T, d) and returns the hidden state
    after the last of them (T, d).  kv[i] receives layer i's cache rows.  biases[i] / q_scales[i]
    (optional): Phase-2 raw-unit key bias (nseq, H, >= max_len) and per-head query scale (H,)
    fp32 of layer i; q_row_scale (T,) fp32: a per-row query scale for every layer (the
    scaled-softmax ratio).  capture: optional list that receives each layer's input hidden state.
    attn_only_last: the last layer stops at its attention residual a = x + o_proj(attn) (the
    split gate layer's boundary, attn_only_forward of gate_forward.py:372-413); its MLP half is
    mlp_sublayer."""
    shape = wts.shape
    T = geo.total
    if x.shape != (T, shape.d_model):
        raise RuntimeError("run_layers: x must be (total_rows, d_model)")
    eps = shape.rms_eps
    scale = 1.0 / math.sqrt(shape.head_dim)
    res, normed, hid = ws.residual[:T], ws.normed[:T], ws.hidden[:T]
    qkv, attn, lse = ws.qkv[:T], ws.attn[:T], ws.lse[:shape.n_heads * T].view(shape.n_heads, T)
    first = True
    layer_ids = list(layer_ids)
    for n_done, i in enumerate(layer_ids):
        lw = wts.layers[i]
        if first:
            res.copy_(x)
            rmsnorm(res, lw.ln1, eps, out=normed)
            first = False
        else:
            rmsnorm(hid, lw.ln1, eps, residual=res, residual_out=res, out=normed)
        if capture is not None:
            capture.append(res.clone())
        torch.matmul(normed, lw.w_qkv.t(), out=qkv)
        cg = geo.cache
        q = qk_norm_rope(qkv, geo.positions, lw, shape, wts.inv_freq, kv[i].k, kv[i].v,
                         q_scales[i] if q_scales is not None else None, q_row_scale,
                         kv_rows=cg.rows_dev if cg is not None else None)
        if cg is None:
            varlen_attention(q, kv[i].k, kv[i].v, geo.cu_dev, geo.max_len, scale,
                             biases[i] if biases is not None else None, out=attn, lse=lse)
        else:
            varlen_kv_attention(q, kv[i].k, kv[i].v, geo.cu_dev, cg.seg_dev, cg.used_dev, geo.max_len,
                                geo.max_len, scale, biases[i] if biases is not None else None, out=attn, lse=lse)
        torch.matmul(attn.view(T, -1), lw.w_o.t(), out=hid)
        if attn_only_last and n_done == len(layer_ids) - 1:
            break
        rmsnorm(hid, lw.ln2, eps, residual=res, residual_out=res, out=normed)
        _mlp_rows(lw, normed, hid, ws)
    out = torch.empty_like(hid)
    torch.add(hid, res, out=out)
    return out


def _mlp_rows(lw: LayerWeights, normed: torch.Tensor, out: torch.Tensor, ws: Workspace) -> None:
    """out = down(silu(gate) * up) of the normed rows, in chunks of ws.mlp_rows."""
    T = normed.shape[0]
    for r0 in range(0, T, ws.mlp_rows):
        r1 = min(T, r0 + ws.mlp_rows)
        gu = ws.gu[:r1 - r0]
        torch.matmul(normed[r0:r1], lw.w_gu.t(), out=gu)
        act = silu_mul(gu, out=ws.act[:r1 - r0])
        torch.matmul(act, lw.w_down.t(), out=out[r0:r1])


def mlp_sublayer(wts: DecoderWeights, i: int, a: torch.Tensor, ws: Workspace) -> torch.Tensor:
    """Layer i's MLP half on rows a (T, d): a + down(silu(gate) * up)(post_attention_layernorm(a))
    (_gate_layer_mlp_eager, gate_forward.py:422-437).  Position-wise, so running it on a subset of
    rows equals running it on all rows and keeping that subset."""
    T = a.shape[0]
    if T > ws.rows:
        raise RuntimeError("mlp_sublayer: workspace has fewer rows than the input")
    lw = wts.layers[i]
    normed, hid = ws.normed[:T], ws.hidden[:T]
    rmsnorm(a, lw.ln2, wts.shape.rms_eps, out=normed)
    _mlp_rows(lw, normed, hid, ws)
    out = torch.empty_like(a)
    torch.add(a, hid, out=out)
    return out


def alloc_kv(shape: DecoderShape, rows: int, device) -> LayerKV:
    return LayerKV(torch.empty(rows, shape.n_kv_heads, shape.head_dim, dtype=torch.bfloat16, device=device),
                   torch.empty(rows, shape.n_kv_heads, shape.head_dim, dtype=torch.bfloat16, device=device))


def lm_head(normed: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """F.linear(normed, weight).float() on bf16 tensors: tg_lm_head (HBM-bound GEMV) for up to 8
    rows, torch's GEMM for larger batches."""
    n, d = normed.shape
    if n > 8 or d % 512 != 0 or normed.stride(1) != 1 or weight.stride(1) != 1 or weight.stride(0) != d:
        return F.linear(normed, weight).float()
    V = weight.shape[0]
    out = torch.empty(n, V, dtype=torch.float32, device=normed.device)
    _lib.call("tg_lm_head", normed.data_ptr(), normed.stride(0), n, weight.data_ptr(), V, d, out.data_ptr(),
              out.stride(0), _stream(normed))
    return out


def linear_rows(x: torch.Tensor, weight: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """F.linear(x, weight) on bf16 tensors for the rows of a decode step: tg_linear_rows (a GEMV
    that streams the weight once) for up to 8 rows, torch's GEMM otherwise."""
    n, d = x.shape
    if n > 8 or d % 512 != 0 or x.stride(1) != 1 or weight.stride(1) != 1 or weight.stride(0) != d \
            or (out is not None and out.stride(1) != 1):
        return torch.matmul(x, weight.t(), out=out)
    N = weight.shape[0]
    out = torch.empty(n, N, dtype=torch.bfloat16, device=x.device) if out is None else out
    _lib.call("tg_linear_rows", x.data_ptr(), x.stride(0), n, weight.data_ptr(), N, d, out.data_ptr(), out.stride(0),
              _stream(x))
    return out


def _rows_ok(*ts) -> bool:
    return all(t is None or (t.stride(-1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0) for t in ts)


def linear_rows_norm(h: torch.Tensor, norm_w: torch.Tensor, eps: float, weight: torch.Tensor,
                     residual: Optional[torch.Tensor] = None, residual_out: Optional[torch.Tensor] = None,
                     out: Optional[torch.Tensor] = None, out_fp32: bool = False) -> torch.Tensor:
    """F.linear(RMSNorm(h + residual), weight) for up to 8 rows in one launch (tg_linear_rows_norm);
    residual_out <- bf16(h + residual) when given (a buffer other than residual)."""
    n, d = h.shape
    N = weight.shape[0]
    if not (1 <= n <= 8 and d % 512 == 0 and _rows_ok(h, residual, residual_out) and weight.stride(1) == 1
            and weight.stride(0) == d):
        raise RuntimeError("linear_rows_norm: 1..8 contiguous 16-byte aligned rows, dim a multiple of 512")
    if out is None:
        out = torch.empty(n, N, dtype=torch.float32 if out_fp32 else torch.bfloat16, device=h.device)
    _lib.call("tg_linear_rows_norm", h.data_ptr(), h.stride(0),
              residual.data_ptr() if residual is not None else None, residual.stride(0) if residual is not None else 0,
              residual_out.data_ptr() if residual_out is not None else None,
              residual_out.stride(0) if residual_out is not None else 0,
              norm_w.data_ptr(), float(eps), n, weight.data_ptr(), N, d, out.data_ptr(), out.stride(0),
              int(out_fp32), _stream(h))
    return out


def linear_rows_swiglu(gate_up: torch.Tensor, weight: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """F.linear(silu(g) * u, weight) of gate/up rows [g | u] for up to 8 rows in one launch."""
    n, two_i = gate_up.shape
    inter = two_i // 2
    N = weight.shape[0]
    if not (1 <= n <= 8 and inter % 512 == 0 and _rows_ok(gate_up) and weight.stride(1) == 1
            and weight.stride(0) == inter):
        raise RuntimeError("linear_rows_swiglu: 1..8 contiguous 16-byte aligned rows, inter a multiple of 512")
    out = torch.empty(n, N, dtype=torch.bfloat16, device=gate_up.device) if out is None else out
    _lib.call("tg_linear_rows_swiglu", gate_up.data_ptr(), gate_up.stride(0), n, inter, weight.data_ptr(), N,
              out.data_ptr(), out.stride(0), _stream(gate_up))
    return out


def argmax_rows(logits: torch.Tensor) -> torch.Tensor:
    """logits.argmax(-1) (int64) of fp32 rows with torch's rules (NaN wins, ties to the lower
    index) in one launch that clears no memory (tg_argmax_rows)."""
    n, V = logits.shape
    if logits.dtype != torch.float32 or logits.stride(1) != 1 or logits.stride(0) % 4 != 0 \
            or logits.data_ptr() % 16 != 0:
        raise RuntimeError("argmax_rows: fp32 rows, contiguous, 16-byte aligned, row stride a multiple of 4")
    out = torch.empty(n, dtype=torch.int64, device=logits.device)
    _lib.call("tg_argmax_rows", logits.data_ptr(), logits.stride(0), n, V, out.data_ptr(), _stream(logits))
    return out


def logits_last(wts: DecoderWeights, h: torch.Tensor, last_rows: torch.Tensor) -> torch.Tensor:
    """Final norm + LM head on the given rows only (the rows that produce the next token)."""
    rows = h.index_select(0, last_rows)
    normed = rmsnorm(rows, wts.final_norm, wts.shape.rms_eps)
    return lm_head(normed, wts.lm_head)
