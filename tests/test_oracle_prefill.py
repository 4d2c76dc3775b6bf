"""Pins oracle/prefill.py (CPU, no GPU).

* One decoder layer against transformers' own Qwen3DecoderLayer (the module the reference runs,
  modeling_qwen3.py) on the same float32 weights with eager attention: causal, with a per-head
  per-key additive bias passed as the attention mask, and with a uniform temperature (q scaled,
  bias scaled — folded into q_norm's weight on the transformers side).
* The reference's padded Phase-2 batch (-1e9 pad slots) equals running each sample alone, and a
  right-padded Phase 1 equals the unpadded one, so the packed (cu_seqlens) layout of the product
  computes the same function.
* The keep lists and kept bias follow oracle.gate on the oracle's own scores.
* The finalized gate's scoring branch against transformers' Qwen3MLP with the (1, I) absorbed
  down_proj that load_gate rebuilds (e2e_gate_module.py:497-514), fed Qwen3RMSNorm of the
  gate layer's attention boundary; the boundary against the transformers layer with its MLP
  output zeroed; and the split (MLP on kept rows only) against the whole layer's kept rows.
"""
import math
from dataclasses import dataclass
from typing import List

import numpy as np
import pytest
import torch

from oracle import gate as og
from oracle import prefill as op

transformers = pytest.importorskip("transformers")
from transformers import Qwen3Config  # noqa: E402
from transformers.models.qwen3 import modeling_qwen3 as mq  # noqa: E402


@dataclass(frozen=True)
class Shape:
    n_layers: int = 3
    d_model: int = 256
    n_heads: int = 4
    n_kv_heads: int = 2
    head_dim: int = 128
    d_ff: int = 384
    vocab: int = 97
    rms_eps: float = 1e-6
    rope_theta: float = 1e6


@dataclass
class LW:
    ln1: torch.Tensor
    w_qkv: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    w_o: torch.Tensor
    ln2: torch.Tensor
    w_gu: torch.Tensor
    w_down: torch.Tensor


@dataclass
class Wts:
    shape: Shape
    embed: torch.Tensor
    layers: List[LW]
    final_norm: torch.Tensor
    lm_head: torch.Tensor
    inv_freq: torch.Tensor


def _wts(shape: Shape, seed=0):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g) * 0.05
    nw = lambda n: 1 + 0.2 * (torch.rand(n, generator=g) - 0.5)
    d, D = shape.d_model, shape.head_dim
    qkv = (shape.n_heads + 2 * shape.n_kv_heads) * D
    layers = [LW(nw(d), r(qkv, d), nw(D), nw(D), r(d, shape.n_heads * D), nw(d), r(2 * shape.d_ff, d),
                 r(d, shape.d_ff)) for _ in range(shape.n_layers)]
    inv = 1.0 / (shape.rope_theta ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    emb = r(shape.vocab, d) * 10
    return Wts(shape, emb, layers, nw(d), emb, inv)


def _hf_layer(shape: Shape, lw: LW, q_norm_mult=1.0):
    cfg = Qwen3Config(hidden_size=shape.d_model, intermediate_size=shape.d_ff, num_attention_heads=shape.n_heads,
                      num_key_value_heads=shape.n_kv_heads, head_dim=shape.head_dim, rms_norm_eps=shape.rms_eps,
                      rope_theta=shape.rope_theta, num_hidden_layers=1, vocab_size=shape.vocab,
                      max_position_embeddings=1 << 17)
    cfg._attn_implementation = "eager"
    L = mq.Qwen3DecoderLayer(cfg, 0).float().eval()
    H, Hkv, D, f = shape.n_heads, shape.n_kv_heads, shape.head_dim, shape.d_ff
    q, k, v = torch.split(lw.w_qkv, [H * D, Hkv * D, Hkv * D])
    gt, up = torch.split(lw.w_gu, [f, f])
    with torch.no_grad():
        L.input_layernorm.weight.copy_(lw.ln1)
        L.post_attention_layernorm.weight.copy_(lw.ln2)
        L.self_attn.q_proj.weight.copy_(q)
        L.self_attn.k_proj.weight.copy_(k)
        L.self_attn.v_proj.weight.copy_(v)
        L.self_attn.o_proj.weight.copy_(lw.w_o)
        L.self_attn.q_norm.weight.copy_(lw.q_norm * q_norm_mult)
        L.self_attn.k_norm.weight.copy_(lw.k_norm)
        L.mlp.gate_proj.weight.copy_(gt)
        L.mlp.up_proj.weight.copy_(up)
        L.mlp.down_proj.weight.copy_(lw.w_down)
    return cfg, L


def _hf_run(shape, lw, x, pos, mask, q_norm_mult=1.0):
    cfg, L = _hf_layer(shape, lw, q_norm_mult)
    rot = mq.Qwen3RotaryEmbedding(cfg)
    cos, sin = rot(x, pos)
    with torch.no_grad():
        out = L(x, attention_mask=mask, position_ids=pos, position_embeddings=(cos, sin))
    return out[0] if isinstance(out, tuple) else out


def _causal_mask(B, n, H=1):
    m = torch.triu(torch.full((n, n), float("-inf")), diagonal=1)
    return m[None, None].expand(B, H, n, n).clone()


def _rel(a, b):
    return float((a - b).norm() / b.norm())


@pytest.mark.parametrize("n,offset", [(37, 0), (160, 40000)])
def test_layer_matches_transformers_causal(n, offset):
    s = Shape()
    W = op.Weights(_wts(s))
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, n, s.d_model, generator=g)
    pos = (torch.arange(n) + offset)[None].expand(2, n).contiguous()
    ours, _, _ = op.layer(W, 0, x, pos)
    ref = _hf_run(s, _wts(s).layers[0], x, pos, _causal_mask(2, n))
    assert _rel(ours, ref) < 1e-5, _rel(ours, ref)


def test_layer_matches_transformers_bias_and_temperature():
    s = Shape()
    W = op.Weights(_wts(s))
    g = torch.Generator().manual_seed(2)
    B, n = 2, 96
    x = torch.randn(B, n, s.d_model, generator=g)
    pos = torch.sort(torch.randperm(5000, generator=g)[:n]).values[None].expand(B, n).contiguous()
    bias = torch.randn(B, s.n_heads, n, generator=g) * 2          # per-head per-key logit bias
    ours, _, _ = op.layer(W, 1, x, pos, bias_logit=bias)
    mask = _causal_mask(B, n, s.n_heads) + bias[:, :, None, :]
    ref = _hf_run(s, _wts(s).layers[1], x, pos, mask)
    assert _rel(ours, ref) < 1e-5
    # uniform temperature a: q * a and bias * a; transformers side: q_norm weight * a, mask bias * a
    a = 1.7
    ours_t, _, _ = op.layer(W, 1, x, pos, bias_logit=bias, q_temp=torch.full((s.n_heads,), a))
    ref_t = _hf_run(s, _wts(s).layers[1], x, pos, _causal_mask(B, n, s.n_heads) + a * bias[:, :, None, :],
                    q_norm_mult=a)
    assert _rel(ours_t, ref_t) < 1e-5
    assert _rel(ours_t, ours) > 1e-3          # the temperature does change the result
    # sampled query rows (each over every key it sees) against the same rows of the full layer
    rows = torch.tensor([0, 1, 17, 50, 94, 95])
    ours_r, k_r, _ = op.layer(W, 1, x, pos, bias_logit=bias, rows=rows)
    assert ours_r.shape == (B, len(rows), s.d_model)
    assert _rel(ours_r, ref[:, rows]) < 1e-5
    qs = 0.5 + torch.rand(B, s.n_heads, n, generator=g)
    full_q, k_f, _ = op.layer(W, 1, x, pos, bias_logit=bias, q_scale=qs)
    rows_q, _, _ = op.layer(W, 1, x, pos, bias_logit=bias, q_scale=qs, rows=rows)
    assert _rel(rows_q, full_q[:, rows]) < 1e-6 and torch.equal(k_r, k_f)


@dataclass
class Head:
    w1: torch.Tensor
    b1: torch.Tensor
    w2: torch.Tensor
    b2: float
    gate_scale: torch.Tensor
    attn_scale: torch.Tensor


def _head(s: Shape, seed=3):
    g = torch.Generator().manual_seed(seed)
    return Head(torch.randn(256, s.d_model, generator=g) * 0.05, torch.zeros(256), torch.randn(256, generator=g) * 0.1,
                0.0, torch.randn(s.n_layers - 2, s.n_heads, generator=g) * 0.3,
                torch.randn(s.n_layers - 2, s.n_heads, generator=g) * 0.3 + math.log(math.expm1(1.0)))


@dataclass
class BHead:
    w_gu: torch.Tensor
    w_row: torch.Tensor
    gate_scale: torch.Tensor
    attn_scale: torch.Tensor
    scaled_softmax: bool = True
    bias_gain: float = 1.0
    split_gate_layer = True


def _bhead(s: Shape, n_above: int, seed=3):
    g = torch.Generator().manual_seed(seed)
    return BHead(torch.randn(2 * s.d_ff, s.d_model, generator=g) * 0.05, torch.randn(s.d_ff, generator=g) * 0.1,
                 torch.randn(n_above, s.n_heads, generator=g) * 0.3,
                 torch.randn(n_above, s.n_heads, generator=g) * 0.3 + math.log(math.expm1(1.0)))


def test_branch_scores_boundary_and_split_match_transformers():
    from types import SimpleNamespace
    s = Shape()
    wts = _wts(s, seed=30)
    W = op.Weights(wts)
    head = _bhead(s, 1, seed=31)
    g = torch.Generator().manual_seed(32)
    B, n = 2, 50
    x = torch.randn(B, n, s.d_model, generator=g)
    pos = torch.arange(n)[None].expand(B, n).contiguous()
    bnd = []
    full, _, _ = op.layer(W, 1, x, pos, boundary=bnd)
    a = bnd[0]
    # boundary == the transformers layer with its MLP output zeroed (down_proj = 0)
    lw = wts.layers[1]
    zero_mlp = LW(lw.ln1, lw.w_qkv, lw.q_norm, lw.k_norm, lw.w_o, lw.ln2, lw.w_gu, torch.zeros_like(lw.w_down))
    ref_a = _hf_run(s, zero_mlp, x, pos, _causal_mask(B, n))
    assert _rel(a, ref_a) < 1e-5
    # the branch: a stock Qwen3MLP whose down_proj is the (1, I) absorbed row, fed Qwen3RMSNorm(a)
    mlp = mq.Qwen3MLP(SimpleNamespace(hidden_size=s.d_model, intermediate_size=s.d_ff, hidden_act="silu"))
    mlp.down_proj = torch.nn.Linear(s.d_ff, 1, bias=False)
    norm = mq.Qwen3RMSNorm(s.d_model, eps=s.rms_eps)
    with torch.no_grad():
        mlp.gate_proj.weight.copy_(head.w_gu[:s.d_ff])
        mlp.up_proj.weight.copy_(head.w_gu[s.d_ff:])
        mlp.down_proj.weight.copy_(head.w_row[None])
        norm.weight.copy_(lw.ln2)
        ref_sc = mlp(norm(ref_a))[..., 0]
    ours_sc = op.branch_scores_f32(head, a.reshape(-1, s.d_model), lw.ln2, s.rms_eps).view(B, n)
    assert _rel(ours_sc, ref_sc) < 1e-5
    assert float(ours_sc.std()) > 1e-3
    # split: the MLP half on a subset of rows == the whole layer's output on those rows
    keep = torch.tensor([0, 3, 4, 17, 49])
    assert _rel(op.mlp_half(W, 1, a[:, keep]), full[:, keep]) < 1e-6
    assert _rel(full, _hf_run(s, lw, x, pos, _causal_mask(B, n))) < 1e-5


def _prompts(lens, vocab, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, vocab, (n,), generator=g).tolist() for n in lens]


@pytest.mark.parametrize("branch", [False, True])
def test_padded_batch_equals_per_sample(branch):
    s = Shape(n_layers=4)
    W = op.Weights(_wts(s, seed=4))
    head = _bhead(s, 2) if branch else _head(s)
    head.gate_scale = torch.randn(2, s.n_heads) * 0.3
    head.attn_scale = torch.randn(2, s.n_heads) * 0.3 + 0.5
    lens, starts, ends, Ks = [90, 140, 61], [5, 10, 3], [80, 120, 50], [7, 200, 1]
    ids = _prompts(lens, s.vocab, 5)
    full = op.prefill(W, head, ids, starts, ends, 1, Ks)
    for b in range(3):
        one = op.prefill(W, head, [ids[b]], [starts[b]], [ends[b]], 1, [Ks[b]])
        assert np.array_equal(one["keep"][0], full["keep"][b])
        n = len(one["keep"][0])
        assert _rel(full["h_last"][b, :n], one["h_last"][0, :n]) < 1e-5
        assert _rel(full["logits"][b], one["logits"][0]) < 1e-5
        # Phase 1 with right padding == Phase 1 alone
        assert _rel(full["h_gate"][b], one["h_gate"][0]) < 1e-5


def test_keep_lists_and_bias_follow_gate_oracle():
    s = Shape(n_layers=3)
    W = op.Weights(_wts(s, seed=6))
    head = _head(s, seed=7)
    head.gate_scale = torch.zeros(2, s.n_heads)
    head.attn_scale = torch.zeros(2, s.n_heads)
    lens, starts, ends, Ks = [70, 55], [4, 0], [60, 55], [10, 100]
    ids = _prompts(lens, s.vocab, 8)
    r = op.prefill(W, head, ids, starts, ends, 0, Ks)
    for b in range(2):
        sc = op.head_scores(head, r["h_gate"][b][starts[b]:ends[b]])
        kp = og.keep_indices(sc, Ks[b], starts[b], ends[b], lens[b])
        assert np.array_equal(kp, r["keep"][b])
        assert len(kp) == starts[b] + og.k_clamped(Ks[b], ends[b] - starts[b]) + lens[b] - ends[b]
        np.testing.assert_allclose(r["kept_bias"][b], og.gate_bias(sc, kp, starts[b], ends[b]))


def test_decode_oracle_first_row_equals_prefill_and_past_form():
    """decode_logits' first row is the prefill's first-token logits; with no pruning below the gate
    and K >= the span, its rows equal a plain causal pass over prompt ++ generated."""
    s = Shape(n_layers=3)
    W = op.Weights(_wts(s, seed=10))
    head = _head(s, seed=11)
    head.gate_scale = torch.randn(2, s.n_heads) * 0.3
    head.attn_scale = torch.randn(2, s.n_heads) * 0.3
    ids = _prompts([50], s.vocab, 12)[0]
    r = op.prefill(W, head, [ids], [5], [40], 0, [10])
    keep = r["keep"][0]
    gen = [7, 3, 9]
    for prune in (False, True):
        d = op.decode_logits(W, head, ids, 5, 40, 0, keep, gen, prune_below_gate=prune)
        assert _rel(d[0], r["logits"][0]) < 1e-5
    # K >= span and zero gate bias: the gated decode is the plain model on prompt ++ generated
    head.gate_scale = torch.full((2, s.n_heads), -30.0)
    head.attn_scale = None
    full = op.prefill(W, head, [ids], [5], [40], 0, [1000])
    keep = full["keep"][0]
    d = op.decode_logits(W, head, ids, 5, 40, 0, keep, gen)
    x = W.embed[torch.as_tensor(ids + gen)][None]
    pos = torch.arange(len(ids) + len(gen))[None]
    for i in range(s.n_layers):
        x, _, _ = op.layer(W, i, x, pos)
    ref = op.rms(x[0, len(ids) - 1:], W.final_norm, s.rms_eps) @ W.lm_head.t()
    assert _rel(d, ref) < 1e-5


def test_scaled_softmax_reduces_to_mean_temperature_without_pruning():
    """Scaled-softmax mode with nothing pruned: every kept slot sits at its own position, so
    r = 1 on every row and the mode equals a uniform temperature mean_h(gamma) on the bias with
    per-head gamma on the query."""
    s = Shape(n_layers=3)
    W = op.Weights(_wts(s, seed=20))
    head = _head(s, seed=21)
    head.gate_scale = torch.randn(2, s.n_heads) * 0.3
    head.attn_scale = torch.randn(2, s.n_heads) * 0.4
    ids = _prompts([64], s.vocab, 22)
    head.scaled_softmax = True
    a = op.prefill(W, head, ids, [4], [60], 0, [1000])          # K >= span: no pruning
    assert list(a["keep"][0]) == list(range(64))
    r = og.ssmax_ratio(np.arange(64))
    assert np.allclose(r, 1.0)
    # the same run by hand, in the reference's bf16 arithmetic: bias = bf16(bf16(b * gs) *
    # bf16(mean_h bf16(gamma_h))), query * bf16(gamma_h)
    bf = lambda t: t.to(torch.bfloat16).float()
    g = bf(torch.nn.functional.softplus(head.attn_scale))
    gs = torch.nn.functional.softplus(head.gate_scale)
    x = W.embed[torch.as_tensor(ids[0])][None]
    pos = torch.arange(64)[None]
    x, _, _ = op.layer(W, 0, x, pos)
    kb = torch.as_tensor(a["kept_bias"][0], dtype=torch.float32)
    for j, i in enumerate(range(1, 3)):
        bl = bf(bf(kb[None, None, :] * gs[j][None, :, None]) * bf(g[j].mean()))
        x, _, _ = op.layer(W, i, x, pos, bias_logit=bl, q_scale=g[j][None, :, None].expand(1, -1, 64))
    ref = op.rms(x[0, -1], W.final_norm, s.rms_eps) @ W.lm_head.t()
    assert _rel(a["logits"][0], ref) < 1e-5
    # and it differs from the per-head temperature mode
    head.scaled_softmax = False
    b = op.prefill(W, head, ids, [4], [60], 0, [1000])
    assert _rel(a["logits"][0], b["logits"][0]) > 1e-4
