"""GPU parity of the reported pruned-prefill TTFT workload itself: one 32,768-token prompt, K=2000,
the 28-layer Qwen3-1.7B shape (d 2048, 16/8 heads, head_dim 128, FFN 6144, vocab 151936), the
synthetic scoring head Linear(2048->256)->SiLU->Linear(256->1) at layer 1, state span 64..32512 --
the decoder, head and prompt that bench.py's TTFT line "32k_K2000" times (the same seeds and the
same prompt draw), through prefill_batch_for_decode's steps (gate_forward.py:1280-1580).

Checked:
  * the timed call (no capture) and the checked call (capture=True keeps references to every
    layer's input; the launches are the same) give the same first token, kept positions and logits;
  * the keep list bit-exact against the oracle's selection on the kernel's own scores (ties to the
    lower position); the packed hidden rows bit-exact against index_select; the kept rows' gate
    bias against the oracle (float32 rounding);
  * both Phase-1 layers (full-context causal attention over 32k rows) and Phase-2 layers 2 and 27,
    teacher-forced on 192 sampled rows (the first and last 64 and 64 random ones, each over every key
    it sees) against the oracle layer evaluated in float32 torch on the device, at the layer bound
    of the other prefill tests (max-abs 2e-2 relative to max(1, |ref|), rel-L2 1e-2);
  * finite first-token logits whose argmax is the first token.
"""
import numpy as np
import pytest
import torch

from oracle import gate as og
from oracle import prefill as op
from tests.attn_util import assert_close_grad, checked_ratio, to_np

pytestmark = pytest.mark.gpu

S, K, START, END = 32768, 2000, 64, 32768 - 256


def _sample(n, gen, k=64):
    if n <= 3 * k:
        return torch.arange(n)
    mid = torch.randperm(n - 2 * k, generator=gen)[:k] + k
    return torch.sort(torch.cat([torch.arange(k), mid, torch.arange(n - k, n)])).values


def test_ttft_32k_k2000_28_layers(cuda):
    from tokengate_amd import decoder as dec
    from tokengate_amd import gate as G
    from tokengate_amd import prefill as P
    torch.set_num_threads(min(16, torch.get_num_threads()))
    shape = dec.QWEN3_1P7B
    # the benchmark's decoder, head and prompt generator: its 32k lines draw the K=100 prompt
    # first, then the K=2000 one
    wts = dec.random_decoder(shape, seed=0, device=cuda)
    head = G.random_head(shape.n_layers - 2, shape.n_heads, seed=5, device=cuda)
    g = torch.Generator().manual_seed(7)
    torch.randint(0, shape.vocab, (S,), generator=g)
    ids = [torch.randint(0, shape.vocab, (S,), generator=g).to(cuda)]
    print(f"[ttft32k] prefill of {S} tokens, K={K}", flush=True)
    timed = P.prefill_batch(wts, head, ids, [START], [END], 1, [K])
    r = P.prefill_batch(wts, head, ids, [START], [END], 1, [K], capture=True)
    torch.cuda.synchronize()
    assert torch.equal(timed.first_tokens, r.first_tokens)
    assert torch.equal(timed.kept_positions, r.kept_positions)
    assert torch.equal(timed.logits, r.logits)
    del timed
    cap = r.capture

    # selection, pack and gate bias
    scores = cap["scores"].cpu().numpy().astype(np.float64)
    sc = scores[START:END]
    want = og.keep_indices(sc, K, START, END, S)
    assert r.n_kept == [len(want)] == [START + K + (S - END)]
    assert np.array_equal(cap["keep"].cpu().numpy(), want), "keep list differs from the oracle"
    assert np.array_equal(r.kept_positions.cpu().numpy(), want)
    assert torch.equal(cap["hs_packed"], cap["h1"].index_select(0, torch.as_tensor(want, device=cuda)))
    np.testing.assert_allclose(r.kept_bias.cpu().numpy(), og.gate_bias(sc, want, START, END), rtol=2e-6, atol=1e-7)
    print(f"[ttft32k] keep list, packed rows and gate bias match ({len(want)} kept)", flush=True)

    W = op.Weights(wts, device=cuda)
    rg = torch.Generator().manual_seed(3)
    ins1 = list(cap["phase1"]) + [cap["h1"]]
    pos1 = torch.arange(S, device=cuda)[None]
    for i in range(2):
        rows = _sample(S, rg)
        ref, _, _ = op.layer(W, i, ins1[i].float()[None], pos1, rows=rows)
        got = ins1[i + 1][rows.to(cuda)]
        ma, rl = assert_close_grad(f"phase1 layer {i}", to_np(got), to_np(ref[0]))
        print(f"[ttft32k] phase1 layer {i} ({len(rows)} rows): max-abs {ma:.2e} rel-L2 {rl:.2e}", flush=True)
        del ref

    ins2 = list(cap["phase2"]) + [cap["h2"]]
    bias_tab, s_tab = op.phase2_tables(head, sc.astype(np.float32), want, START, END,
                                       ratio=checked_ratio(r.kept_ratio, want))[:2]
    pos2 = torch.as_tensor(want, device=cuda)[None]
    for i in (2, shape.n_layers - 1):
        j = i - 2
        rows = _sample(len(want), rg)
        ref, _, _ = op.layer(W, i, ins2[j].float()[None], pos2, bias_logit=bias_tab[j].to(cuda)[None],
                             q_scale=s_tab[j].to(cuda)[None] if s_tab[j] is not None else None, rows=rows)
        got = ins2[j + 1][rows.to(cuda)]
        ma, rl = assert_close_grad(f"phase2 layer {i}", to_np(got), to_np(ref[0]))
        print(f"[ttft32k] phase2 layer {i} ({len(rows)} rows): max-abs {ma:.2e} rel-L2 {rl:.2e}", flush=True)

    logits = cap["logits"].float()
    assert bool(torch.isfinite(logits).all())
    assert torch.equal(r.first_tokens, logits.argmax(-1))
