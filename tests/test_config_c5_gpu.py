"""GPU parity of the gated prefill at the ragged long-prompt configuration: 8 prompts of
16k-128k tokens (713,238 in all), the 28-layer Qwen3-1.7B shape (d 2048, 16/8 heads, head_dim
128, FFN 6144, vocab 151936), gate at layer 1, K per prompt from {100, 500, 2000, 4000}, state
span = prompt minus a 64-token prefix and a 256-token suffix -- the workload of the TTFT bench's
"ragged8" line (prefill_batch_for_decode, gate_forward.py:1280-1580, over a ragged batch).

Checked, per prompt:
  * keep lists and kept positions bit-exact against the oracle's selection on the kernel's own
    scores; the packed hidden rows bit-exact against index_select; the kept rows' gate bias
    against the oracle (float32 rounding);
  * both Phase-1 layers (the ~240 ms varlen launches over all 713k rows), teacher-forced, on
    sampled rows (the first and last 64 and 64 random ones, each over every key it sees), against
    the oracle layer evaluated in float32 torch on the device (the same bound as the other layer
    tests: max-abs 2e-2 relative to max(1, |ref|), rel-L2 1e-2);
  * the first and the last Phase-2 layer, teacher-forced the same way with the oracle's bf16
    Phase-2 key bias and query multipliers (scaled softmax);
  * finite first-token logits whose argmax is the first token.
"""
import numpy as np
import pytest
import torch

from oracle import gate as og
from oracle import prefill as op
from tests.attn_util import assert_close_grad, checked_ratio, to_np

pytestmark = pytest.mark.gpu

LENS = [114517, 57946, 113394, 80391, 42386, 123699, 106754, 74151]
KS = [2000, 4000, 100, 4000, 100, 100, 4000, 500]


def _sample(n, gen, k=64):
    if n <= 3 * k:
        return torch.arange(n)
    mid = torch.randperm(n - 2 * k, generator=gen)[:k] + k
    return torch.sort(torch.cat([torch.arange(k), mid, torch.arange(n - k, n)])).values


def test_ragged8_28_layers(cuda):
    from tokengate_amd import decoder as dec
    from tokengate_amd import gate as G
    from tokengate_amd import prefill as P
    torch.set_num_threads(min(16, torch.get_num_threads()))
    shape = dec.QWEN3_1P7B
    wts = dec.random_decoder(shape, seed=0, device=cuda)
    head = G.random_head(shape.n_layers - 2, shape.n_heads, seed=5, device=cuda, scaled_softmax=True)
    g = torch.Generator(device=cuda).manual_seed(9)
    head.gate_scale = head.gate_scale + 0.5 * torch.randn(head.gate_scale.shape, generator=g, device=cuda)
    head.attn_scale = head.attn_scale + 0.3 * torch.randn(head.attn_scale.shape, generator=g, device=cuda)
    gen = torch.Generator().manual_seed(17)
    ids = [torch.randint(0, shape.vocab, (n,), generator=gen).to(cuda) for n in LENS]
    starts, ends = [64] * len(LENS), [n - 256 for n in LENS]
    print(f"[c5] prefill of {sum(LENS)} tokens, K {KS}", flush=True)
    r = P.prefill_batch(wts, head, ids, starts, ends, 1, KS, capture=True)
    torch.cuda.synchronize()
    cap = r.capture
    cu1, cu2 = r.cu_prompt, r.cu_kept
    assert cu1[-1] == sum(LENS)

    # selection, pack and gate bias
    scores = cap["scores"].cpu().numpy().astype(np.float64)
    keep = cap["keep"].cpu().numpy()
    kpos = r.kept_positions.cpu().numpy()
    kb = r.kept_bias.cpu().numpy()
    keeps = []
    for b, L in enumerate(LENS):
        sc = scores[cu1[b] + starts[b]:cu1[b] + ends[b]]
        want = og.keep_indices(sc, KS[b], starts[b], ends[b], L)
        assert np.array_equal(keep[cu2[b]:cu2[b + 1]], want), f"seq {b}: keep list differs"
        assert np.array_equal(kpos[cu2[b]:cu2[b + 1]], want)
        assert r.n_kept[b] == len(want) == 320 + og.k_clamped(KS[b], ends[b] - starts[b])
        idx = torch.as_tensor(cu1[b] + want, device=cuda)
        assert torch.equal(cap["hs_packed"][cu2[b]:cu2[b + 1]], cap["h1"].index_select(0, idx)), f"seq {b}: rows"
        np.testing.assert_allclose(kb[cu2[b]:cu2[b + 1]], og.gate_bias(sc, want, starts[b], ends[b]),
                                   rtol=2e-6, atol=1e-7)
        keeps.append(want)
    print(f"[c5] keep lists, packed rows and gate bias of {len(LENS)} prompts match ({cu2[-1]} kept)", flush=True)

    W = op.Weights(wts, device=cuda)
    rg = torch.Generator().manual_seed(3)
    ins1 = list(cap["phase1"]) + [cap["h1"]]
    for i in range(2):
        for b, L in enumerate(LENS):
            x = ins1[i][cu1[b]:cu1[b + 1]].float()[None]
            pos = torch.arange(L, device=cuda)[None]
            rows = _sample(L, rg)
            ref, _, _ = op.layer(W, i, x, pos, rows=rows)
            got = ins1[i + 1][cu1[b]:cu1[b + 1]][rows.to(cuda)]
            ma, rl = assert_close_grad(f"phase1 layer {i} seq {b}", to_np(got), to_np(ref[0]))
            print(f"[c5] phase1 layer {i} seq {b} (L {L}, {len(rows)} rows): max-abs {ma:.2e} rel-L2 {rl:.2e}",
                  flush=True)
            del x, ref

    ins2 = list(cap["phase2"]) + [cap["h2"]]
    tables = [op.phase2_tables(head, scores[cu1[b] + starts[b]:cu1[b] + ends[b]].astype(np.float32), keeps[b],
                               starts[b], ends[b],
                               ratio=checked_ratio(r.kept_ratio[cu2[b]:cu2[b + 1]] if r.kept_ratio is not None
                                                   else None, keeps[b]))
              for b in range(len(LENS))]
    for i in (2, shape.n_layers - 1):
        j = i - 2
        for b in range(len(LENS)):
            n = r.n_kept[b]
            x = ins2[j][cu2[b]:cu2[b + 1]].float()[None]
            pos = torch.as_tensor(keeps[b], device=cuda)[None]
            bias_ref, s_ref = tables[b][0][j].to(cuda), tables[b][1][j]
            rows = _sample(n, rg)
            ref, _, _ = op.layer(W, i, x, pos, bias_logit=bias_ref[None],
                                 q_scale=s_ref.to(cuda)[None] if s_ref is not None else None, rows=rows)
            got = ins2[j + 1][cu2[b]:cu2[b + 1]][rows.to(cuda)]
            ma, rl = assert_close_grad(f"phase2 layer {i} seq {b}", to_np(got), to_np(ref[0]))
            print(f"[c5] phase2 layer {i} seq {b} (n {n}, {len(rows)} rows): max-abs {ma:.2e} rel-L2 {rl:.2e}",
                  flush=True)

    logits = cap["logits"].float()
    assert bool(torch.isfinite(logits).all())
    assert torch.equal(r.first_tokens, logits.argmax(-1))
