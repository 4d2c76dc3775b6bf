"""Pins the gate-path oracle (CPU): brute-force ranking, torch.topk on tie-free inputs, invariants
of the keep list, the reference's two keep constructions, library forms of the scoring head and
closed-form points of the ssmax ratio."""
import itertools

import numpy as np
import pytest
import torch

from oracle import gate as og


def _brute_keep(scores, K):
    """Element i is kept iff fewer than K_c elements beat it (beat = larger score, or NaN over
    non-NaN, or equal score at a lower index) — a counting definition, independent of sorting."""
    s = np.asarray(scores, dtype=np.float64)
    n = len(s)
    kc = og.k_clamped(K, n)
    kept = []
    for i in range(n):
        beats = 0
        for j in range(n):
            if j == i:
                continue
            ni, nj = np.isnan(s[i]), np.isnan(s[j])
            if nj and not ni:
                beats += 1
            elif nj and ni:
                beats += j < i
            elif not nj and not ni:
                beats += (s[j] > s[i]) or (s[j] == s[i] and j < i)
        if beats < kc:
            kept.append(i)
    return np.array(kept, dtype=np.int64)


def test_select_topk_matches_brute_force_on_all_small_tie_patterns():
    vals = [-1.0, 0.0, 2.0]
    for n in range(1, 6):
        for combo in itertools.product(vals, repeat=n):
            for K in range(0, n + 2):
                assert np.array_equal(og.select_topk(np.array(combo), K), _brute_keep(combo, K)), (combo, K)


def test_nan_and_signed_zero():
    s = np.array([0.0, -0.0, np.nan, 1.0, -0.0, np.nan])
    for K in range(0, 8):
        assert np.array_equal(og.select_topk(s, K), _brute_keep(s, K)), K
    assert np.array_equal(og.select_topk(s, 1), [2])          # NaN ranks first
    assert np.array_equal(og.select_topk(s, 4), [0, 2, 3, 5])  # then 1.0, then the lowest-index zero


def test_select_topk_matches_torch_topk_without_ties():
    rng = np.random.default_rng(0)
    for n, K in [(100, 7), (1000, 500), (5000, 5000), (300, 1)]:
        s = (rng.permutation(n) * 0.25 - n / 8).astype(np.float32)   # distinct, exactly representable
        assert len(np.unique(s)) == n
        ref = torch.sort(torch.topk(torch.from_numpy(s), K).indices).values.numpy()
        assert np.array_equal(og.select_topk(s, K), ref)


def test_keep_list_invariants_and_reference_constructions():
    rng = np.random.default_rng(1)
    L, s, e = 500, 64, 400
    sc = rng.standard_normal(e - s)
    for K in [0, 1, 100, e - s, 10_000_000]:
        kp = og.keep_indices(sc, K, s, e, L)
        kc = og.k_clamped(K, e - s)
        assert len(kp) == s + kc + (L - e)
        assert np.all(np.diff(kp) > 0)
        assert np.array_equal(kp[:s], np.arange(s)) and np.array_equal(kp[s + kc:], np.arange(e, L))
        # gate_forward.py:77-81 builds the same list as sort(cat(...))
        topk = og.topk_order(sc)[:kc]
        alt = np.sort(np.concatenate([np.arange(s), s + topk, np.arange(e, L)]))
        assert np.array_equal(kp, alt)


def test_gate_bias_is_rms_normalised_on_article_rows_only():
    rng = np.random.default_rng(2)
    s, e, L = 10, 60, 80
    sc = rng.standard_normal(e - s)
    kp = og.keep_indices(sc, 20, s, e, L)
    b = og.gate_bias(sc, kp, s, e)
    rms = np.sqrt(np.mean(sc ** 2) + og.RMS_EPS)
    art = (kp >= s) & (kp < e)
    assert np.all(b[~art] == 0)
    np.testing.assert_allclose(b[art], sc[kp[art] - s] / rms, rtol=1e-12)
    # torch's RMSNorm over the sequence axis gives the same normalised scores
    t = torch.from_numpy(sc)[None, :]
    tn = t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + og.RMS_EPS)
    np.testing.assert_allclose(b[art], tn[0, kp[art] - s].numpy(), rtol=1e-12)


def test_score_mlp_matches_torch_linear_silu():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(50, 64, generator=g, dtype=torch.float64)
    l1 = torch.nn.Linear(64, 16).double()
    l2 = torch.nn.Linear(16, 1).double()
    ref = l2(torch.nn.functional.silu(l1(x)))[:, 0].detach().numpy()
    got = og.score_mlp(x.numpy(), l1.weight.detach().numpy(), l1.bias.detach().numpy(),
                       l2.weight.detach().numpy()[0], float(l2.bias))
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_select_and_pack_concatenates_sequences():
    rng = np.random.default_rng(4)
    seqs = [(0, 30, 5, 25, 4), (30, 10, 2, 9, 100), (40, 20, 0, 20, 3), (60, 7, 3, 3, 5)]
    scores = rng.standard_normal(67)
    keep, starts, kcs = og.select_and_pack(scores, seqs)
    assert kcs == [4, 7, 3, 0]
    for (r0, L, s, e, K), st in zip(seqs, starts):
        kp = og.keep_indices(scores[r0 + s:r0 + e], K, s, e, L)
        assert np.array_equal(keep[st:st + len(kp)], kp)


def test_ssmax_ratio_closed_form():
    r = og.ssmax_ratio([0, 1, 5, 99])
    # slots 1..4 -> m = max(1,2)=2, 2, 3, 4; positions +1 -> max(1,2)=2, 2, 6, 100
    np.testing.assert_allclose(r, [min(1, np.log(2) / np.log(2)), 1.0, np.log(3) / np.log(6), np.log(4) / np.log(100)])
