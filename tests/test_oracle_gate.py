"""Pins the gate-path oracle (CPU): brute-force ranking, torch.topk on tie-free inputs, invariants
of the keep list, the reference's two keep constructions, library forms of the scoring head and
of the bias normalisation (transformers' Qwen3RMSNorm), closed-form points of the ssmax ratio, and
the bias / Phase-2 rounding chain against vectors written by the reference's own functions
(tests/golden/gate_chain.npz)."""
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


def _qwen3_seq_rms(raw_np, L2=3, H=4, gain=1.0):
    """transformers' Qwen3RMSNorm(1, eps=1e-6) over the sequence axis of the (n_art, L2, H)
    broadcast of the scores, as E2EGate._seq_rms_norm_qwen applies it (e2e_gate_module.py:342-344)."""
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm
    norm = Qwen3RMSNorm(1, eps=og.RMS_EPS)
    with torch.no_grad():
        norm.weight.fill_(gain)
        raw = torch.from_numpy(np.asarray(raw_np, np.float32))[:, None]
        b = raw.view(-1, 1, 1).expand(-1, L2, H)
        return norm(b.movedim(-3, -1)).movedim(-1, -3).numpy()


@pytest.mark.parametrize("n,gain,ties", [(1, 1.0, False), (7, 1.0, False), (4096, 1.0, False),
                                         (3001, 0.75, True), (500, 1.0, True)])
def test_seq_rms_norm_matches_transformers_qwen3_rmsnorm(n, gain, ties):
    rng = np.random.default_rng(n)
    raw = rng.standard_normal(n).astype(np.float32) * 3
    if ties:
        raw = np.round(raw * 4) / 4
    raw = og.bf16(raw)
    ref = _qwen3_seq_rms(raw, gain=gain)
    got = og.seq_rms_norm(raw, gain=gain)
    for l in range(ref.shape[1]):
        for h in range(ref.shape[2]):
            # fp32 throughout; the two fp32 means may differ in their last bit (summation order)
            np.testing.assert_allclose(got, ref[:, l, h], rtol=4e-7, atol=0)
    # the eps sits inside the square root, added to the mean square (not to the rms)
    tiny = np.full(8, 1e-4, np.float32)
    np.testing.assert_allclose(og.seq_rms_norm(tiny), _qwen3_seq_rms(tiny)[:, 0, 0], rtol=4e-7)
    np.testing.assert_allclose(og.seq_rms_norm(tiny), 1e-4 / np.sqrt(1e-8 + 1e-6), rtol=1e-6)


def test_gate_bias_is_rms_normalised_on_article_rows_only():
    rng = np.random.default_rng(2)
    s, e, L = 10, 60, 80
    sc = og.bf16(rng.standard_normal(e - s))
    kp = og.keep_indices(sc, 20, s, e, L)
    b = og.gate_bias(sc, kp, s, e)
    art = (kp >= s) & (kp < e)
    assert np.all(b[~art] == 0)
    np.testing.assert_allclose(b[art], _qwen3_seq_rms(sc)[kp[art] - s, 0, 0], rtol=4e-7)


def _golden():
    import os
    return np.load(os.path.join(os.path.dirname(__file__), "golden", "gate_chain.npz"))


def _bf16_ulp_diff(a, b):
    """Distance in bf16 units in the last place between bf16-valued arrays."""
    def key(x):
        u = np.asarray(x, np.float32).view(np.int32).astype(np.int64) >> 16
        return np.where(u < 0, -(u & 0x7FFF), u)
    return np.abs(key(a) - key(b))


@pytest.mark.parametrize("case", [0, 1])
def test_gate_chain_matches_reference_vectors(case):
    """The fp32 bias, the selection key, the bf16 stored bias and both Phase-2 transforms against
    vectors written by the reference's own E2EGate.forward / aggregate /
    build_gate_bias_vectorized / _ssmax_ratio / Qwen3FlexAttention._phase2_q_bias."""
    z = _golden()
    p = f"c{case}_"
    L, s, e, K, L2, H, D = (int(x) for x in z[p + "geom"])
    raw, gs, at = z[p + "raw"], z[p + "gate_scale"], z[p + "attn_scale"]
    b = og.gate_bias_layers(raw, gs)
    np.testing.assert_allclose(b, z[p + "b"], rtol=5e-7, atol=0)
    np.testing.assert_allclose(og.aggregate(b), z[p + "agg"], rtol=1e-6, atol=1e-7)
    keep = z[p + "keep"]
    assert np.array_equal(og.keep_indices(raw, K, s, e, L), keep)     # same kept set by the raw score
    gb = og.kept_bias_layers(b, keep, s, e)
    assert np.array_equal(gb, z[p + "gb"])
    r = og.ssmax_ratio(keep).astype(np.float32)
    np.testing.assert_allclose(r, z[p + "ratio"], rtol=2e-7, atol=0)
    q = z[p + "q"][0]                                                  # (H, n, D) bf16 values
    temp = og.softplus32(at)
    for l in range(L2):
        s_ss = og.phase2_query_scale(temp[l], z[p + "ratio"])
        assert np.array_equal(og.phase2_query(q, s_ss), z[p + "q_ssmax"][l, 0])
        assert np.array_equal(og.phase2_bias(gb[:, l, :], temp[l], z[p + "ratio"]), z[p + "bias_ssmax"][l, 0])
        s_ph = og.phase2_query_scale(temp[l])
        assert np.array_equal(og.phase2_query(q, s_ph), z[p + "q_perhead"][l, 0])
        assert np.array_equal(og.phase2_bias(gb[:, l, :], temp[l]), z[p + "bias_perhead"][l, 0])


def test_gate_chain_rounding_points_are_not_interchangeable():
    """Mistakes the golden vectors must catch: the products in fp32 with one rounding at the end,
    and the bias stored in fp32, each change the reference's Phase-2 values."""
    z = _golden()
    p = "c0_"
    raw, gs, at = z[p + "raw"], z[p + "gate_scale"], z[p + "attn_scale"]
    L, s, e = (int(x) for x in z[p + "geom"][:3])
    keep = z[p + "keep"]
    temp = og.softplus32(at)
    b = og.gate_bias_layers(raw, gs)
    gb32 = np.zeros((len(keep),) + b.shape[1:], np.float32)
    art = (keep >= s) & (keep < e)
    gb32[art] = b[keep[art] - s]
    r = z[p + "ratio"]
    one_rounding = og.bf16(gb32[:, 0, :] * (temp[0][:, None] * r[None, :]).mean(0)[:, None])
    assert not np.array_equal(one_rounding, z[p + "bias_ssmax"][0, 0])
    assert not np.array_equal(og.phase2_bias(gb32[:, 0, :], temp[0], r), z[p + "bias_ssmax"][0, 0])
    q = z[p + "q"][0]
    fused = og.bf16(q * (temp[0][:, None] * r[None, :])[:, :, None])
    assert not np.array_equal(fused, z[p + "q_ssmax"][0, 0])


@pytest.mark.parametrize("seed", range(4))
def test_raw_score_ranking_equals_reference_selection_key(seed):
    """Top-K by the raw bf16 score equals top-K by the reference's selection key (aggregate of
    E2EGate.forward), ties at lower positions first in both: for bf16-valued scores the fp32
    chain raw -> agg is strictly increasing (distinct bf16 values are 2^-8 apart relative, each
    fp32 step moves a value by at most 2^-24 relative), and equal scores map to equal keys."""
    rng = np.random.default_rng(100 + seed)
    n = 5000
    raw = og.bf16(rng.standard_normal(n).astype(np.float32) * (0.5 + seed))
    if seed % 2:
        raw = og.bf16(np.round(raw * 8) / 8)          # heavy ties
    gs = (np.log(np.expm1(1.5)) + 0.3 * rng.standard_normal((3, 16))).astype(np.float32)
    agg = og.aggregate(og.gate_bias_layers(raw, gs))
    ref_agg = torch.from_numpy(og.gate_bias_layers(raw, gs))[:, 0, :]
    ref_agg = (ref_agg * torch.full((16,), 1.0 / 16)).sum(-1).numpy()   # torch's own head sum
    for key in (agg, ref_agg):
        for K in (1, 100, 2000, n):
            assert np.array_equal(og.select_topk(raw, K), og.select_topk(key, K))
    # equal raw -> equal key; order preserved
    o = np.argsort(raw, kind="stable")
    assert np.all(np.diff(agg[o]) >= 0)
    assert np.array_equal(np.diff(raw[o]) == 0, np.diff(agg[o]) == 0)


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
