"""GPU parity of the gate path: keep lists and packed rows bit-exact against the oracle on the same
score tensor; the scoring head within tolerance of a float64 evaluation.

Covers the reference's selection semantics (gate_forward.py:1409-1421): K_c = max(1, min(K, n_art)),
K >= n_art keeps everything, prefix/suffix always kept, ascending order; ties (bf16-rounded scores
make them common) go to the lower position; NaN and signed zeros; ragged batches; articles longer
than the LDS-resident limit; and the 32k scoring + pruning workload (hidden [1, 32768, 2048], state
span 64..32511, K in {100, 500, 2000}, two layers of K/V [8 heads, 128]).
"""
import math

import numpy as np
import pytest
import torch

from oracle import gate as og
from tests.attn_util import assert_close, to_np

pytestmark = pytest.mark.gpu


def _run_select(scores_np, seqs, dev):
    from tokengate_amd import gate
    scores = torch.tensor(scores_np, dtype=torch.float32, device=dev)
    p = gate.plan([s[0] for s in seqs], [s[1] for s in seqs], [s[2] for s in seqs], [s[3] for s in seqs],
                  [s[4] for s in seqs], dev)
    keep, sumsq = gate.select_keep(scores, p)
    torch.cuda.synchronize()
    return keep.cpu().numpy(), sumsq.cpu().numpy(), p


def _check_select_pack(scores_np, seqs, ref, p, dev):
    """The fused launch (gate.select_pack): keep lists bit-exact, positions, gate bias of the kept
    rows (float32 chain of the oracle), and a row stream gathered at the kept positions."""
    from tokengate_amd import gate
    scores = torch.tensor(scores_np, dtype=torch.float32, device=dev)
    rows = len(scores_np)
    src = torch.arange(rows * 8, dtype=torch.int32, device=dev).view(rows, 8)
    dst = torch.full((p.total_kept, 8), -1, dtype=torch.int32, device=dev)
    pos = torch.full((p.total_kept,), -7, dtype=torch.int64, device=dev)
    bias = torch.full((p.total_kept,), float("nan"), dtype=torch.float32, device=dev)
    keep = gate.select_pack(scores, p, [(src, dst)], positions=pos, bias_out=bias, check=True)
    torch.cuda.synchronize()
    k = keep.cpu().numpy()
    assert np.array_equal(k, ref), "select_pack keep list differs from the oracle"
    assert np.array_equal(pos.cpu().numpy(), ref)
    row_of = np.concatenate([seqs[b][0] + ref[p.cu_kept[b]:p.cu_kept[b + 1]] for b in range(len(seqs))]) \
        if p.total_kept else np.zeros(0, np.int64)
    assert np.array_equal(dst.cpu().numpy(), src.cpu().numpy()[row_of])
    bo = bias.cpu().numpy()
    for b, (r0, L, s_, e, K) in enumerate(seqs):
        art = scores_np[r0 + s_:r0 + e]
        if len(art) == 0 or not np.isfinite(art).all() or np.sum(art.astype(np.float64) ** 2) > 1e37:
            continue
        want = og.gate_bias(art, ref[p.cu_kept[b]:p.cu_kept[b + 1]], s_, e)
        np.testing.assert_allclose(bo[p.cu_kept[b]:p.cu_kept[b + 1]], want, rtol=2e-6, atol=1e-30)


def _check_select(scores_np, seqs, dev):
    keep, sumsq, p = _run_select(scores_np, seqs, dev)
    ref, starts, kcs = og.select_and_pack(scores_np.astype(np.float64), seqs)
    assert p.k_clamped == kcs and p.cu_kept[:-1] == starts
    assert keep.dtype == np.int64 and np.array_equal(keep, ref)
    _check_select_pack(scores_np, seqs, ref, p, dev)
    for b, (r0, L, s, e, K) in enumerate(seqs):
        art = scores_np[r0 + s:r0 + e].astype(np.float64)
        art = art[np.isfinite(art)] if not np.isfinite(scores_np).all() else art
        if len(art) and np.isfinite(scores_np[r0 + s:r0 + e]).all():
            want = np.sum(art * art)
            if want > np.finfo(np.float32).max:     # the float32 sum overflows, as the reference's does
                assert np.isinf(sumsq[b])
            else:
                # squares below float32's range flush to zero, as in the reference's float32 mean
                np.testing.assert_allclose(sumsq[b], want, rtol=1e-4, atol=1e-37)
    return keep, p


def test_random_ragged_batch(cuda):
    rng = np.random.default_rng(0)
    seqs, r0 = [], 0
    for L, s, e, K in [(5000, 64, 4744, 100), (300, 0, 300, 10_000_000), (1, 0, 1, 5), (2000, 10, 1990, 0),
                       (777, 700, 700, 9), (4096, 64, 3840, 2000), (64, 3, 60, 57)]:
        seqs.append((r0, L, s, e, K))
        r0 += L
    scores = rng.standard_normal(r0).astype(np.float32)
    _check_select(scores, seqs, cuda)
    # bf16-rounded scores: many exact ties at the threshold
    scores_bf = torch.from_numpy(scores).to(torch.bfloat16).float().numpy()
    _check_select(scores_bf, seqs, cuda)


@pytest.mark.parametrize("seed", range(12))
def test_random_selection_sweep(cuda, seed):
    """Seeded random batches: 1-8 sequences, lengths up to 70k (past the register-resident limit,
    so the streaming top-K runs too), random state spans (empty ones included) and K (0, 1,
    keep-all, around the article length), scores normal, bf16-rounded (many ties) or few-valued."""
    rng = np.random.default_rng(500 + seed)
    seqs, r0 = [], 0
    for _ in range(int(rng.integers(1, 9))):
        L = int(rng.integers(1, 70000)) if rng.random() < 0.2 else int(rng.integers(1, 9000))
        s = int(rng.integers(0, min(L, 300) + 1))
        e = int(rng.integers(s, L + 1))
        K = int(rng.choice([0, 1, 5, 100, 500, 2000, 10_000_000, int(rng.integers(0, e - s + 2))]))
        seqs.append((r0, L, s, e, K))
        r0 += L
    scores = rng.standard_normal(r0).astype(np.float32)
    kind = int(rng.integers(3))
    if kind == 1:
        scores = torch.from_numpy(scores).to(torch.bfloat16).float().numpy()
    elif kind == 2:
        scores = np.round(scores * 4).astype(np.float32)
    _check_select(scores, seqs, cuda)


@pytest.mark.parametrize("kind", ["all_equal", "few_values", "nan_and_zeros", "steps", "infinities", "huge_range",
                                  "two_clusters", "tiny_range", "denormals", "negative_only"])
def test_heavy_ties(cuda, kind):
    """Tie patterns plus the ranges that steer the value-space first pass: infinities and spans
    that overflow float (pass skipped), two far clusters (everything in the end bins), ranges of a
    few ulps and of denormals, negative-only scores."""
    rng = np.random.default_rng(1)
    n = 10_000
    if kind == "all_equal":
        s = np.full(n, 0.5, np.float32)
    elif kind == "few_values":
        s = rng.integers(0, 4, n).astype(np.float32)
    elif kind == "nan_and_zeros":
        s = rng.choice(np.array([0.0, -0.0, 1.0, -1.0, np.nan], np.float32), n)
    elif kind == "infinities":
        s = rng.standard_normal(n).astype(np.float32)
        s[rng.choice(n, 50, replace=False)] = np.inf
        s[rng.choice(n, 50, replace=False)] = -np.inf
    elif kind == "huge_range":
        s = (rng.standard_normal(n) * 10.0 ** rng.uniform(-38, 38, n)).astype(np.float32)
        s[:2] = [np.finfo(np.float32).max, -np.finfo(np.float32).max]
    elif kind == "two_clusters":
        s = np.where(rng.random(n) < 0.5, 1e6, -1e6).astype(np.float32) + rng.standard_normal(n).astype(np.float32)
    elif kind == "tiny_range":
        s = (np.float32(1.0) + rng.integers(0, 8, n).astype(np.float32) * np.finfo(np.float32).eps).astype(np.float32)
    elif kind == "denormals":
        s = (rng.integers(-50, 50, n) * np.float32(1e-44)).astype(np.float32)
    elif kind == "negative_only":
        s = (-np.abs(rng.standard_normal(n)) - 3.0).astype(np.float32)
    else:
        s = np.repeat(np.arange(100, dtype=np.float32), 100)[rng.permutation(n)]
    seqs = [(0, n, 7, n - 3, K) for K in (1,)]
    for K in (1, 2, 17, 1000, 4999, 9989, 9990, 20000):
        _check_select(s, [(0, n, 7, n - 3, K)], cuda)


def test_long_article_global_path(cuda):
    """Articles longer than the register-resident limit (65536 keys) take the streaming variant
    (32768-key chunks re-read on every pass)."""
    rng = np.random.default_rng(2)
    L = 100_000
    s = torch.from_numpy(rng.standard_normal(2 * L).astype(np.float32)).to(torch.bfloat16).float().numpy()
    seqs = [(0, L, 64, L - 256, 4000), (L, L, 0, L, 50_000)]
    _check_select(s, seqs, cuda)


def test_understated_max_article_len_falls_back_to_streaming(cuda):
    """The C ABI's max_article_len only picks the kernel: a caller that understates it still gets
    every keep list whole (sequences longer than the register capacity take the streaming path)."""
    from tokengate_amd import _lib, gate
    rng = np.random.default_rng(3)
    lens = [70_000, 3000, 40_000]
    seqs, r0 = [], 0
    for L, K in zip(lens, [5000, 100, 20_000]):
        seqs.append((r0, L, 64, L - 256, K))
        r0 += L
    sc = torch.from_numpy(rng.standard_normal(r0).astype(np.float32)).to(torch.bfloat16).float().numpy()
    scores = torch.from_numpy(sc).to(cuda)
    p = gate.plan([x[0] for x in seqs], [x[1] for x in seqs], [x[2] for x in seqs], [x[3] for x in seqs],
                  [x[4] for x in seqs], cuda)
    for hint in (1000, 32 * 1024, 64 * 1024):
        keep = torch.full((p.total_kept,), -1, dtype=torch.int64, device=cuda)
        sumsq = torch.empty(len(seqs), dtype=torch.float32, device=cuda)
        _lib.call("tg_gate_topk_keep", scores.data_ptr(), p.geom.data_ptr(), len(seqs), hint, keep.data_ptr(),
                  sumsq.data_ptr(), torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        got = keep.cpu().numpy()
        for b, (r, L, s_, e_, K) in enumerate(seqs):
            want = og.keep_indices(sc[r + s_:r + e_], K, s_, e_, L)
            assert np.array_equal(got[p.cu_kept[b]:p.cu_kept[b + 1]], want), f"hint {hint} seq {b}"
            np.testing.assert_allclose(float(sumsq[b]), float(np.sum(sc[r + s_:r + e_].astype(np.float64) ** 2)),
                                       rtol=1e-5)


@pytest.mark.parametrize("kind", ["few_values", "bf16_normal"])
def test_streaming_ties_across_chunks(cuda, kind):
    """Ties at the threshold spread over several 32768-key chunks (the compaction carries the tie
    and output counts from chunk to chunk); a ragged batch whose longest article forces the
    streaming variant on every sequence, short ones included."""
    rng = np.random.default_rng(4)
    lens = [200_003, 70_000, 5, 40_000]
    n = sum(lens)
    if kind == "few_values":
        s = rng.integers(0, 7, n).astype(np.float32)
    else:
        s = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(torch.bfloat16).float().numpy()
    seqs, r0 = [], 0
    for L, K in zip(lens, [60_000, 9_999, 2, 35_000]):
        seqs.append((r0, L, 1, L - 1 if L > 2 else L, K))
        r0 += L
    _check_select(s, seqs, cuda)


def test_single_sequence_helper(cuda):
    from tokengate_amd import gate
    rng = np.random.default_rng(3)
    art = rng.standard_normal(500).astype(np.float32)
    kp = gate.keep_indices(torch.from_numpy(art).to(cuda), 40, 12, 512, 600).cpu().numpy()
    assert np.array_equal(kp, og.keep_indices(art, 40, 12, 512, 600))


def test_pack_bit_exact_row_and_head_major(cuda):
    from tokengate_amd import gate
    rng = np.random.default_rng(4)
    g = torch.Generator(device=cuda).manual_seed(4)
    seqs, r0 = [], 0
    for L, s, e, K in [(1000, 16, 900, 50), (333, 0, 333, 333), (2048, 64, 1792, 700)]:
        seqs.append((r0, L, s, e, K))
        r0 += L
    total = r0
    scores = torch.from_numpy(rng.standard_normal(total).astype(np.float32)).to(cuda)
    p = gate.plan([x[0] for x in seqs], [x[1] for x in seqs], [x[2] for x in seqs], [x[3] for x in seqs],
                  [x[4] for x in seqs], cuda)
    keep, sumsq = gate.select_keep(scores, p)
    hidden = torch.randn(total, 2048, generator=g, device=cuda).to(torch.bfloat16)
    k_rows = torch.randn(total, 8, 128, generator=g, device=cuda).to(torch.bfloat16)
    v_head_major = torch.randn(8, total, 128, generator=g, device=cuda).to(torch.bfloat16)   # (Hkv, S, D)
    T = p.total_kept
    hs_out = torch.empty(T, 2048, dtype=torch.bfloat16, device=cuda)
    k_out = torch.empty(T, 8, 128, dtype=torch.bfloat16, device=cuda)
    v_out = torch.empty(T, 8, 128, dtype=torch.bfloat16, device=cuda)
    pos = torch.empty(T, dtype=torch.int64, device=cuda)
    bias = torch.empty(T, dtype=torch.float32, device=cuda)
    gate.pack(keep, p, [(hidden, hs_out), (k_rows, k_out), (v_head_major.transpose(0, 1), v_out)],
              positions=pos, bias_src=scores, sumsq=sumsq, bias_out=bias)
    torch.cuda.synchronize()
    src_rows = np.concatenate([x[0] + keep.cpu().numpy()[p.cu_kept[b]:p.cu_kept[b + 1]] for b, x in enumerate(seqs)])
    idx = torch.from_numpy(src_rows).to(cuda)
    assert torch.equal(hs_out, hidden.index_select(0, idx))
    assert torch.equal(k_out, k_rows.index_select(0, idx))
    assert torch.equal(v_out, v_head_major.index_select(1, idx).transpose(0, 1))
    assert torch.equal(pos.cpu(), keep.cpu())
    sc = scores.cpu().numpy().astype(np.float64)
    ref_bias = np.concatenate([og.gate_bias(sc[x[0] + x[2]:x[0] + x[3]], keep.cpu().numpy()[p.cu_kept[b]:p.cu_kept[b + 1]],
                                            x[2], x[3]) for b, x in enumerate(seqs)])
    assert_close("pack bias", to_np(bias), ref_bias, max_abs=1e-5, rel_l2=1e-6)
    # the fused launch: the same rows, head-major source included
    outs2 = [torch.empty_like(t) for t in (hs_out, k_out, v_out)]
    pos2 = torch.empty_like(pos)
    bias2 = torch.empty_like(bias)
    keep2 = gate.select_pack(scores, p, [(hidden, outs2[0]), (k_rows, outs2[1]),
                                         (v_head_major.transpose(0, 1), outs2[2])],
                             positions=pos2, bias_out=bias2, check=True)
    torch.cuda.synchronize()
    assert torch.equal(keep2, keep) and torch.equal(pos2, pos)
    for a_, b_ in zip(outs2, (hs_out, k_out, v_out)):
        assert torch.equal(a_, b_)
    np.testing.assert_allclose(bias2.cpu().numpy(), bias.cpu().numpy(), rtol=2e-6, atol=0)
    # destinations with free rows after each sequence (a KV cache with decode headroom): kept row j
    # of sequence b lands on row j + b * gap, the free rows keep their contents
    gap = 5
    nseq = len(seqs)
    for fused in (False, True):
        kg = torch.full((T + nseq * gap, 8, 128), 7.0, dtype=torch.bfloat16, device=cuda)
        vg = torch.full_like(kg, 7.0)
        hg = torch.empty_like(hs_out)
        pairs = [(hidden, hg), (k_rows, kg, gap), (v_head_major.transpose(0, 1), vg, gap)]
        if fused:
            gate.select_pack(scores, p, pairs, check=True)
        else:
            gate.pack(keep, p, pairs)
        torch.cuda.synchronize()
        assert torch.equal(hg, hs_out)
        for b in range(nseq):
            c0, c1 = p.cu_kept[b], p.cu_kept[b + 1]
            assert torch.equal(kg[c0 + b * gap:c1 + b * gap], k_out[c0:c1])
            assert torch.equal(vg[c0 + b * gap:c1 + b * gap], v_out[c0:c1])
            assert bool((kg[c1 + b * gap:c1 + (b + 1) * gap] == 7.0).all())
            assert bool((vg[c1 + b * gap:c1 + (b + 1) * gap] == 7.0).all())
    with pytest.raises(RuntimeError, match="fewer rows"):
        gate.pack(keep, p, [(k_rows, torch.empty(T + gap, 8, 128, dtype=torch.bfloat16, device=cuda), gap)])


def _xavier(shape, g, dev):
    fan_out, fan_in = shape
    a = math.sqrt(6.0 / (fan_in + fan_out))
    return (torch.rand(shape, generator=g, device=dev) * 2 - 1) * a


@pytest.mark.parametrize("K", [100, 500, 2000])
def test_config_scoring_and_pruning_32k(cuda, K):
    from tokengate_amd import gate
    S, d, s, e = 32768, 2048, 64, 32512
    g = torch.Generator(device=cuda).manual_seed(5)
    hidden = torch.randn(1, S, d, generator=g, device=cuda).to(torch.bfloat16)
    w1 = _xavier((256, d), g, cuda).to(torch.bfloat16)
    w2 = _xavier((1, 256), g, cuda)[0].contiguous()
    b1 = torch.zeros(256, device=cuda)
    x = hidden[0]
    scores = gate.score_mlp(x, w1, b1, w2, 0.0)
    torch.cuda.synchronize()
    ref = og.score_mlp(to_np(x[s:e]), to_np(w1), np.zeros(256), to_np(w2), 0.0)
    assert_close(f"scores K={K}", to_np(scores[s:e]), ref, max_abs=2e-3, rel_l2=1e-4)
    # selection and pack on the kernel's own score tensor, bit-exact
    p = gate.plan([0], [S], [s], [e], [K], cuda)
    keep, sumsq = gate.select_keep(scores, p)
    kv = [torch.randn(S, 8, 128, generator=g, device=cuda).to(torch.bfloat16) for _ in range(4)]   # K,V x 2 layers
    T = p.total_kept
    assert T == s + K + (S - e)
    outs = [torch.empty(T, 2048, dtype=torch.bfloat16, device=cuda)] + \
           [torch.empty(T, 8, 128, dtype=torch.bfloat16, device=cuda) for _ in kv]
    pos = torch.empty(T, dtype=torch.int64, device=cuda)
    bias = torch.empty(T, dtype=torch.float32, device=cuda)
    gate.pack(keep, p, list(zip([x] + kv, outs)), positions=pos, bias_src=scores, sumsq=sumsq, bias_out=bias)
    torch.cuda.synchronize()
    ref_keep = og.keep_indices(scores.cpu().numpy()[s:e], K, s, e, S)
    assert np.array_equal(keep.cpu().numpy(), ref_keep)
    idx = torch.from_numpy(ref_keep).to(cuda)
    for src, out in zip([x] + kv, outs):
        assert torch.equal(out, src.index_select(0, idx))
    assert np.array_equal(pos.cpu().numpy(), ref_keep)
    ref_bias = og.gate_bias(scores.cpu().numpy()[s:e].astype(np.float64), ref_keep, s, e)
    assert_close("bias", to_np(bias), ref_bias, max_abs=1e-5, rel_l2=1e-6)
    # the fused launch on the same workload
    outs2 = [torch.empty_like(t) for t in outs]
    pos2, bias2 = torch.empty_like(pos), torch.empty_like(bias)
    keep2 = gate.select_pack(scores, p, list(zip([x] + kv, outs2)), positions=pos2, bias_out=bias2, check=True)
    torch.cuda.synchronize()
    assert np.array_equal(keep2.cpu().numpy(), ref_keep) and torch.equal(pos2, pos)
    for a_, b_ in zip(outs2, outs):
        assert torch.equal(a_, b_)
    assert_close("fused bias", to_np(bias2), ref_bias, max_abs=1e-5, rel_l2=1e-6)


def test_scoring_wide_workgroups(cuda):
    """The scoring head's 256-row workgroup form (taken when the grid still gives every CU two of
    them): a ragged row count that covers chips of up to 304 CUs, checked on sampled rows (every
    97th, the first and last 300) against the float64 oracle, and row for row equal to the same
    rows scored in small launches, which take the 128-row form."""
    from tokengate_amd import gate
    n = 256 * 2 * 304 + 77
    g = torch.Generator(device=cuda).manual_seed(11)
    x = torch.randn(n, 2048, generator=g, device=cuda).to(torch.bfloat16)
    w1 = _xavier((256, 2048), g, cuda).to(torch.bfloat16)
    w2 = _xavier((1, 256), g, cuda)[0].contiguous()
    b1 = torch.randn(256, generator=g, device=cuda) * 0.1
    scores = gate.score_mlp(x, w1, b1, w2, 0.25)
    small = torch.cat([gate.score_mlp(x[r:r + 8192], w1, b1, w2, 0.25) for r in (0, n - 8192)])
    torch.cuda.synchronize()
    assert torch.equal(scores[:8192], small[:8192]) and torch.equal(scores[n - 8192:], small[8192:])
    rows = np.unique(np.concatenate([np.arange(0, n, 97), np.arange(300), np.arange(n - 300, n)]))
    idx = torch.from_numpy(rows).to(cuda)
    ref = og.score_mlp(to_np(x.index_select(0, idx)), to_np(w1), to_np(b1), to_np(w2), 0.25)
    assert_close("wide scores", to_np(scores.index_select(0, idx)), ref, max_abs=2e-3, rel_l2=1e-4)


@pytest.mark.parametrize("n", [32448, 256 * 2 * 304 + 77, 1000, 129])
def test_scoring_ktiled_w1_bit_identical(cuda, n):
    """The k-step-major W1 (gate.ktile_w1, tg_gate_score_mlp_ktiled) changes only where the
    kernel's weight stream reads from: scores bit-identical to the row-major W1 in both workgroup
    forms (32k and 256 x 2 x 304 + 77 rows take the 128- and 256-row forms), ragged tails included,
    and ScoringHead.scores (which streams the tiled copy) equal to both."""
    from tokengate_amd import gate
    g = torch.Generator(device=cuda).manual_seed(17)
    x = torch.randn(n, 2048, generator=g, device=cuda).to(torch.bfloat16)
    w1 = _xavier((256, 2048), g, cuda).to(torch.bfloat16)
    w2 = _xavier((1, 256), g, cuda)[0].contiguous()
    b1 = torch.randn(256, generator=g, device=cuda) * 0.1
    w1k = gate.ktile_w1(w1)
    assert torch.equal(w1k[5, 17], w1[17, 160:192])
    rm = gate.score_mlp(x, w1, b1, w2, 0.25)
    kt = gate.score_mlp(x, w1, b1, w2, 0.25, w1_ktiled=w1k)
    head = gate.ScoringHead(w1, b1, w2, 0.25, torch.zeros(1, 16, device=cuda))
    hd = head.scores(x)
    torch.cuda.synchronize()
    assert torch.equal(rm, kt) and torch.equal(rm, hd)
    rows = torch.arange(0, n, 101, device=cuda)
    ref = og.score_mlp(to_np(x.index_select(0, rows)), to_np(w1), to_np(b1), to_np(w2), 0.25)
    assert_close("ktiled scores", to_np(kt.index_select(0, rows)), ref, max_abs=2e-3, rel_l2=1e-4)


def test_ragged8_select_pack(cuda):
    """The ragged pruned-prefill batch at full size: 8 prompts of 16k-128k tokens (prefix 64,
    suffix 256), K from {100, 500, 2000, 4000}, bf16-valued scores (ties at every threshold), the
    hidden rows (2048 bf16) and two layers of K/V (8 x 128 bf16) gathered; keep lists, positions
    and rows bit-exact, bias against the oracle's float32 chain."""
    from tokengate_amd import gate
    rng = np.random.default_rng(8)
    lens = [int(x) for x in rng.integers(16384, 131073, size=8)]
    Ks = [int(x) for x in rng.choice([100, 500, 2000, 4000], size=8)]
    seqs, r0 = [], 0
    for L, K in zip(lens, Ks):
        seqs.append((r0, L, 64, L - 256, K))
        r0 += L
    print(f"[ragged8] lens={lens} K={Ks}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(8)
    scores = torch.randn(r0, generator=g, device=cuda).to(torch.bfloat16).float()
    hidden = torch.randn(r0, 2048, generator=g, device=cuda).to(torch.bfloat16)
    kv = [torch.randn(r0, 8, 128, generator=g, device=cuda).to(torch.bfloat16) for _ in range(4)]
    p = gate.plan([x[0] for x in seqs], lens, [x[2] for x in seqs], [x[3] for x in seqs], Ks, cuda)
    T = p.total_kept
    outs = [torch.empty(T, 2048, dtype=torch.bfloat16, device=cuda)] + \
           [torch.empty(T, 8, 128, dtype=torch.bfloat16, device=cuda) for _ in kv]
    pos = torch.empty(T, dtype=torch.int64, device=cuda)
    bias = torch.empty(T, dtype=torch.float32, device=cuda)
    keep = gate.select_pack(scores, p, list(zip([hidden] + kv, outs)), positions=pos, bias_out=bias, check=True)
    torch.cuda.synchronize()
    sc = scores.cpu().numpy()
    ref, starts, kcs = og.select_and_pack(sc, seqs)
    assert np.array_equal(keep.cpu().numpy(), ref) and np.array_equal(pos.cpu().numpy(), ref)
    rows = torch.from_numpy(np.concatenate([x[0] + ref[p.cu_kept[b]:p.cu_kept[b + 1]]
                                            for b, x in enumerate(seqs)])).to(cuda)
    for src, out in zip([hidden] + kv, outs):
        assert torch.equal(out, src.index_select(0, rows))
    ref_bias = np.concatenate([og.gate_bias(sc[x[0] + x[2]:x[0] + x[3]], ref[p.cu_kept[b]:p.cu_kept[b + 1]], x[2], x[3])
                               for b, x in enumerate(seqs)])
    np.testing.assert_allclose(bias.cpu().numpy(), ref_bias, rtol=2e-6, atol=0)


def test_select_pack_workspace_reuse_across_batch_sizes(cuda):
    """Stream-ordered select_pack calls of different batch sizes share one workspace: its counters
    sit at offsets fixed by the capacities, so a call after a smaller one starts from zeroed
    counters (the regression: a layout that moved with the batch size let a later call read the
    previous call's records as counters).  Every call bit-exact; the error flag stays clear."""
    rng = np.random.default_rng(12)
    for nseq in (3, 8, 1, 6, 2, 8):
        seqs, r0 = [], 0
        for _ in range(nseq):
            L = int(rng.integers(300, 20000))
            s = int(rng.integers(0, 200))
            e = int(rng.integers(s + 1, L + 1))
            seqs.append((r0, L, s, e, int(rng.choice([1, 100, 500, 2000, 10_000_000]))))
            r0 += L
        scores = rng.standard_normal(r0).astype(np.float32)
        p = _run_select(scores, seqs, cuda)[2]
        ref, _, _ = og.select_and_pack(scores.astype(np.float64), seqs)
        _check_select_pack(scores, seqs, ref, p, cuda)


@pytest.mark.parametrize("over", [-1, 0, 1, 97])
def test_select_pack_one_and_three_launch_forms(cuda, over):
    """tg_gate_select_pack runs the selection in one launch when its chunk workgroups (4096 keys
    each here) all fit the chip at once (at most one per CU) and in three launches above that:
    batches of CU count - 1, CU count, CU count + 1 and CU count + 97 chunks, sequences of 1-8
    chunks (ragged lengths inside the last chunk, a few empty spans), bf16-valued scores (ties at
    every threshold), K from 1 to beyond the span; keep lists, positions, rows bit-exact, bias
    against the oracle's float32 chain, the error word clear."""
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    target = cus + over
    rng = np.random.default_rng(40 + over)
    seqs, r0, n_chunks = [], 0, 0
    while n_chunks < target:
        g = int(min(rng.integers(1, 9), target - n_chunks))
        n_art = int(rng.integers((g - 1) * 4096 + 1, g * 4096 + 1))
        pre, suf = int(rng.integers(0, 70)), int(rng.integers(0, 300))
        L = pre + n_art + suf
        seqs.append((r0, L, pre, pre + n_art, int(rng.choice([1, 100, 500, 2000, n_art, n_art + 5]))))
        r0 += L
        n_chunks += g
        if rng.random() < 0.1:                       # an empty span: no chunk, prefix and suffix kept
            seqs.append((r0, 40, 20, 20, 100))
            r0 += 40
    print(f"[launch forms] cus={cus} chunks={n_chunks} seqs={len(seqs)} rows={r0}", flush=True)
    scores = og.bf16(rng.standard_normal(r0).astype(np.float32))
    keep, p = _check_select(scores, seqs, cuda)
    assert p.sel_kpt == 8 and p.sel_starts[-1] == target


def test_one_launch_selection_many_geometries(cuda):
    """60 random batches through the one-launch selection (chunk counts up to the CU count,
    sequences of 1-16 chunks, K from 0 to beyond the span including span - 1 and the span itself,
    normal, bf16-valued and few-valued scores): every keep list bit-exact through select_keep and
    select_pack, positions and gathered rows, the error word clear.  A chunk that saw its sequence's
    phase flag before the data the flag publishes had reached memory (a release whose L2
    write-back was not waited for) compacted at a stale offset about once in a hundred such batches,
    silently."""
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    for case in range(60):
        rng = np.random.default_rng(7000 + case)
        target = int(rng.choice([8, 40, cus // 2, cus - 1, cus]))
        seqs, r0, n_chunks = [], 0, 0
        while n_chunks < target:
            g = int(min(rng.integers(1, 17), target - n_chunks))
            n_art = int(rng.integers((g - 1) * 4096 + 1, g * 4096 + 1))
            pre, suf = int(rng.integers(0, 70)), int(rng.integers(0, 300))
            L = pre + n_art + suf
            K = int(rng.choice([0, 1, 7, 100, 500, 2000, n_art - 1, n_art, n_art + 5, int(rng.integers(1, n_art + 1))]))
            seqs.append((r0, L, pre, pre + n_art, K))
            r0 += L
            n_chunks += g
            if rng.random() < 0.1:
                seqs.append((r0, 40, 20, 20, 100))
                r0 += 40
        kind = int(rng.integers(3))
        scores = rng.standard_normal(r0).astype(np.float32)
        if kind == 1:
            scores = og.bf16(scores)
        elif kind == 2:
            scores = np.round(scores * 3).astype(np.float32)
        print(f"[one-launch geometries] case {case}: chunks={n_chunks} seqs={len(seqs)} rows={r0} kind={kind}",
              flush=True)
        _check_select(scores, seqs, cuda)


def test_four_keys_per_thread_both_launch_forms(cuda, monkeypatch):
    """4 keys per thread (chunks of 2048 scores) through both selection forms.  gate.plan gives 4 keys
    per thread only to batches of at most 64 chunks, so that limit is lifted here.  Batches of CU
    count - 1 chunks (one launch) and CU count + 40 chunks (three launches) are run, with spans of up
    to 16 chunks.  Every keep list must be bit-exact against the oracle, with positions, gathered
    rows and gate bias checked as well."""
    from tokengate_amd import gate
    monkeypatch.setattr(gate, "_SEL_SMALL_CHUNKS", 1 << 20)
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    for case, target in enumerate([cus - 1, cus + 40]):
        rng = np.random.default_rng(7500 + case)
        seqs, r0, n_chunks = [], 0, 0
        while n_chunks < target:
            g = int(min(rng.integers(1, 17), target - n_chunks))
            n_art = int(rng.integers((g - 1) * 2048 + 1, g * 2048 + 1))
            pre, suf = int(rng.integers(0, 70)), int(rng.integers(0, 300))
            L = pre + n_art + suf
            K = int(rng.choice([1, 100, 500, 2000, n_art - 1, n_art, int(rng.integers(1, n_art + 1))]))
            seqs.append((r0, L, pre, pre + n_art, K))
            r0 += L
            n_chunks += g
        scores = og.bf16(rng.standard_normal(r0).astype(np.float32))
        print(f"[4 keys per thread] case {case}: chunks={n_chunks} cus={cus} seqs={len(seqs)} rows={r0}", flush=True)
        keep, p = _check_select(scores, seqs, cuda)
        assert p.sel_kpt == 4 and p.sel_starts[-1] == target


def test_pack_skips_positions_outside_their_sequence(cuda):
    """A kept position outside [0, seq_len) of its sequence (what an unwritten keep entry holds)
    gathers nothing: that destination row and its position / bias entries keep their contents, the
    other rows are gathered as usual.  The kernel's own range check turns these entries into skips;
    no access leaves the source rows of the entry's sequence."""
    from tokengate_amd import gate
    seqs = [(0, 300, 10, 290, 20), (300, 500, 0, 500, 40)]
    p = gate.plan([x[0] for x in seqs], [x[1] for x in seqs], [x[2] for x in seqs], [x[3] for x in seqs],
                  [x[4] for x in seqs], cuda)
    rng = np.random.default_rng(11)
    scores = torch.from_numpy(rng.standard_normal(800).astype(np.float32)).to(cuda)
    keep, sumsq = gate.select_keep(scores, p)
    bad = keep.clone()
    # sequence 0 (300 rows): -1 and 300 (its own length); sequence 1: 10^9 and -2^40
    c0, c1 = p.cu_kept[1], p.cu_kept[2]
    bad_rows = [0, 5, c0 + 3, c1 - 1]
    bad[bad_rows[0]] = -1
    bad[bad_rows[1]] = 300
    bad[bad_rows[2]] = 10 ** 9
    bad[bad_rows[3]] = -(2 ** 40)
    src = torch.arange(800 * 8, dtype=torch.int32, device=cuda).view(800, 8)
    dst = torch.full((p.total_kept, 8), -1, dtype=torch.int32, device=cuda)
    pos = torch.full((p.total_kept,), -7, dtype=torch.int64, device=cuda)
    bias = torch.full((p.total_kept,), 5.0, dtype=torch.float32, device=cuda)
    gate.pack(bad, p, [(src, dst)], positions=pos, bias_src=scores, sumsq=sumsq, bias_out=bias)
    torch.cuda.synchronize()
    good = torch.ones(p.total_kept, dtype=torch.bool)
    good[bad_rows] = False
    k = keep.cpu().numpy()
    row_of = np.concatenate([seqs[b][0] + k[p.cu_kept[b]:p.cu_kept[b + 1]] for b in range(2)])
    d, s_ = dst.cpu(), src.cpu()
    assert torch.equal(d[good], s_[torch.from_numpy(row_of)][good])
    assert bool((d[~good] == -1).all()) and bool((pos.cpu()[~good] == -7).all())
    assert bool((bias.cpu()[~good] == 5.0).all())
    assert torch.equal(pos.cpu()[good], keep.cpu()[good])


def test_select_pack_error_word_round_trip(cuda):
    """The error word of tg_gate_select_pack's workspace stays set until reported: select_pack
    (check=True) raises on it and clears it, so the next call is clean; error_out receives it."""
    from tokengate_amd import gate
    rng = np.random.default_rng(12)
    seqs = [(0, 4000, 64, 3800, 100), (4000, 9000, 0, 9000, 700)]
    scores_np = rng.standard_normal(13000).astype(np.float32)
    scores = torch.from_numpy(scores_np).to(cuda)
    p = gate.plan([x[0] for x in seqs], [x[1] for x in seqs], [x[2] for x in seqs], [x[3] for x in seqs],
                  [x[4] for x in seqs], cuda)
    ref, _, _ = og.select_and_pack(scores_np.astype(np.float64), seqs)
    keep = gate.select_pack(scores, p, [], check=True)
    assert np.array_equal(keep.cpu().numpy(), ref)
    stream = torch.cuda.current_stream().cuda_stream
    ws = gate._SEL_WS[(torch.device(cuda).index, stream)][0]
    gate._error_word(ws).fill_(1)        # as a timed-out wait leaves it
    err = torch.zeros(1, dtype=torch.int32, pin_memory=True)
    with pytest.raises(RuntimeError, match="error word 1"):
        gate.select_pack(scores, p, [], check=True, error_out=err)
    assert int(err[0]) == 1
    assert int(gate._error_word(ws).item()) == 0      # cleared by the report
    keep2 = gate.select_pack(scores, p, [], check=True, error_out=err)
    torch.cuda.synchronize()
    assert int(err[0]) == 0 and np.array_equal(keep2.cpu().numpy(), ref)


def _threshold_batch(rng):
    """A ragged batch for the threshold mode: (scores, seqs) with seqs (row_start, len, s, e)."""
    parts, seqs, r0 = [], [], 0
    specs = [(3000, 64, 2744, "normal"), (5000, 0, 5000, "bf16"), (900, 10, 890, "zeros"), (1200, 100, 1100, "nan"),
             (700, 700, 700, "empty"), (70000, 64, 69744, "normal"), (2500, 5, 2495, "few"), (40, 3, 37, "normal")]
    for L, s, e, kind in specs:
        x = rng.standard_normal(L).astype(np.float32)
        if kind == "bf16":
            x = og.bf16(x)
        elif kind == "zeros":
            x[:] = 0.0
        elif kind == "nan":
            x[s + 17] = np.nan
        elif kind == "few":
            x = np.round(x * 2).astype(np.float32) / 2
        parts.append(x)
        seqs.append((r0, L, s, e))
        r0 += L
    return np.concatenate(parts), seqs


@pytest.mark.parametrize("tau", [0.5, 0.62, 0.4, 0.995])
def test_threshold_selection_matches_oracle(cuda, tau):
    """tg_gate_threshold_select + the top-K selection over its derived scores (gate.threshold_plan,
    then select_pack and the bias pack): the selection values bit-exact against the oracle's fp32
    chain (aggregate of the per-head bias), kept counts, keep lists bit-exact against the oracle's
    _select_threshold restatement (non-strict sigmoid(agg) >= tau; the argmax when nothing passes;
    NaN never passes), packed rows against index_select, kept positions and gate bias.  The batch
    holds the init case (every score 0: everything kept at tau 0.5), a span with a NaN (all of its
    values NaN: the argmax fallback takes the first), ties, an empty span and a 70k span."""
    from tokengate_amd import gate
    rng = np.random.default_rng(21)
    scores_np, seqs = _threshold_batch(rng)
    g = torch.Generator(device=cuda).manual_seed(3)
    head = gate.random_head(3, 16, seed=7, device=cuda)
    head.gate_scale = head.gate_scale + 0.5 * torch.randn(head.gate_scale.shape, generator=g, device=cuda)
    head.selection_mode, head.tau, head.bias_gain = "threshold", tau, 1.25
    scores = torch.from_numpy(scores_np).to(cuda)
    rs, lens, ss, es = ([x[i] for x in seqs] for i in range(4))
    p, sel, agg, sumsq, counts = gate.threshold_plan(scores, rs, lens, ss, es, head, cuda)
    b_star = gate.sigmoid_threshold(tau, cuda)
    # b_star is the device torch.sigmoid's own boundary: the two predicates agree around it
    if np.isfinite(b_star):
        u = int(np.float32(b_star).view(np.uint32))
        key = ((~u) & 0xFFFFFFFF) if u & 0x80000000 else (u | 0x80000000)
        near = torch.from_numpy(gate._f32_of_keys(key + np.arange(-512, 513)).copy()).to(cuda)
        assert torch.equal(torch.sigmoid(near) >= tau, near >= b_star)
    sp = np.asarray(head.selection_head_scale(), np.float32)
    gs = head.gate_scale.float().cpu().numpy()
    assert np.array_equal(sp, og.softplus32(gs[0])) or np.abs(sp - og.softplus32(gs[0])).max() <= 1.2e-7
    agg_np = agg.cpu().numpy()
    src = torch.arange(len(scores_np) * 8, dtype=torch.int32, device=cuda).view(-1, 8)
    dst = torch.full((p.total_kept, 8), -1, dtype=torch.int32, device=cuda)
    pos = torch.full((p.total_kept,), -7, dtype=torch.int64, device=cuda)
    bias = torch.full((p.total_kept,), float("nan"), dtype=torch.float32, device=cuda)
    keep = gate.select_pack(sel, p, [(src, dst)], positions=pos, check=True)
    gate.pack(keep, p, [], bias_src=scores, sumsq=sumsq, bias_out=bias)
    torch.cuda.synchronize()
    keep_np, pos_np, bias_np, dst_np = keep.cpu().numpy(), pos.cpu().numpy(), bias.cpu().numpy(), dst.cpu().numpy()
    src_np = src.cpu().numpy()
    for b, (r0, L, s, e) in enumerate(seqs):
        raw = scores_np[r0 + s:r0 + e]
        # the oracle's chain (gate_bias_layers then aggregate) with the product's softplus values
        b0 = (og.seq_rms_norm(raw, gain=1.25)[:, None] * sp[None, :]).astype(np.float32)[:, None, :]
        want_agg = og.aggregate(b0)
        got_agg = agg_np[r0 + s:r0 + e]
        assert np.array_equal(got_agg, want_agg, equal_nan=True), f"seq {b}: selection values differ"
        with np.errstate(invalid="ignore"):
            assert counts[b] == int(np.sum(want_agg >= np.float32(b_star))), f"seq {b}: count"
        want = og.threshold_keep_indices(want_agg, b_star, s, e, L)
        c0, c1 = p.cu_kept[b], p.cu_kept[b + 1]
        assert np.array_equal(keep_np[c0:c1], want), f"seq {b}: keep list differs (tau {tau})"
        assert np.array_equal(pos_np[c0:c1], want)
        assert np.array_equal(dst_np[c0:c1], src_np[r0 + want])
        if np.isfinite(raw).all():
            np.testing.assert_allclose(bias_np[c0:c1], og.gate_bias(raw, want, s, e), rtol=2e-6, atol=1e-30)
    if tau == 0.5:
        assert counts[2] == 900 - 20         # every score 0: the whole span passes
    assert counts[4] == 0 and p.n_kept[4] == 700   # empty span: prefix and suffix only
    assert counts[3] == 0                    # a NaN makes the span's values NaN: the argmax fallback
