"""Pins the attention oracle (CPU) against library routines and invariants.

Each check is chosen so that a plausible mistake in the oracle fails it: a dropped or unscaled
bias (SDPA with an additive float mask), a wrong GQA head mapping (SDPA enable_gqa / repeat),
log2 instead of natural LSE (torch.logsumexp), top-left instead of bottom-right causal alignment
(row-suffix invariant), a wrong dBias scale or sign (autograd through SDPA; finite differences).
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as ora


def _inputs(B, Sq, Sk, H, Hkv, D, seed, bias=True):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Sq, H, D, generator=g).to(torch.bfloat16).double()
    k = torch.randn(B, Sk, Hkv, D, generator=g).to(torch.bfloat16).double()
    v = torch.randn(B, Sk, Hkv, D, generator=g).to(torch.bfloat16).double()
    b = (torch.randn(B, H, Sk, generator=g) * 3.0).double() if bias else None
    return q, k, v, b


def _sdpa(q, k, v, bias_raw, scale, causal):
    """torch SDPA (math path, float64) with the key bias as an additive float mask."""
    B, Sq, H, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    qt, kt, vt = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    mask = torch.zeros(B, H, Sq, Sk, dtype=q.dtype)
    if bias_raw is not None:
        mask = mask + scale * bias_raw[:, :, None, :]
    if causal:
        i = torch.arange(Sq)[:, None]
        j = torch.arange(Sk)[None, :]
        mask = mask.masked_fill(j > i + (Sk - Sq), float("-inf"))
    out = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=scale, enable_gqa=(H != Hkv))
    logits = (qt @ kt.repeat_interleave(H // Hkv, 1).transpose(-1, -2)) * scale + mask
    return out.transpose(1, 2), torch.logsumexp(logits, dim=-1)


@pytest.mark.parametrize("H,Hkv", [(4, 4), (4, 2), (6, 2), (8, 1)])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("with_bias", [True, False])
def test_fwd_matches_sdpa(H, Hkv, causal, with_bias):
    q, k, v, b = _inputs(2, 37, 37, H, Hkv, 16, seed=H * 10 + Hkv, bias=with_bias)
    scale = 16 ** -0.5
    out, lse = ora.keybias_fwd(q.numpy(), k.numpy(), v.numpy(), None if b is None else b.numpy(), scale, causal)
    ro, rl = _sdpa(q, k, v, b, scale, causal)
    np.testing.assert_allclose(out, ro.numpy(), rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(lse, rl.numpy(), rtol=1e-10, atol=1e-10)


def test_bias_shift_invariance():
    q, k, v, b = _inputs(1, 20, 20, 4, 2, 8, seed=3)
    scale = 8 ** -0.5
    o1, l1 = ora.keybias_fwd(q.numpy(), k.numpy(), v.numpy(), b.numpy(), scale, True)
    o2, l2 = ora.keybias_fwd(q.numpy(), k.numpy(), v.numpy(), b.numpy() + 5.0, scale, True)
    np.testing.assert_allclose(o1, o2, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(l2, l1 + 5.0 * scale, rtol=1e-12, atol=1e-12)


def test_pad_bias_removes_key():
    """bias -1e9 (logit units) on key j is attention without key j (the reference's pad rule)."""
    q, k, v, b = _inputs(1, 9, 12, 2, 1, 8, seed=4)
    scale = 8 ** -0.5
    bb = b.numpy().copy()
    bb[:, :, 5] = -1e9 / scale
    o1, _ = ora.keybias_fwd(q.numpy(), k.numpy(), v.numpy(), bb, scale, False)
    keep = [j for j in range(12) if j != 5]
    o2, _ = ora.keybias_fwd(q.numpy(), k.numpy()[:, keep], v.numpy()[:, keep], b.numpy()[:, :, keep], scale, False)
    np.testing.assert_allclose(o1, o2, rtol=1e-12, atol=1e-12)


def test_causal_alignment_is_bottom_right():
    """Sq < Sk: the rows equal the last Sq rows of the square causal attention;
    Sq > Sk: the first Sq-Sk rows see nothing (out 0, lse +inf), the rest equal the square case."""
    q, k, v, b = _inputs(1, 30, 30, 4, 2, 8, seed=5)
    scale = 8 ** -0.5
    full_o, full_l = ora.keybias_fwd(q.numpy(), k.numpy(), v.numpy(), b.numpy(), scale, True)
    o, l = ora.keybias_fwd(q.numpy()[:, 18:], k.numpy(), v.numpy(), b.numpy(), scale, True)
    np.testing.assert_allclose(o, full_o[:, 18:], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(l, full_l[:, :, 18:], rtol=1e-12, atol=1e-12)
    q2 = np.concatenate([np.random.default_rng(0).standard_normal((1, 7, 4, 8)), q.numpy()], axis=1)
    o2, l2 = ora.keybias_fwd(q2, k.numpy(), v.numpy(), b.numpy(), scale, True)
    assert np.all(o2[:, :7] == 0) and np.all(np.isinf(l2[:, :, :7]))
    np.testing.assert_allclose(o2[:, 7:], full_o, rtol=1e-12, atol=1e-12)


def test_rows_subset_matches_full():
    q, k, v, b = _inputs(1, 50, 50, 4, 2, 8, seed=6)
    scale = 8 ** -0.5
    fo, fl = ora.keybias_fwd(q.numpy(), k.numpy(), v.numpy(), b.numpy(), scale, True)
    rows = np.array([0, 7, 31, 49])
    so, sl = ora.keybias_fwd(q.numpy(), k.numpy(), v.numpy(), b.numpy(), scale, True, rows=rows)
    np.testing.assert_allclose(so, fo[:, rows], rtol=1e-12)
    np.testing.assert_allclose(sl, fl[:, :, rows], rtol=1e-12)


@pytest.mark.parametrize("H,Hkv,causal", [(4, 2, True), (4, 4, False), (6, 2, True)])
def test_bwd_matches_autograd(H, Hkv, causal):
    q, k, v, b = _inputs(2, 23, 23, H, Hkv, 8, seed=7 + H)
    scale = 8 ** -0.5
    g = torch.Generator().manual_seed(99)
    dout = torch.randn(2, 23, H, 8, generator=g).double()
    qr, kr, vr, br = [t.clone().requires_grad_(True) for t in (q, k, v, b)]
    out, _ = _sdpa(qr, kr, vr, br, scale, causal)
    (out * dout).sum().backward()
    dq, dk, dv, dbias, sd = ora.keybias_bwd(dout.numpy(), q.numpy(), k.numpy(), v.numpy(), b.numpy(), scale, causal)
    np.testing.assert_allclose(dq, qr.grad.numpy(), rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(dk, kr.grad.numpy(), rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(dv, vr.grad.numpy(), rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(dbias, br.grad.numpy(), rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(sd, (out.detach() * dout).sum(-1).transpose(1, 2).numpy(), rtol=1e-9, atol=1e-10)


def test_dbias_finite_difference():
    """dL/dbias_raw by central differences: the scale factor and sign of the bias gradient."""
    q, k, v, b = _inputs(1, 6, 6, 2, 1, 4, seed=8)
    scale = 0.37
    rng = np.random.default_rng(1)
    dout = rng.standard_normal((1, 6, 2, 4))
    _, _, _, dbias, _ = ora.keybias_bwd(dout, q.numpy(), k.numpy(), v.numpy(), b.numpy(), scale, True)

    def loss(bb):
        o, _ = ora.keybias_fwd(q.numpy(), k.numpy(), v.numpy(), bb, scale, True)
        return float((o * dout).sum())

    eps = 1e-6
    for (h, j) in [(0, 0), (1, 3), (0, 5)]:
        bp = b.numpy().copy(); bp[0, h, j] += eps
        bm = b.numpy().copy(); bm[0, h, j] -= eps
        fd = (loss(bp) - loss(bm)) / (2 * eps)
        assert abs(fd - dbias[0, h, j]) < 1e-6 * max(1.0, abs(fd)), (h, j, fd, dbias[0, h, j])


def test_varlen_matches_block_diagonal_sdpa():
    lens = [5, 1, 9, 0, 4]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    total, H, Hkv, D = int(cu[-1]), 4, 2, 8
    g = torch.Generator().manual_seed(10)
    q = torch.randn(total, H, D, generator=g).double()
    k = torch.randn(total, Hkv, D, generator=g).double()
    v = torch.randn(total, Hkv, D, generator=g).double()
    bias = torch.randn(len(lens), H, max(lens), generator=g).double()
    scale = D ** -0.5
    out, lse = ora.keybias_varlen_fwd(q.numpy(), k.numpy(), v.numpy(), bias.numpy(), cu, scale, True)
    # one packed row with a block-diagonal causal mask and each key's own-sequence bias
    seq = np.repeat(np.arange(len(lens)), lens)
    pos = np.concatenate([np.arange(n) for n in lens])
    mask = torch.full((H, total, total), float("-inf"), dtype=torch.float64)
    for i in range(total):
        for j in range(total):
            if seq[i] == seq[j] and pos[j] <= pos[i]:
                mask[:, i, j] = scale * bias[seq[j], :, pos[j]]
    ro = F.scaled_dot_product_attention(q.transpose(0, 1)[None], k.transpose(0, 1)[None], v.transpose(0, 1)[None],
                                        attn_mask=mask[None], scale=scale, enable_gqa=True)[0].transpose(0, 1)
    np.testing.assert_allclose(out, ro.numpy(), rtol=1e-10, atol=1e-10)
    logits = (q.transpose(0, 1) @ k.transpose(0, 1).repeat_interleave(2, 0).transpose(-1, -2)) * scale + mask
    np.testing.assert_allclose(lse, torch.logsumexp(logits, -1).numpy(), rtol=1e-10, atol=1e-10)


def test_bf16_round_matches_torch():
    x = np.random.default_rng(0).standard_normal(10000).astype(np.float32) * 100
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ora.bf16_round(x), ref)


@pytest.mark.parametrize("causal", [True, False])
def test_torch_oracle_matches_numpy(causal):
    from oracle import attention_torch as ort
    q, k, v, b = _inputs(2, 41, 45, 6, 2, 16, seed=21)
    scale = 16 ** -0.5
    g = torch.Generator().manual_seed(5)
    dout = torch.randn(2, 41, 6, 16, generator=g).double()
    o, l = ora.keybias_fwd(q.numpy(), k.numpy(), v.numpy(), b.numpy(), scale, causal)
    to, tl = ort.fwd(q.float(), k.float(), v.float(), b.float(), scale, causal, chunk=16)
    np.testing.assert_allclose(to.numpy(), o, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(tl.numpy(), l, rtol=1e-5, atol=1e-5)
    ref = ora.keybias_bwd(dout.numpy(), q.numpy(), k.numpy(), v.numpy(), b.numpy(), scale, causal)
    got = ort.bwd(dout.float(), q.float(), k.float(), v.float(), b.float(), scale, causal, chunk=16)
    for r, t in zip(ref, got):
        np.testing.assert_allclose(t.numpy(), r, rtol=1e-3, atol=1e-4)
    if causal:
        # sampled query rows of a self-attention (Sq = Sk) against the numpy oracle's `rows`
        q2, k2, v2, b2 = _inputs(1, 45, 45, 6, 2, 16, seed=22)
        rows = np.array([0, 3, 20, 44])
        o2, l2 = ora.keybias_fwd(q2.numpy(), k2.numpy(), v2.numpy(), b2.numpy(), scale, True, rows=rows)
        t2, tl2 = ort.fwd(q2[:, rows].float(), k2.float(), v2.float(), b2.float(), scale, True, chunk=3,
                          q_pos=torch.from_numpy(rows))
        np.testing.assert_allclose(t2.numpy(), o2, rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(tl2.numpy(), l2, rtol=1e-5, atol=1e-5)


def test_bwd_given_out_and_bf16_operands():
    """The backward's two options.  out: D = rowsum(dO * out) from the output handed in — with the
    oracle's own forward output it is the default; with the output perturbed, only D (softmax_d)
    and the dS-derived gradients move (dV = P^T dO does not depend on D).  bf16_operands: exact
    when P and dS are bf16 values (uniform attention over 8 keys, small-integer V / dO); on random
    inputs every changed gradient stays within the rounding bound 2^-8 * sum |x_i y_i| of its
    products and differs from the exact one."""
    q, k, v, b = _inputs(1, 12, 12, 4, 2, 16, seed=31)
    g = torch.Generator().manual_seed(32)
    dout = torch.randn(1, 12, 4, 16, generator=g).double().numpy()
    scale = 16 ** -0.5
    args = (dout, q.numpy(), k.numpy(), v.numpy(), b.numpy(), scale, True)
    ref = ora.keybias_bwd(*args)
    o, _ = ora.keybias_fwd(*args[1:])
    same = ora.keybias_bwd(*args, out=o)
    for r, t in zip(ref, same):
        np.testing.assert_array_equal(r, t)
    moved = ora.keybias_bwd(*args, out=o * 1.01)
    np.testing.assert_allclose(moved[4], 1.01 * ref[4], rtol=1e-12)
    np.testing.assert_array_equal(moved[2], ref[2])
    assert not np.allclose(moved[0], ref[0]) and not np.allclose(moved[3], ref[3])

    # bf16-exact operands: non-causal, q = 0 and bias 0 -> P = 1/8; V, dO in {-1, 0, 1}, head dim 4
    rng = np.random.default_rng(33)
    Dh = 4
    qz = np.zeros((1, 8, 2, Dh))
    kk = rng.integers(-1, 2, (1, 8, 1, Dh)).astype(np.float64)
    vv = rng.integers(-1, 2, (1, 8, 1, Dh)).astype(np.float64)
    dd = rng.integers(-1, 2, (1, 8, 2, Dh)).astype(np.float64)
    e = ora.keybias_bwd(dd, qz, kk, vv, None, 0.5, False)
    r = ora.keybias_bwd(dd, qz, kk, vv, None, 0.5, False, bf16_operands=True)
    for x, y in zip(e[:3], r[:3]):      # exp(-ln 8) is 1/8 to within float64 rounding
        np.testing.assert_allclose(x, y, rtol=1e-12, atol=1e-15)

    # random operands: bounded, and not a no-op
    q, k, v, b = _inputs(1, 40, 40, 2, 1, 16, seed=34)
    dout = torch.randn(1, 40, 2, 16, generator=g).double().numpy()
    e = ora.keybias_bwd(dout, q.numpy(), k.numpy(), v.numpy(), b.numpy(), scale, True)
    r = ora.keybias_bwd(dout, q.numpy(), k.numpy(), v.numpy(), b.numpy(), scale, True, bf16_operands=True)
    np.testing.assert_array_equal(e[3], r[3])
    np.testing.assert_array_equal(e[4], r[4])
    # |sum r(x) y - sum x y| <= 2^-8 sum |x| |y|, with x = P or dS (from the exact run's own P, dS)
    out, lse = ora.keybias_fwd(q.numpy(), k.numpy(), v.numpy(), b.numpy(), scale, True)
    z = ora._logits(q.numpy()[0, :, 0], k.numpy()[0, :, 0], b.numpy()[0, 0], scale, True, np.arange(40), 40, 40)
    p = np.exp(z - lse[0, 0][:, None])
    do = dout[0, :, 0]
    ds = p * (do @ v.numpy()[0, :, 0].T - (do * out[0, :, 0]).sum(1)[:, None])
    # head 0's contribution to dq (one head per query row)
    bound_dq = 2.0 ** -8 * scale * np.abs(ds) @ np.abs(k.numpy()[0, :, 0])
    assert np.all(np.abs(r[0][0, :, 0] - e[0][0, :, 0]) <= bound_dq + 1e-12)
    assert np.abs(r[0] - e[0]).max() > 0 and np.abs(r[1] - e[1]).max() > 0 and np.abs(r[2] - e[2]).max() > 0


@pytest.mark.parametrize("bf16_operands", [False, True])
def test_torch_oracle_bwd_options_match_numpy(bf16_operands):
    from oracle import attention_torch as ort
    q, k, v, b = _inputs(2, 33, 33, 4, 2, 16, seed=41)
    scale = 16 ** -0.5
    g = torch.Generator().manual_seed(6)
    dout = torch.randn(2, 33, 4, 16, generator=g).double()
    o, _ = ora.keybias_fwd(q.numpy(), k.numpy(), v.numpy(), b.numpy(), scale, True)
    o16 = ora.bf16_round(o).astype(np.float64)
    ref = ora.keybias_bwd(dout.numpy(), q.numpy(), k.numpy(), v.numpy(), b.numpy(), scale, True, out=o16,
                          bf16_operands=bf16_operands)
    got = ort.bwd(dout.float(), q.float(), k.float(), v.float(), b.float(), scale, True, chunk=16,
                  out=torch.from_numpy(o16).float(), bf16_operands=bf16_operands)
    for name, r, t in zip(["dq", "dk", "dv", "dbias", "sd"], ref, got):
        # fp32 vs float64 evaluation: an operand near a bf16 rounding boundary may round the other
        # way (one bf16 unit of that operand), hence the absolute term
        np.testing.assert_allclose(t.numpy(), r, rtol=2e-3, atol=2e-3, err_msg=name)
