"""Seeded random-shape parity of the key-bias attention (forward, backward, varlen forward) against
the float64 oracle: batch sizes, unequal and odd lengths, GQA group sizes 1-4, softmax scales,
bias kinds (none, per head, broadcast over heads, with -1e9 padding keys) drawn from one numpy
generator, so that combinations the hand-picked cases do not name are covered as well.  The
fa2bias entry points plan the key-range split themselves, so small random grids exercise it too.
Tolerance: max-abs <= 2e-2 and rel-L2 <= 1e-2 (gradients: max-abs relative to max(1, max|ref|)).
"""
import numpy as np
import pytest
import torch

from oracle import attention as ora
from tests.attn_util import assert_close, assert_close_grad, to_np

pytestmark = pytest.mark.gpu

GROUPS = [(16, 8), (4, 4), (6, 2), (8, 2), (12, 4), (2, 1), (8, 8)]


def _draw(rng):
    H, Hkv = GROUPS[rng.integers(len(GROUPS))]
    B = int(rng.integers(1, 4))
    sq = int(rng.integers(1, 700))
    sk = sq if rng.random() < 0.6 else int(rng.integers(1, 700))
    causal = bool(rng.random() < 0.7)
    kind = ["none", "per_head", "broadcast"][rng.integers(3)]
    scale = float(rng.uniform(0.05, 0.15))
    pad = int(rng.integers(0, 65)) if kind != "none" and rng.random() < 0.3 else 0
    return B, sq, sk, H, Hkv, causal, kind, scale, pad


def _inputs(cfg, seed, dev):
    B, sq, sk, H, Hkv, causal, kind, scale, pad = cfg
    g = torch.Generator(device=dev).manual_seed(seed)
    q = (torch.randn(B, sq, H, 128, generator=g, device=dev) * 0.7).to(torch.bfloat16)
    k = (torch.randn(B, sk, Hkv, 128, generator=g, device=dev) * 0.7).to(torch.bfloat16)
    v = torch.randn(B, sk, Hkv, 128, generator=g, device=dev).to(torch.bfloat16)
    bias_raw = None
    if kind != "none":
        kb = torch.randn(B, H if kind == "per_head" else 1, sk, generator=g, device=dev) * 2.0
        pad = min(pad, sk - 1)   # key 0 stays unpadded: every row sees at least one real key
        if pad:
            kb[..., sk - pad:] = -1e9
        bias_raw = (kb.expand(B, H, sk) / scale).contiguous()
    return q, k, v, bias_raw


@pytest.mark.parametrize("i", range(16))
def test_random_forward(cuda, i):
    rng = np.random.default_rng(1000 + i)
    cfg = _draw(rng)
    B, sq, sk, H, Hkv, causal, kind, scale, pad = cfg
    if causal and sq > sk:
        sq = sk   # causal with more queries than keys leaves rows with no key (covered elsewhere)
        cfg = (B, sq, sk, H, Hkv, causal, kind, scale, pad)
    q, k, v, bias_raw = _inputs(cfg, 7 * i + 3, cuda)
    from tokengate_amd.fa2bias.keybias import ext
    out, lse, _, _ = ext().fwd(q, k, v, None, bias_raw, 0.0, scale, causal, -1, -1, 0.0, False, None)
    torch.cuda.synchronize()
    ro, rl = ora.keybias_fwd(to_np(q), to_np(k), to_np(v), None if bias_raw is None else to_np(bias_raw),
                             scale, causal)
    assert_close(f"out {cfg}", to_np(out), ro)
    assert_close(f"lse {cfg}", to_np(lse), rl)


@pytest.mark.parametrize("i", range(8))
def test_random_backward(cuda, i):
    rng = np.random.default_rng(2000 + i)
    B, sq, sk, H, Hkv, causal, kind, scale, pad = _draw(rng)
    sq = min(sq, 300)
    sk = sq if causal else min(sk, 300)
    cfg = (B, sq, sk, H, Hkv, causal, kind, scale, pad)
    q, k, v, bias_raw = _inputs(cfg, 11 * i + 5, cuda)
    if bias_raw is None:
        bias_raw = torch.zeros(B, H, sk, device=cuda)
    g = torch.Generator(device=cuda).manual_seed(13 * i + 1)
    dout = torch.randn(B, sq, H, 128, generator=g, device=cuda).to(torch.bfloat16)
    from tokengate_amd.fa2bias.keybias import ext
    out, lse, _, _ = ext().fwd(q, k, v, None, bias_raw, 0.0, scale, causal, -1, -1, 0.0, False, None)
    dq, dk, dv, sd, db = ext().bwd(dout, q, k, v, out, lse, None, None, None, bias_raw, 0.0, scale, causal,
                                   -1, -1, 0.0, False, None, None)
    torch.cuda.synchronize()
    r = ora.keybias_bwd(to_np(dout), to_np(q), to_np(k), to_np(v), to_np(bias_raw), scale, causal)
    for name, got, ref in zip(["dq", "dk", "dv", "dbias_raw", "softmax_d"], [dq, dk, dv, db, sd], r):
        assert_close_grad(f"{name} {cfg}", to_np(got), ref)


@pytest.mark.parametrize("i", range(6))
def test_random_varlen_forward(cuda, i):
    rng = np.random.default_rng(3000 + i)
    n = int(rng.integers(1, 7))
    lens = [int(x) for x in rng.integers(0, 600, size=n)]
    lens[int(rng.integers(n))] = max(lens[0], 1)   # at least one non-empty sequence
    H, Hkv = GROUPS[rng.integers(len(GROUPS))]
    causal = bool(rng.random() < 0.7)
    scale = float(rng.uniform(0.05, 0.15))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    total, maxlen = int(cu[-1]), max(lens)
    g = torch.Generator(device=cuda).manual_seed(17 * i + 2)
    q = (torch.randn(total, H, 128, generator=g, device=cuda) * 0.7).to(torch.bfloat16)
    k = (torch.randn(total, Hkv, 128, generator=g, device=cuda) * 0.7).to(torch.bfloat16)
    v = torch.randn(total, Hkv, 128, generator=g, device=cuda).to(torch.bfloat16)
    bias_raw = (torch.randn(n, H, maxlen, generator=g, device=cuda) * 2.0 / scale).contiguous() \
        if rng.random() < 0.7 else None
    from tokengate_amd.fa2bias.keybias import ext
    cu_t = torch.tensor(cu, device=cuda)
    out, lse, _, _ = ext().varlen_fwd(q, k, v, None, cu_t, cu_t, None, None, None, bias_raw, maxlen, maxlen,
                                      0.0, scale, False, causal, -1, -1, 0.0, False, None)
    torch.cuda.synchronize()
    ro, rl = ora.keybias_varlen_fwd(to_np(q), to_np(k), to_np(v), None if bias_raw is None else to_np(bias_raw),
                                    cu, scale, causal)
    tag = f"lens={lens} H={H}/{Hkv} causal={causal}"
    assert_close(f"varlen out {tag}", to_np(out), ro)
    assert_close(f"varlen lse {tag}", to_np(lse), rl)
