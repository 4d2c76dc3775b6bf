"""Seeded random-shape parity of the key-bias attention (forward, backward, varlen forward) against
the float64 oracle: batch sizes, unequal and odd lengths, GQA group sizes 1-4, softmax scales,
bias kinds (none, per head, broadcast over heads, with -1e9 padding keys) drawn from one numpy
generator, so that combinations the hand-picked cases do not name are covered as well.  The
fa2bias entry points plan the key-range split themselves, so small random grids exercise it too.
Tolerance: max-abs <= 2e-2 and rel-L2 <= 1e-2 (gradients: tests/attn_util.check_bwd — fp32
outputs absolute against the exact math; bf16 outputs ulp-relative against the exact math and
absolute below 4 against the math with P and dS rounded to bf16 as the reference kernel rounds
them; D and P from the forward output and log-sum-exp handed to the backward).  The varlen backward
draws ragged batches with one sequence of 8k+ tokens (the reference's only varlen user is packed
training, gate_forward.py:2097-2159 -> keybias.py:90-141) and checks each sequence against the
float32 torch evaluation on the device.
"""
import numpy as np
import pytest
import torch

from oracle import attention as ora
from oracle import attention_torch as ort
from tests.attn_util import assert_close, check_bwd, to_np

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
    a = (to_np(dout), to_np(q), to_np(k), to_np(v), to_np(bias_raw), scale, causal)
    ex = ora.keybias_bwd(*a, out=to_np(out), lse=to_np(lse))
    fa = ora.keybias_bwd(*a, out=to_np(out), lse=to_np(lse), bf16_operands=True)
    check_bwd(f"{cfg}", [to_np(t) for t in (dq, dk, dv, db, sd)], ex, fa)


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


@pytest.mark.parametrize("i", range(5))
def test_random_varlen_backward(cuda, i):
    rng = np.random.default_rng(4000 + i)
    n = int(rng.integers(2, 6))
    lens = [int(x) for x in rng.integers(0, 2500, size=n)]
    if i < 3:
        lens[int(rng.integers(n))] = int(rng.integers(8192, 9700))     # one sequence of 8k+ tokens
    lens[0] = max(lens[0], 1)
    H, Hkv = GROUPS[rng.integers(len(GROUPS))] if i else (16, 8)
    causal = bool(rng.random() < 0.8) or i == 0
    scale = float(rng.uniform(0.07, 0.12))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    total, maxlen = int(cu[-1]), max(lens)
    g = torch.Generator(device=cuda).manual_seed(19 * i + 4)
    q = (torch.randn(total, H, 128, generator=g, device=cuda) * 0.7).to(torch.bfloat16)
    k = (torch.randn(total, Hkv, 128, generator=g, device=cuda) * 0.7).to(torch.bfloat16)
    v = torch.randn(total, Hkv, 128, generator=g, device=cuda).to(torch.bfloat16)
    dout = torch.randn(total, H, 128, generator=g, device=cuda).to(torch.bfloat16)
    with_bias = i == 0 or rng.random() < 0.7
    bias_raw = None
    if with_bias:
        kb = torch.nn.functional.logsigmoid(torch.randn(n, H, maxlen, generator=g, device=cuda) * 2.0)
        bias_raw = (kb / scale).contiguous()
    from tokengate_amd.fa2bias.keybias import ext
    cu_t = torch.tensor(cu, device=cuda)
    out, lse, _, _ = ext().varlen_fwd(q, k, v, None, cu_t, cu_t, None, None, None, bias_raw, maxlen, maxlen,
                                      0.0, scale, False, causal, -1, -1, 0.0, False, None)
    dq, dk, dv, sd, db = ext().varlen_bwd(dout, q, k, v, out, lse, None, None, None, cu_t, cu_t, bias_raw,
                                          maxlen, maxlen, 0.0, scale, False, causal, -1, -1, 0.0, False, None, None)
    torch.cuda.synchronize()
    tag = f"lens={lens} H={H}/{Hkv} causal={causal} bias={with_bias}"
    print(f"[varlen bwd] {tag}", flush=True)
    for s_, (st, ln) in enumerate(ora.varlen_to_dense(cu)):
        if ln == 0:
            continue
        sl = slice(st, st + ln)
        br = None if bias_raw is None else bias_raw[s_:s_ + 1, :, :ln].contiguous()
        a = (dout[None, sl], q[None, sl], k[None, sl], v[None, sl], br, scale, causal)
        ls = lse[None, :, sl].contiguous()
        ex = ort.bwd(*a, chunk=2048, out=out[None, sl], lse=ls)
        fa = ort.bwd(*a, chunk=2048, out=out[None, sl], lse=ls, bf16_operands=True)
        got = [dq[None, sl], dk[None, sl], dv[None, sl], None if db is None else db[s_:s_ + 1, :, :ln],
               sd[None, :, sl]]
        check_bwd(f"varlen seq {s_} ({ln})", [None if t is None else to_np(t) for t in got],
                  [None if t is None else to_np(t) for t in ex], [None if t is None else to_np(t) for t in fa])
