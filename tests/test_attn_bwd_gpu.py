"""GPU parity of the key-bias attention backward (dQ, dK, dV, dBias, softmax_d).

Small shapes against the float64 numpy oracle; the reference's own GPU-test shapes
(tests/attention/test_attention_backends_grad.py:21-31,65: S in {1024, 4096, 4093}, H16/Hkv8,
inputs randn*0.5, bias randn*2 with the last 64 keys at -1e9) and the B4 x 8192 training shape
against the float32 torch evaluation of the same math on the device.  Both oracles take D and P
from the forward output and log-sum-exp the kernel was handed (the reference's op saves the bf16
`out` and the fp32 `lse`; its FA2 backward forms D = rowsum(dO * out) and P = exp(z - lse) from
them).  Tolerances (tests/attn_util.check_bwd; absolute
max-abs and rel-L2 of every gradient printed): dBias and softmax_d (fp32 outputs) max-abs <= 2e-2
and rel-L2 <= 1e-2 against the exact math; dQ/dK/dV (bf16 outputs) rel-L2 <= 1e-2 and max-abs
<= 2e-2 relative to max(1, max|ref|) against the exact math, and max-abs <= 2e-2 on entries below
4 (2e-2 * |ref| / 4 above) against the same math with P and dS rounded to bf16 where the reference
kernel rounds them (oracle bf16_operands).
"""
import numpy as np
import pytest
import torch

from oracle import attention as ora
from oracle import attention_torch as ort
from tests.attn_util import bias_logsigmoid, check_bwd, qkv, to_np


def _np_oracles(dout, q, k, v, bias_raw, scale, causal, out, lse):
    a = (to_np(dout), to_np(q), to_np(k), to_np(v), None if bias_raw is None else to_np(bias_raw), scale, causal)
    kw = dict(out=to_np(out), lse=to_np(lse))
    return ora.keybias_bwd(*a, **kw), ora.keybias_bwd(*a, **kw, bf16_operands=True)

pytestmark = pytest.mark.gpu


def _fwd_bwd(q, k, v, bias_raw, dout, scale, causal):
    from tokengate_amd.fa2bias.keybias import ext
    out, lse, _, _ = ext().fwd(q, k, v, None, bias_raw, 0.0, scale, causal, -1, -1, 0.0, False, None)
    dq, dk, dv, sd, db = ext().bwd(dout, q, k, v, out, lse, None, None, None, bias_raw, 0.0, scale, causal,
                                   -1, -1, 0.0, False, None, None)
    torch.cuda.synchronize()
    return dq, dk, dv, db, sd, out, lse


@pytest.mark.parametrize("S", [1, 33, 64, 100, 257])
@pytest.mark.parametrize("H,Hkv", [(16, 8), (4, 4), (6, 2), (8, 2)])
@pytest.mark.parametrize("causal", [True, False])
def test_bwd_small_vs_oracle(cuda, S, H, Hkv, causal):
    g = torch.Generator(device=cuda).manual_seed(S * 7 + H + (1 if causal else 0))
    q, k, v = qkv(2, S, S, H, Hkv, g, cuda)
    scale = 128 ** -0.5
    bias_raw = (torch.randn(2, H, S, device=cuda, generator=g) * 2.0 / scale).contiguous()
    dout = torch.randn(2, S, H, 128, device=cuda, generator=g).to(torch.bfloat16)
    dq, dk, dv, db, sd, out, lse = _fwd_bwd(q, k, v, bias_raw, dout, scale, causal)
    ex, fa = _np_oracles(dout, q, k, v, bias_raw, scale, causal, out, lse)
    check_bwd(f"S={S} H={H}/{Hkv} causal={causal}", [to_np(t) for t in (dq, dk, dv, db, sd)], ex, fa)


@pytest.mark.parametrize("Sq,Sk", [(100, 300), (300, 100), (129, 128)])
def test_bwd_unequal_lengths(cuda, Sq, Sk):
    g = torch.Generator(device=cuda).manual_seed(Sq * 3 + Sk)
    H, Hkv = 16, 8
    q, k, v = qkv(1, Sq, Sk, H, Hkv, g, cuda)
    scale = 128 ** -0.5
    bias_raw = (torch.randn(1, H, Sk, device=cuda, generator=g) / scale).contiguous()
    dout = torch.randn(1, Sq, H, 128, device=cuda, generator=g).to(torch.bfloat16)
    for causal in (True, False):
        dq, dk, dv, db, sd, out, lse = _fwd_bwd(q, k, v, bias_raw, dout, scale, causal)
        ex, fa = _np_oracles(dout, q, k, v, bias_raw, scale, causal, out, lse)
        check_bwd(f"Sq={Sq} Sk={Sk} causal={causal}", [to_np(t) for t in (dq, dk, dv, db, sd)], ex, fa)


def test_bwd_no_bias(cuda):
    g = torch.Generator(device=cuda).manual_seed(5)
    q, k, v = qkv(1, 200, 200, 16, 8, g, cuda)
    scale = 128 ** -0.5
    dout = torch.randn(1, 200, 16, 128, device=cuda, generator=g).to(torch.bfloat16)
    dq, dk, dv, db, sd, out, lse = _fwd_bwd(q, k, v, None, dout, scale, True)
    assert db is None
    ex, fa = _np_oracles(dout, q, k, v, None, scale, True, out, lse)
    check_bwd("no-bias", [to_np(t) for t in (dq, dk, dv)] + [None, to_np(sd)], ex, fa)


@pytest.mark.parametrize("S", [1024, 4096, 4093])
def test_reference_grad_test_shapes_autograd(cuda, S):
    """The public op's autograd (flash_attn_key_bias) against the fp32 evaluation: dQ, dK, dV and the
    gradient of the per-head bias in logit units (keybias.py:85-87 divides by the scale)."""
    from tokengate_amd.fa2bias.keybias import flash_attn_key_bias
    g = torch.Generator(device=cuda).manual_seed(0)
    B, H, Hkv, D = 1, 16, 8, 128
    mk = lambda h: (torch.randn(B, h, S, D, device=cuda, generator=g) * 0.5).to(torch.bfloat16)
    Q, K, V = mk(H), mk(Hkv), mk(Hkv)
    bias = torch.randn(S, H, device=cuda, generator=g) * 2.0
    bias[-64:] = -1e9
    dO = torch.randn(B, H, S, D, device=cuda, generator=g).to(torch.bfloat16)
    scale = D ** -0.5
    q, k, v = [t.transpose(1, 2).detach().requires_grad_(True) for t in (Q, K, V)]
    key_bias = bias.t().unsqueeze(0).detach().requires_grad_(True)        # (1, H, S)
    out = flash_attn_key_bias(q, k, v, key_bias, scale, causal=True)
    out.backward(dO.transpose(1, 2))
    torch.cuda.synchronize()
    braw = (key_bias.detach().float() / scale).contiguous()
    _, lse = torch.ops.recursive_kvs.fa2_keybias_fwd(q.detach(), k.detach(), v.detach(), braw, scale, True)
    args = (dO.transpose(1, 2), q.detach(), k.detach(), v.detach(), braw, scale, True)
    ex = ort.bwd(*args, out=out.detach(), lse=lse)
    fa = ort.bwd(*args, out=out.detach(), lse=lse, bf16_operands=True)
    # d/d key_bias = (d/d bias_raw) / scale; the -1e9 keys get exactly zero gradient
    check_bwd(f"S={S}", [to_np(q.grad), to_np(k.grad), to_np(v.grad), to_np(key_bias.grad)],
              [to_np(t) for t in (ex[0], ex[1], ex[2], ex[3] / scale)], [to_np(t) for t in fa[:3]] + [None],
              names=("dq", "dk", "dv", "dbias"))
    assert float(key_bias.grad[0, :, -64:].abs().max()) == 0.0


def test_config_bwd_8k_b4(cuda):
    """Training shape: B4, S8192, 16/8 heads, causal; bias [4, 8192] = log(sigmoid(z)), z~N(0,2),
    broadcast over heads with requires_grad; dO ~ N(0,1).  dBias summed over heads and queries."""
    from tokengate_amd.fa2bias.keybias import flash_attn_key_bias
    g = torch.Generator(device=cuda).manual_seed(4)
    B, S, H, Hkv = 4, 8192, 16, 8
    q, k, v = qkv(B, S, S, H, Hkv, g, cuda)
    kb = bias_logsigmoid((B, S), 2.0, g, cuda).requires_grad_(True)
    dO = torch.randn(B, S, H, 128, device=cuda, generator=g).to(torch.bfloat16)
    scale = 128 ** -0.5
    q, k, v = [t.requires_grad_(True) for t in (q, k, v)]
    out = flash_attn_key_bias(q, k, v, kb[:, None, :].expand(B, H, S), scale, causal=True)
    out.backward(dO)
    torch.cuda.synchronize()
    braw = (kb.detach()[:, None, :].expand(B, H, S) / scale).contiguous()
    _, lse = torch.ops.recursive_kvs.fa2_keybias_fwd(q.detach(), k.detach(), v.detach(), braw, scale, True)
    args = (dO, q.detach(), k.detach(), v.detach(), braw, scale, True)
    ex = ort.bwd(*args, chunk=2048, out=out.detach(), lse=lse)
    fa = ort.bwd(*args, chunk=2048, out=out.detach(), lse=lse, bf16_operands=True)
    check_bwd("8k b4", [to_np(q.grad), to_np(k.grad), to_np(v.grad), to_np(kb.grad)],
              [to_np(t) for t in (ex[0], ex[1], ex[2], ex[3].sum(1) / scale)], [to_np(t) for t in fa[:3]] + [None],
              names=("dq", "dk", "dv", "dbias (sum over heads)"))


def test_varlen_bwd_vs_oracle(cuda):
    g = torch.Generator(device=cuda).manual_seed(9)
    lens = [1, 100, 0, 257, 64]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    total, H, Hkv, D = int(cu[-1]), 16, 8, 128
    q = torch.randn(total, H, D, device=cuda, generator=g).to(torch.bfloat16)
    k = torch.randn(total, Hkv, D, device=cuda, generator=g).to(torch.bfloat16)
    v = torch.randn(total, Hkv, D, device=cuda, generator=g).to(torch.bfloat16)
    dout = torch.randn(total, H, D, device=cuda, generator=g).to(torch.bfloat16)
    maxlen = max(lens)
    scale = D ** -0.5
    bias_raw = (torch.randn(len(lens), H, maxlen, device=cuda, generator=g) / scale).contiguous()
    from tokengate_amd.fa2bias.keybias import ext
    cu_t = torch.tensor(cu, device=cuda)
    out, lse, _, _ = ext().varlen_fwd(q, k, v, None, cu_t, cu_t, None, None, None, bias_raw, maxlen, maxlen,
                                      0.0, scale, False, True, -1, -1, 0.0, False, None)
    dq, dk, dv, sd, db = ext().varlen_bwd(dout, q, k, v, out, lse, None, None, None, cu_t, cu_t, bias_raw,
                                          maxlen, maxlen, 0.0, scale, False, True, -1, -1, 0.0, False, None, None)
    torch.cuda.synchronize()
    qn, kn, vn, dn, bn, on, ln = to_np(q), to_np(k), to_np(v), to_np(dout), to_np(bias_raw), to_np(out), to_np(lse)
    for s, (st, n) in enumerate(ora.varlen_to_dense(cu)):
        if n == 0:
            continue
        a = (dn[None, st:st + n], qn[None, st:st + n], kn[None, st:st + n], vn[None, st:st + n],
             bn[s:s + 1, :, :n], scale, True)
        kw = dict(out=on[None, st:st + n], lse=ln[None, :, st:st + n])
        ex = ora.keybias_bwd(*a, **kw)
        fa = ora.keybias_bwd(*a, **kw, bf16_operands=True)
        got = [to_np(dq)[None, st:st + n], to_np(dk)[None, st:st + n], to_np(dv)[None, st:st + n],
               to_np(db)[s:s + 1, :, :n], to_np(sd)[None, :, st:st + n]]
        check_bwd(f"varlen seq {s}", got, ex, fa)
