"""GPU parity of the key-bias attention backward (dQ, dK, dV, dBias, softmax_d).

Small shapes against the float64 numpy oracle; the reference's own GPU-test shapes
(tests/attention/test_attention_backends_grad.py:21-31,65: S in {1024, 4096, 4093}, H16/Hkv8,
inputs randn*0.5, bias randn*2 with the last 64 keys at -1e9) and the B4 x 8192 training shape
against the float32 torch evaluation of the same math on the device.  Tolerance: max-abs
<= 2e-2 relative to max(1, max|ref|) and rel-L2 <= 1e-2 (tests/attn_util.assert_close_grad).
"""
import numpy as np
import pytest
import torch

from oracle import attention as ora
from oracle import attention_torch as ort
from tests.attn_util import assert_close_grad as assert_close, bias_logsigmoid, qkv, to_np

pytestmark = pytest.mark.gpu


def _fwd_bwd(q, k, v, bias_raw, dout, scale, causal):
    from tokengate_amd.fa2bias.keybias import ext
    out, lse, _, _ = ext().fwd(q, k, v, None, bias_raw, 0.0, scale, causal, -1, -1, 0.0, False, None)
    dq, dk, dv, sd, db = ext().bwd(dout, q, k, v, out, lse, None, None, None, bias_raw, 0.0, scale, causal,
                                   -1, -1, 0.0, False, None, None)
    torch.cuda.synchronize()
    return dq, dk, dv, db, sd


@pytest.mark.parametrize("S", [1, 33, 64, 100, 257])
@pytest.mark.parametrize("H,Hkv", [(16, 8), (4, 4), (6, 2), (8, 2)])
@pytest.mark.parametrize("causal", [True, False])
def test_bwd_small_vs_oracle(cuda, S, H, Hkv, causal):
    g = torch.Generator(device=cuda).manual_seed(S * 7 + H + (1 if causal else 0))
    q, k, v = qkv(2, S, S, H, Hkv, g, cuda)
    scale = 128 ** -0.5
    bias_raw = (torch.randn(2, H, S, device=cuda, generator=g) * 2.0 / scale).contiguous()
    dout = torch.randn(2, S, H, 128, device=cuda, generator=g).to(torch.bfloat16)
    dq, dk, dv, db, sd = _fwd_bwd(q, k, v, bias_raw, dout, scale, causal)
    r = ora.keybias_bwd(to_np(dout), to_np(q), to_np(k), to_np(v), to_np(bias_raw), scale, causal)
    for name, got, ref in zip(["dq", "dk", "dv", "dbias_raw", "softmax_d"], [dq, dk, dv, db, sd], r):
        assert_close(f"{name} S={S} H={H}/{Hkv} causal={causal}", to_np(got), ref)


@pytest.mark.parametrize("Sq,Sk", [(100, 300), (300, 100), (129, 128)])
def test_bwd_unequal_lengths(cuda, Sq, Sk):
    g = torch.Generator(device=cuda).manual_seed(Sq * 3 + Sk)
    H, Hkv = 16, 8
    q, k, v = qkv(1, Sq, Sk, H, Hkv, g, cuda)
    scale = 128 ** -0.5
    bias_raw = (torch.randn(1, H, Sk, device=cuda, generator=g) / scale).contiguous()
    dout = torch.randn(1, Sq, H, 128, device=cuda, generator=g).to(torch.bfloat16)
    for causal in (True, False):
        dq, dk, dv, db, sd = _fwd_bwd(q, k, v, bias_raw, dout, scale, causal)
        r = ora.keybias_bwd(to_np(dout), to_np(q), to_np(k), to_np(v), to_np(bias_raw), scale, causal)
        for name, got, ref in zip(["dq", "dk", "dv", "dbias_raw", "softmax_d"], [dq, dk, dv, db, sd], r):
            assert_close(f"{name} Sq={Sq} Sk={Sk} causal={causal}", to_np(got), ref)


def test_bwd_no_bias(cuda):
    g = torch.Generator(device=cuda).manual_seed(5)
    q, k, v = qkv(1, 200, 200, 16, 8, g, cuda)
    scale = 128 ** -0.5
    dout = torch.randn(1, 200, 16, 128, device=cuda, generator=g).to(torch.bfloat16)
    dq, dk, dv, db, sd = _fwd_bwd(q, k, v, None, dout, scale, True)
    assert db is None
    r = ora.keybias_bwd(to_np(dout), to_np(q), to_np(k), to_np(v), None, scale, True)
    for name, got, ref in zip(["dq", "dk", "dv"], [dq, dk, dv], r[:3]):
        assert_close(f"{name} no-bias", to_np(got), ref)


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
    rdq, rdk, rdv, rdb, _ = ort.bwd(dO.transpose(1, 2), q.detach(), k.detach(), v.detach(),
                                    key_bias.detach().float() / scale, scale, True)
    assert_close(f"dq S={S}", to_np(q.grad), to_np(rdq))
    assert_close(f"dk S={S}", to_np(k.grad), to_np(rdk))
    assert_close(f"dv S={S}", to_np(v.grad), to_np(rdv))
    # d/d key_bias = (d/d bias_raw) / scale; the -1e9 keys get exactly zero gradient
    assert_close(f"dbias S={S}", to_np(key_bias.grad), to_np(rdb / scale))
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
    rdq, rdk, rdv, rdb, _ = ort.bwd(dO, q.detach(), k.detach(), v.detach(),
                                    (kb.detach()[:, None, :].expand(B, H, S) / scale).contiguous(), scale, True,
                                    chunk=2048)
    assert_close("dq 8k", to_np(q.grad), to_np(rdq))
    assert_close("dk 8k", to_np(k.grad), to_np(rdk))
    assert_close("dv 8k", to_np(v.grad), to_np(rdv))
    assert_close("dbias 8k (sum over heads)", to_np(kb.grad), to_np(rdb.sum(1) / scale))


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
    qn, kn, vn, dn, bn = to_np(q), to_np(k), to_np(v), to_np(dout), to_np(bias_raw)
    for s, (st, n) in enumerate(ora.varlen_to_dense(cu)):
        if n == 0:
            continue
        r = ora.keybias_bwd(dn[None, st:st + n], qn[None, st:st + n], kn[None, st:st + n], vn[None, st:st + n],
                            bn[s:s + 1, :, :n], scale, True)
        assert_close(f"varlen dq seq {s}", to_np(dq)[st:st + n], r[0][0])
        assert_close(f"varlen dk seq {s}", to_np(dk)[st:st + n], r[1][0])
        assert_close(f"varlen dv seq {s}", to_np(dv)[st:st + n], r[2][0])
        assert_close(f"varlen dbias seq {s}", to_np(db)[s, :, :n], r[3][0])
        assert_close(f"varlen softmax_d seq {s}", to_np(sd)[:, st:st + n], r[4][0])
