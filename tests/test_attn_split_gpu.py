"""GPU parity of the forward's key-range split, which the library plans for launches that leave
much of the GPU idle (Phase 2 at small K, a few rows or one decode row over a long cache).

Each case is run with the planned workspace (handed over full of 0xFF bytes, so any read of a
partial the kernel did not write shows up as NaN) and without one (no split), and both are
checked against the float64 oracle; a workspace smaller than planned must fall back to the
unsplit launch bit for bit.
"""
import numpy as np
import pytest
import torch

from oracle import attention as ora
from tests.attn_util import assert_close, qkv, to_np
from tokengate_amd import _lib

pytestmark = pytest.mark.gpu


def _dense(q, k, v, bias_raw, scale, causal, ws_mode="planned"):
    """tg_keybias_fwd with ws_mode 'planned' (the size the library asks for), 'none' or 'short'
    (one byte less than planned).  Returns out, lse and the planned workspace size."""
    B, Sq, H, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    out = torch.empty_like(q)
    lse = torch.empty(B, H, Sq, dtype=torch.float32, device=q.device)
    n = int(_lib.load().tg_keybias_fwd_workspace_size(B, Sq, Sk, H, Hkv, int(causal)))
    ws = None
    if ws_mode != "none" and n > 0:
        ws = torch.full((n if ws_mode == "planned" else n - 1,), 0xFF, dtype=torch.uint8, device=q.device)
    _lib.call("tg_keybias_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(),
              bias_raw.data_ptr() if bias_raw is not None else None, out.data_ptr(), lse.data_ptr(),
              B, Sq, Sk, H, Hkv, D, q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1), k.stride(2),
              v.stride(0), v.stride(1), v.stride(2), out.stride(0), out.stride(1), out.stride(2),
              bias_raw.stride(0) if bias_raw is not None else 0, bias_raw.stride(1) if bias_raw is not None else 0,
              float(scale), int(causal), ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out, lse, n


def _rows(Sq):
    if Sq <= 400:
        return None
    return np.unique(np.concatenate([np.arange(0, 70), np.linspace(0, Sq - 1, 120).astype(int), np.arange(Sq - 70, Sq)]))


CASES = [
    # B, Sq, Sk, H, Hkv, causal, bias
    (1, 2320, 2320, 16, 8, True, True),      # Phase 2 at K=2000
    (2, 1500, 1500, 6, 2, True, True),       # odd GQA group (one head per MFMA column block)
    (1, 2048, 2048, 16, 8, False, True),     # non-causal: every tile split
    (1, 700, 3000, 16, 8, True, False),      # Sq < Sk, no bias
    (1, 1, 20000, 16, 8, True, True),        # one decode row over a long cache
    (2, 3, 9000, 16, 8, True, True),         # a few rows per sequence
]


@pytest.mark.parametrize("B,Sq,Sk,H,Hkv,causal,has_bias", CASES,
                         ids=["2320", "odd_group", "noncausal", "sq_lt_sk", "decode_row", "few_rows"])
def test_split_matches_oracle_and_unsplit(cuda, B, Sq, Sk, H, Hkv, causal, has_bias):
    g = torch.Generator(device=cuda).manual_seed(Sq * 7 + Sk + H)
    q, k, v = qkv(B, Sq, Sk, H, Hkv, g, cuda)
    scale = 128 ** -0.5
    bias_raw = (torch.randn(B, H, Sk, device=cuda, generator=g) * 2.0 / scale).contiguous() if has_bias else None
    out_s, lse_s, n = _dense(q, k, v, bias_raw, scale, causal, "planned")
    assert n > 0, "this shape is expected to be split"
    out_u, lse_u, _ = _dense(q, k, v, bias_raw, scale, causal, "none")
    rows = _rows(Sq)
    ro, rl = ora.keybias_fwd(to_np(q), to_np(k), to_np(v), None if bias_raw is None else to_np(bias_raw),
                             scale, causal, rows=rows)
    sel = (lambda o, l: (to_np(o), to_np(l))) if rows is None else (lambda o, l: (to_np(o)[:, rows], to_np(l)[:, :, rows]))
    go, gl = sel(out_s, lse_s)
    assert_close("split out", go, ro)
    assert_close("split lse", gl, rl)
    uo, ul = sel(out_u, lse_u)
    assert_close("unsplit out", uo, ro)
    assert_close("unsplit lse", ul, rl)
    # split and unsplit agree everywhere (not only on the sampled rows)
    assert_close("split vs unsplit out", to_np(out_s), to_np(out_u))
    assert_close("split vs unsplit lse", to_np(lse_s), to_np(lse_u))


def test_short_workspace_runs_unsplit(cuda):
    g = torch.Generator(device=cuda).manual_seed(5)
    q, k, v = qkv(1, 2320, 2320, 16, 8, g, cuda)
    scale = 128 ** -0.5
    bias_raw = (torch.randn(1, 16, 2320, device=cuda, generator=g) / scale).contiguous()
    out_short, lse_short, n = _dense(q, k, v, bias_raw, scale, True, "short")
    out_none, lse_none, _ = _dense(q, k, v, bias_raw, scale, True, "none")
    assert n > 0
    assert torch.equal(out_short, out_none) and torch.equal(lse_short, lse_none)


@pytest.mark.parametrize("lens,causal,has_bias", [([2320], True, True), ([1000, 0, 600], True, True),
                                                  ([1000, 0, 600], False, True), ([700, 1500], True, False)],
                         ids=["phase2_K2000", "ragged3", "ragged3_noncausal", "two_nobias"])
def test_varlen_split(cuda, lens, causal, has_bias):
    """Varlen launches as Phase 2 makes them at small K: split through the fa2bias shim."""
    g = torch.Generator(device=cuda).manual_seed(sum(lens))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    total, H, Hkv, D = int(cu[-1]), 16, 8, 128
    maxlen = max(lens)
    assert _lib.load().tg_keybias_varlen_fwd_workspace_size(len(lens), maxlen, H, Hkv, int(causal)) > 0
    q = torch.randn(total, H, D, device=cuda, generator=g).to(torch.bfloat16)
    k = torch.randn(total, Hkv, D, device=cuda, generator=g).to(torch.bfloat16)
    v = torch.randn(total, Hkv, D, device=cuda, generator=g).to(torch.bfloat16)
    scale = D ** -0.5
    bias_raw = (torch.randn(len(lens), H, maxlen, device=cuda, generator=g) / scale).contiguous() if has_bias else None
    from tokengate_amd.fa2bias.keybias import ext
    cu_t = torch.tensor(cu, device=cuda)
    out, lse, _, _ = ext().varlen_fwd(q, k, v, None, cu_t, cu_t, None, None, None, bias_raw, maxlen, maxlen,
                                      0.0, scale, False, causal, -1, -1, 0.0, False, None)
    torch.cuda.synchronize()
    ro, rl = ora.keybias_varlen_fwd(to_np(q), to_np(k), to_np(v), None if bias_raw is None else to_np(bias_raw), cu,
                                    scale, causal)
    assert_close("varlen split out", to_np(out), ro)
    assert_close("varlen split lse", to_np(lse), rl)
