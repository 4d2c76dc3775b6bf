"""tg_keybias_fwd_noalloc (the forward for callers that cannot allocate: its key-range split
writes into the library's static per-device scratch) against tg_keybias_fwd with the workspace the
library plans, through the C ABI: two calls in a row whose launches both split, the second with a
smaller input (so a stale first-call scratch would show), each bit-exact with the existing entry
point (itself checked against the oracle in tests/test_attn_split_gpu.py); then an unsplit launch
(no scratch used)."""
import pytest
import torch

from tokengate_amd import _lib

pytestmark = pytest.mark.gpu


def _args(q, k, v, bias_raw, out, lse):
    B, Sq, H, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    return (q.data_ptr(), k.data_ptr(), v.data_ptr(), bias_raw.data_ptr() if bias_raw is not None else None,
            out.data_ptr(), lse.data_ptr(), B, Sq, Sk, H, Hkv, D,
            q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1), k.stride(2),
            v.stride(0), v.stride(1), v.stride(2), out.stride(0), out.stride(1), out.stride(2),
            bias_raw.stride(0) if bias_raw is not None else 0, bias_raw.stride(1) if bias_raw is not None else 0)


def _inputs(B, Sq, Sk, H, Hkv, seed, dev, bias=True):
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(B, Sq, H, 128, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(B, Sk, Hkv, 128, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(B, Sk, Hkv, 128, generator=g, device=dev).to(torch.bfloat16)
    scale = 128 ** -0.5
    b = (torch.nn.functional.logsigmoid(torch.randn(B, H, Sk, generator=g, device=dev) * 2) / scale).contiguous() \
        if bias else None
    return q, k, v, b, scale


def _both(q, k, v, b, scale, causal):
    B, Sq, H, _ = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    stream = torch.cuda.current_stream().cuda_stream
    n = int(_lib.load().tg_keybias_fwd_workspace_size(B, Sq, Sk, H, Hkv, int(causal)))
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device=q.device)
    o1, o2 = torch.empty_like(q), torch.full_like(q, float("nan"))
    l1 = torch.empty(B, H, Sq, dtype=torch.float32, device=q.device)
    l2 = torch.full_like(l1, float("nan"))
    _lib.call("tg_keybias_fwd", *_args(q, k, v, b, o1, l1), float(scale), int(causal),
              ws.data_ptr() if n else None, n, stream)
    _lib.call("tg_keybias_fwd_noalloc", *_args(q, k, v, b, o2, l2), float(scale), int(causal), stream)
    torch.cuda.synchronize()
    return n, (o1, l1), (o2, l2)


def test_noalloc_matches_workspace_entry_point(cuda):
    # (B, Sq, Sk, H, Hkv, causal): a few rows over long caches, then one decode row over a shorter one
    for i, (B, Sq, Sk, H, Hkv, causal) in enumerate([(2, 3, 9000, 16, 8, True), (1, 1, 3000, 16, 8, True)]):
        print(f"[noalloc] call {i}: B{B} Sq{Sq} Sk{Sk} H{H}/{Hkv}", flush=True)
        q, k, v, b, scale = _inputs(B, Sq, Sk, H, Hkv, 40 + i, cuda)
        n, (o1, l1), (o2, l2) = _both(q, k, v, b, scale, causal)
        assert n > 0, "this launch is meant to use the key-range split (and so the scratch)"
        assert torch.equal(o1, o2) and torch.equal(l1, l2), f"call {i}: noalloc differs from tg_keybias_fwd"


def test_noalloc_unsplit_launch(cuda):
    q, k, v, b, scale = _inputs(1, 4096, 4096, 16, 8, 7, cuda, bias=False)
    n, (o1, l1), (o2, l2) = _both(q, k, v, None, scale, True)
    assert n == 0
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
