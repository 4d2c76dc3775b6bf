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
    # then grids of more than half the resident slots (a few thousand rows over a long cache, and a
    # non-causal one), whose split plans once needed more than the static scratch
    shapes = [(2, 3, 9000, 16, 8, True), (1, 1, 3000, 16, 8, True), (1, 3072, 32768, 16, 8, True),
              (1, 3000, 32768, 16, 8, True), (1, 3072, 4096, 16, 8, False)]
    for i, (B, Sq, Sk, H, Hkv, causal) in enumerate(shapes):
        print(f"[noalloc] call {i}: B{B} Sq{Sq} Sk{Sk} H{H}/{Hkv}", flush=True)
        q, k, v, b, scale = _inputs(B, Sq, Sk, H, Hkv, 40 + i, cuda)
        n, (o1, l1), (o2, l2) = _both(q, k, v, b, scale, causal)
        assert n > 0, "this launch is meant to use the key-range split (and so the scratch)"
        assert torch.equal(o1, o2) and torch.equal(l1, l2), f"call {i}: noalloc differs from tg_keybias_fwd"


_CAPTURE_SCRIPT = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
import tests.test_zz_no_alloc as T
from tokengate_amd import _lib
dev = torch.device("cuda:0")
B, Sq, Sk, H, Hkv = 1, 5, 9000, 16, 8
q, k, v, b, scale = T._inputs(B, Sq, Sk, H, Hkv, 90, dev)
o = torch.empty_like(q)
l = torch.empty(B, H, Sq, dtype=torch.float32, device=dev)
stream = torch.cuda.Stream()
g = torch.cuda.CUDAGraph()
torch.cuda.synchronize()
# the first tg_keybias_fwd_noalloc call of this process (its scratch lookup) happens under capture
with torch.cuda.graph(g, stream=stream):
    _lib.call("tg_keybias_fwd_noalloc", *T._args(q, k, v, b, o, l), float(scale), 1,
              torch.cuda.current_stream().cuda_stream)
for rep in range(3):
    q2, k2, v2, b2, _ = T._inputs(B, Sq, Sk, H, Hkv, 91 + rep, dev)
    q.copy_(q2); k.copy_(k2); v.copy_(v2); b.copy_(b2)
    g.replay()
    torch.cuda.synchronize()
    n, (o1, l1), _ = T._both(q, k, v, b, scale, True)
    assert n > 0
    ok = torch.equal(o, o1) and torch.equal(l, l1)
    print(f"replay {rep}: bit-exact {ok}", flush=True)
    assert ok, f"replay {rep} differs from tg_keybias_fwd"
print("capture ok", flush=True)
"""


def test_noalloc_first_call_under_graph_capture(cuda):
    """In a fresh process, the first noalloc call (which looks up the device scratch) is made under
    HIP graph capture; three replays over new inputs each equal tg_keybias_fwd bit for bit."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-u", "-c", _CAPTURE_SCRIPT, root], capture_output=True, text=True,
                       timeout=300, cwd=root)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0 and "capture ok" in r.stdout


def test_noalloc_unsplit_launch(cuda):
    q, k, v, b, scale = _inputs(1, 4096, 4096, 16, 8, 7, cuda, bias=False)
    n, (o1, l1), (o2, l2) = _both(q, k, v, None, scale, True)
    assert n == 0
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
