"""Oracle: the key-bias attention math of oracle/attention.py evaluated in float32 torch, chunked
over query rows (TEST INFRASTRUCTURE ONLY).

Used by the GPU tests for full-size shapes (e.g. B=4, S=8192) where the float64 numpy oracle
is too slow; it runs on whatever device its inputs live on.  Pinned against the numpy oracle by
tests/test_oracle_attention.py::test_torch_oracle_matches_numpy.  Same conventions: q (B,Sq,H,D),
k/v (B,Sk,Hkv,D), bias_raw (B,H,Sk) in raw-score units or None, bottom-right causal alignment,
natural-log LSE, rows with no visible key -> out 0 / lse +inf; the backward returns the
gradient with respect to bias_raw (scale * sum_i dS) as in kernels/fa2bias/keybias.patch:267.
"""
import torch


def _logits(qh, kg, brow, scale, causal, i0, i1, sq, sk, q_pos=None):
    z = qh[i0:i1] @ kg.t()
    if brow is not None:
        z = z + brow[None, :]
    z = z * scale
    if causal:
        j = torch.arange(sk, device=z.device)[None, :]
        if q_pos is None:
            i = torch.arange(i0, i1, device=z.device)[:, None]
            z = z.masked_fill(j > i + (sk - sq), float("-inf"))
        else:
            z = z.masked_fill(j > q_pos[i0:i1, None], float("-inf"))
    return z


def fwd(q, k, v, bias_raw, scale, causal=True, chunk=1024, q_pos=None):
    """q_pos (Sq,) int64, optional: q holds only these rows of a self-attention over the Sk keys
    (row q_pos[i] sees keys j <= q_pos[i]) -- sampled rows of a long sequence."""
    B, Sq, H, D = q.shape
    if q_pos is not None:
        q_pos = torch.as_tensor(q_pos, dtype=torch.int64, device=q.device)
    Sk, Hkv = k.shape[1], k.shape[2]
    G = H // Hkv
    out = torch.zeros(B, Sq, H, D, dtype=torch.float32, device=q.device)
    lse = torch.full((B, H, Sq), float("inf"), dtype=torch.float32, device=q.device)
    for b in range(B):
        for h in range(H):
            g = h // G
            qh = q[b, :, h].float().contiguous()
            kg = k[b, :, g].float().contiguous()
            vg = v[b, :, g].float().contiguous()
            brow = None if bias_raw is None else bias_raw[b, h].float()
            for i0 in range(0, Sq, chunk):
                i1 = min(Sq, i0 + chunk)
                z = _logits(qh, kg, brow, scale, causal, i0, i1, Sq, Sk, q_pos)
                m = z.amax(dim=1)
                ok = torch.isfinite(m)
                p = torch.exp(z - torch.where(ok, m, torch.zeros_like(m))[:, None])
                l = p.sum(1)
                o = (p @ vg) / torch.where(l > 0, l, torch.ones_like(l))[:, None]
                out[b, i0:i1, h] = torch.where(ok[:, None], o, torch.zeros_like(o))
                lse[b, h, i0:i1] = torch.where(ok, m + torch.log(torch.where(l > 0, l, torch.ones_like(l))),
                                               torch.full_like(m, float("inf")))
    return out, lse


def bwd(dout, q, k, v, bias_raw, scale, causal=True, chunk=1024, out=None, bf16_operands=False, lse=None):
    """Returns dq, dk, dv (float32, input shapes), dbias_raw (B,H,Sk) or None, softmax_d (B,H,Sq).
    out / lse / bf16_operands as in oracle.attention.keybias_bwd: D and P from the forward output
    and log-sum-exp handed to the backward, P and dS rounded to bf16 before the products that
    consume them."""
    B, Sq, H, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    G = H // Hkv
    o_fwd, lse_fwd = fwd(q, k, v, bias_raw, scale, causal, chunk)
    out = o_fwd if out is None else out.float()
    lse = lse_fwd if lse is None else lse.float()
    rnd = (lambda x: x.to(torch.bfloat16).float()) if bf16_operands else (lambda x: x)
    dq = torch.zeros(B, Sq, H, D, dtype=torch.float32, device=q.device)
    dk = torch.zeros(B, Sk, Hkv, D, dtype=torch.float32, device=q.device)
    dv = torch.zeros(B, Sk, Hkv, D, dtype=torch.float32, device=q.device)
    dbias = None if bias_raw is None else torch.zeros(B, H, Sk, dtype=torch.float32, device=q.device)
    sd = (dout.float() * out).sum(-1).permute(0, 2, 1).contiguous()
    for b in range(B):
        for h in range(H):
            g = h // G
            qh = q[b, :, h].float().contiguous()
            kg = k[b, :, g].float().contiguous()
            vg = v[b, :, g].float().contiguous()
            do = dout[b, :, h].float().contiguous()
            brow = None if bias_raw is None else bias_raw[b, h].float()
            for i0 in range(0, Sq, chunk):
                i1 = min(Sq, i0 + chunk)
                z = _logits(qh, kg, brow, scale, causal, i0, i1, Sq, Sk)
                l = lse[b, h, i0:i1]
                fin = torch.isfinite(l)
                p = torch.exp(z - torch.where(fin, l, torch.zeros_like(l))[:, None])
                p = torch.where(fin[:, None], p, torch.zeros_like(p))
                dp = do[i0:i1] @ vg.t()
                ds = p * (dp - sd[b, h, i0:i1][:, None])
                dsr = rnd(ds)
                dq[b, i0:i1, h] = scale * (dsr @ kg)
                dk[b, :, g] += scale * (dsr.t().contiguous() @ qh[i0:i1])
                dv[b, :, g] += rnd(p).t().contiguous() @ do[i0:i1]
                if dbias is not None:
                    dbias[b, h] += scale * ds.sum(0)
    return dq, dk, dv, dbias, sd
