"""Oracle: key-bias causal GQA attention in float64 numpy (TEST INFRASTRUCTURE ONLY).

Restates the reference math of the FA2 key-bias kernels:
  * kernels/fa2bias/keybias.py:85-87 — bias_raw = key_bias / softmax_scale (raw-score units);
  * kernels/fa2bias/keybias.patch:404-416, 440-461 — the bias of key j is added to every row's
    raw score before the softmax scaling; keys j >= Sk masked;
  * FA2 causal mask (bottom-right aligned): key j visible to query i iff j <= i + Sk - Sq;
  * LSE in natural log; rows with no visible key give out = 0, lse = +inf;
  * kernels/fa2bias/keybias.patch:219-271 — backward: dS = P * (dO V^T - D), D = rowsum(dO * O),
    dQ = scale dS K, dK = scale dS^T Q, dV = P^T dO summed over the query heads of a KV head
    (keybias.patch:125 context), dbias_raw = scale * sum_i dS (keybias.patch:228-229, 267);
  * tests/attention/test_attention_backends_grad.py:8-18 — the reference's own fp32 oracle
    (repeat_interleave GQA, QK^T/sqrt(D) + bias, causal -inf, softmax, @V).

Inputs are numpy arrays holding the values the kernel sees (bf16-rounded by the caller).
"""
import numpy as np


def bf16_round(x):
    """Round float32/float64 values to bfloat16 (round to nearest even) and return float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = np.isnan(x)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = u.astype(np.uint32).view(np.float32)
    return np.where(nan, np.float32(np.nan), out)


def _logits(qb, kg, bias_row, scale, causal, q_rows, sq, sk):
    z = (qb[q_rows] @ kg.T)            # raw scores (len(q_rows), Sk)
    if bias_row is not None:
        z = z + bias_row[None, :]
    z = z * scale
    if causal:
        j = np.arange(sk)[None, :]
        i = np.asarray(q_rows)[:, None]
        z = np.where(j > i + (sk - sq), -np.inf, z)
    return z


def keybias_fwd(q, k, v, bias_raw, scale, causal=True, rows=None, dtype=np.float64):
    """Forward.  q (B,Sq,H,D), k/v (B,Sk,Hkv,D), bias_raw (B,H,Sk) or None.

    rows: optional index array of query rows to evaluate (all by default).
    dtype: evaluation precision (float64 for checking; float32 for the timed CPU baseline).
    Returns out (B,len(rows),H,D) and lse (B,H,len(rows)) in that precision."""
    B, Sq, H, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    G = H // Hkv
    rows = np.arange(Sq) if rows is None else np.asarray(rows)
    out = np.zeros((B, len(rows), H, D), dtype=dtype)
    lse = np.full((B, H, len(rows)), np.inf, dtype=dtype)
    for b in range(B):
        for h in range(H):
            g = h // G
            z = _logits(q[b, :, h].astype(dtype), k[b, :, g].astype(dtype),
                        None if bias_raw is None else bias_raw[b, h].astype(dtype),
                        dtype(scale), causal, rows, Sq, Sk)
            m = z.max(axis=1, initial=-np.inf)
            ok = np.isfinite(m)
            p = np.exp(z - np.where(ok, m, 0.0)[:, None])
            l = p.sum(axis=1)
            o = (p @ v[b, :, g].astype(dtype)) / np.where(l > 0, l, 1.0)[:, None]
            out[b, :, h] = np.where(ok[:, None], o, 0.0)
            lse[b, h] = np.where(ok, m + np.log(np.where(l > 0, l, 1.0)), np.inf)
    return out, lse


def keybias_bwd(dout, q, k, v, bias_raw, scale, causal=True, out=None, bf16_operands=False, lse=None):
    """Backward of keybias_fwd.  Returns dq, dk, dv (input shapes), dbias_raw (B,H,Sk) — the
    gradient with respect to bias_raw, i.e. scale * sum_i dS — and softmax_d (B,H,Sq).

    out: the forward output handed to the backward (B,Sq,H,D), as the reference's op receives
    it (keybias.py:52-63, 66-82: the saved bf16 `out`); D = rowsum(dO * out) then uses it, as
    FA2's backward does.  Default: the oracle's own float64 forward output.
    lse: the forward's log-sum-exp handed to the backward (B,H,Sq), likewise an input of the
    reference's op; P = exp(z - lse) then uses it.  Default: the oracle's own.
    bf16_operands: round P and dS to bf16 before the products that consume them (dV = P^T dO;
    dK, dQ from dS), the FlashAttention-2 backward's operand precision (flash-attn 2.8.3
    flash_bwd_kernel.h, not vendored: the patch context keybias.patch:243-248 forms dS in fp32
    just before that conversion); dBias and D stay in full precision (keybias.patch:246)."""
    B, Sq, H, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    G = H // Hkv
    o_fwd, lse_fwd = keybias_fwd(q, k, v, bias_raw, scale, causal)
    o_d = o_fwd if out is None else np.asarray(out, dtype=np.float64)
    lse = lse_fwd if lse is None else np.asarray(lse, dtype=np.float64)
    rnd = (lambda x: bf16_round(x).astype(np.float64)) if bf16_operands else (lambda x: x)
    dq = np.zeros(q.shape)
    dk = np.zeros(k.shape)
    dv = np.zeros(v.shape)
    dbias = np.zeros((B, H, Sk))
    sd = np.zeros((B, H, Sq))
    rows = np.arange(Sq)
    for b in range(B):
        for h in range(H):
            g = h // G
            qb = q[b, :, h].astype(np.float64)
            kg = k[b, :, g].astype(np.float64)
            vg = v[b, :, g].astype(np.float64)
            do = dout[b, :, h].astype(np.float64)
            z = _logits(qb, kg, None if bias_raw is None else bias_raw[b, h].astype(np.float64),
                        scale, causal, rows, Sq, Sk)
            fin = np.isfinite(lse[b, h])
            p = np.exp(z - np.where(fin, lse[b, h], 0.0)[:, None])
            p[~fin] = 0.0
            Dv = (do * o_d[b, :, h]).sum(axis=1)
            sd[b, h] = Dv
            dp = do @ vg.T
            ds = p * (dp - Dv[:, None])
            dq[b, :, h] = scale * rnd(ds) @ kg
            dk[b, :, g] += scale * rnd(ds).T @ qb
            dv[b, :, g] += rnd(p).T @ do
            dbias[b, h] = scale * ds.sum(axis=0)
    return dq, dk, dv, dbias, sd


def varlen_to_dense(cu_seqlens):
    """[(start, length)] of each packed sequence."""
    cu = np.asarray(cu_seqlens)
    return [(int(cu[i]), int(cu[i + 1] - cu[i])) for i in range(len(cu) - 1)]


def keybias_varlen_fwd(q, k, v, bias_raw, cu_seqlens, scale, causal=True):
    """Varlen forward: q (total,H,D), k/v (total,Hkv,D), bias_raw (nseq,H,max_seqlen) indexed by
    each key's position inside its own sequence (kernels/fa2bias/build.py:54-57).
    Returns out (total,H,D) and lse (H,total)."""
    total, H, D = q.shape
    out = np.zeros((total, H, D))
    lse = np.full((H, total), np.inf)
    for s, (st, n) in enumerate(varlen_to_dense(cu_seqlens)):
        if n == 0:
            continue
        br = None if bias_raw is None else bias_raw[s:s + 1, :, :n]
        o, l = keybias_fwd(q[None, st:st + n], k[None, st:st + n], v[None, st:st + n], br, scale, causal)
        out[st:st + n] = o[0]
        lse[:, st:st + n] = l[0]
    return out, lse


def causal_flops(batch, heads, seqlen, head_dim=128):
    """Algorithmic FLOPs of the causal forward: 4*D per visible (query, key) pair,
    S(S+1)/2 pairs per (batch, head)."""
    return 2.0 * batch * heads * head_dim * seqlen * (seqlen + 1)
