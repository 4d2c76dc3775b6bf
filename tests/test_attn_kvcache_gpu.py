"""GPU parity of tg_keybias_varlen_kv_fwd: varlen attention whose keys sit in a cache with free
rows after every sequence (the gated prefill's decode headroom and the decode step's one launch
per layer).

The free rows of K / V and the bias columns past each sequence's keys are filled with NaN, so a
read of anything outside a sequence's used key rows shows up in the output.  Each case is checked
against the float64 oracle per sequence (bottom-right causal alignment), and the prefill-shaped
case (queries = keys) bit for bit against tg_keybias_varlen_fwd on the same rows packed back to
back: the same tiles over the same keys must give the same bits.
"""
import numpy as np
import pytest
import torch

from oracle import attention as ora
from tests.attn_util import assert_close, to_np
from tokengate_amd import _lib
from tokengate_amd import decoder as dec

pytestmark = pytest.mark.gpu

H, HKV, D = 16, 8, 128


def _cache(lens_k, gap, gen, dev):
    """K / V caches with `gap` NaN rows after each sequence's lens_k[b] rows; returns k, v, the
    segment starts and the packed (gap-free) copies."""
    B = len(lens_k)
    seg = [sum(lens_k[:b]) + b * gap for b in range(B)]
    rows = sum(lens_k) + B * gap
    k = torch.full((rows, HKV, D), float("nan"), device=dev).to(torch.bfloat16)
    v = torch.full((rows, HKV, D), float("nan"), device=dev).to(torch.bfloat16)
    kp = torch.randn(sum(lens_k), HKV, D, generator=gen, device=dev).to(torch.bfloat16)
    vp = torch.randn(sum(lens_k), HKV, D, generator=gen, device=dev).to(torch.bfloat16)
    o = 0
    for b, n in enumerate(lens_k):
        k[seg[b]:seg[b] + n] = kp[o:o + n]
        v[seg[b]:seg[b] + n] = vp[o:o + n]
        o += n
    return k, v, seg, kp, vp


def _run(q, k, v, bias, cu_q, seg, used, max_q, max_k, scale):
    dev = q.device
    cuq = torch.tensor(cu_q, dtype=torch.int32, device=dev)
    segd = torch.tensor(seg, dtype=torch.int32, device=dev)
    usedd = torch.tensor(used, dtype=torch.int32, device=dev)
    out = torch.full_like(q, float("nan"))
    lse = torch.full((H, q.shape[0]), float("nan"), dtype=torch.float32, device=dev)
    dec.varlen_kv_attention(q, k, v, cuq, segd, usedd, max_q, max_k, scale, bias, out=out, lse=lse)
    torch.cuda.synchronize()
    return out, lse


def _oracle_check(tag, q, kp, vp, bias, cu_q, lens_k, scale, out, lse):
    offk = np.concatenate([[0], np.cumsum(lens_k)])
    for b in range(len(lens_k)):
        q0, q1 = cu_q[b], cu_q[b + 1]
        if q1 == q0:
            continue
        qb = to_np(q[q0:q1])[None]
        kb = to_np(kp[offk[b]:offk[b + 1]])[None]
        vb = to_np(vp[offk[b]:offk[b + 1]])[None]
        bb = None if bias is None else to_np(bias[b, :, :lens_k[b]])[None]
        ro, rl = ora.keybias_fwd(qb, kb, vb, bb, scale, True)
        ma, rel = assert_close(f"{tag} seq {b} out", to_np(out[q0:q1]), ro[0])
        assert_close(f"{tag} seq {b} lse", to_np(lse[:, q0:q1]), rl[0])
        print(f"[kv-cache fwd] {tag} seq {b} (q {q1 - q0}, k {lens_k[b]}): max-abs {ma:.2e} rel-L2 {rel:.2e}",
              flush=True)


@pytest.mark.parametrize("lens,gap,has_bias", [([1000, 1, 600], 37, True), ([2320], 16, True),
                                               ([700, 1500, 64], 5, False)],
                         ids=["ragged3", "phase2_K2000", "nobias"])
def test_prefill_shape_matches_packed_and_oracle(cuda, lens, gap, has_bias):
    g = torch.Generator(device=cuda).manual_seed(sum(lens) + gap)
    k, v, seg, kp, vp = _cache(lens, gap, g, cuda)
    cu = [0] + list(np.cumsum(lens))
    T, maxlen = cu[-1], max(lens)
    q = torch.randn(T, H, D, generator=g, device=cuda).to(torch.bfloat16)
    scale = D ** -0.5
    bias = None
    if has_bias:
        bias = torch.full((len(lens), H, maxlen + gap), float("nan"), device=cuda)
        for b, n in enumerate(lens):
            bias[b, :, :n] = torch.randn(H, n, generator=g, device=cuda) / scale
    out, lse = _run(q, k, v, bias, cu, seg, lens, maxlen, maxlen, scale)
    # the same rows packed back to back through the self-attention entry point
    outp = torch.empty_like(q)
    lsep = torch.empty(H, T, dtype=torch.float32, device=cuda)
    dec.varlen_attention(q, kp, vp, torch.tensor(cu, dtype=torch.int32, device=cuda), maxlen, scale,
                         bias, out=outp, lse=lsep)
    torch.cuda.synchronize()
    assert torch.equal(out, outp) and torch.equal(lse, lsep), "cache layout changed the result bits"
    _oracle_check("prefill", q, kp, vp, bias, cu, lens, scale, out, lse)


@pytest.mark.parametrize("lens_k,nq,gap", [([5000, 1, 20000], 1, 9), ([300, 2048], 3, 4), ([130000], 1, 2),
                                           ([1, 2, 3, 70, 64, 65, 4000, 9], 1, 1)],
                         ids=["decode3", "few_rows", "decode_128k", "decode8_short"])
def test_decode_shape_matches_oracle(cuda, lens_k, nq, gap):
    """nq query rows per sequence over its used keys (decode: nq = 1); bias on every key, NaN past
    the used keys; max_seqlen_k above the longest (a cache's capacity)."""
    g = torch.Generator(device=cuda).manual_seed(len(lens_k) * 7 + nq)
    k, v, seg, kp, vp = _cache(lens_k, gap, g, cuda)
    B = len(lens_k)
    nqs = [min(nq, n) for n in lens_k]
    cu_q = [0] + list(np.cumsum(nqs))
    q = torch.randn(cu_q[-1], H, D, generator=g, device=cuda).to(torch.bfloat16)
    scale = D ** -0.5
    cap = max(lens_k) + gap
    bias = torch.full((B, H, cap), float("nan"), device=cuda)
    for b, n in enumerate(lens_k):
        bias[b, :, :n] = torch.nn.functional.logsigmoid(torch.randn(H, n, generator=g, device=cuda) * 3) / scale
    out, lse = _run(q, k, v, bias, cu_q, seg, lens_k, max(nqs), cap, scale)
    _oracle_check("decode", q, kp, vp, bias, cu_q, lens_k, scale, out, lse)


def test_kv_entry_errors(cuda):
    q = torch.zeros(4, H, D, dtype=torch.bfloat16, device=cuda)
    k = torch.zeros(8, HKV, D, dtype=torch.bfloat16, device=cuda)
    cu = torch.tensor([0, 4], dtype=torch.int32, device=cuda)
    out = torch.empty_like(q)
    lse = torch.empty(H, 4, dtype=torch.float32, device=cuda)
    with pytest.raises(RuntimeError, match="cu_seqlens_k is null"):
        _lib.call("tg_keybias_varlen_kv_fwd", q.data_ptr(), k.data_ptr(), k.data_ptr(), None, out.data_ptr(),
                  lse.data_ptr(), cu.data_ptr(), None, None, 1, 4, 4, 4, H, HKV, D,
                  q.stride(0), q.stride(1), k.stride(0), k.stride(1), k.stride(0), k.stride(1),
                  out.stride(0), out.stride(1), 0, 0, 0.1, 1, None, 0, torch.cuda.current_stream().cuda_stream)
