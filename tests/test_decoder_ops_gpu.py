"""GPU parity of the decoder ops of the gated prefill against float32 torch evaluations of the same
math (the oracle's Qwen3 layer pieces, pinned against transformers by test_oracle_prefill.py):
residual add + RMSNorm, per-head q/k RMSNorm + RoPE (positions up to 2^17, per-head and per-row
query scales, k/v cache writes), SiLU(gate) * up.  Bound: max-abs <= 2e-2 relative to max(1, |ref|) and
rel-L2 <= 1e-2 (one bf16 rounding of the output)."""
import math

import pytest
import torch

from oracle import prefill as op
from tests.attn_util import assert_close_grad, to_np

pytestmark = pytest.mark.gpu


def _bf(t):
    return t.to(torch.bfloat16)


@pytest.mark.parametrize("rows,d,with_res", [(1, 2048, False), (777, 2048, True), (64, 1024, True),
                                             (5, 4096, False), (33, 2560, True)])
def test_rmsnorm(cuda, rows, d, with_res):
    from tokengate_amd import decoder as dec
    g = torch.Generator(device=cuda).manual_seed(rows + d)
    x = _bf(torch.randn(rows, d, generator=g, device=cuda) * 3)
    w = _bf(1 + 0.3 * torch.randn(d, generator=g, device=cuda))
    res = _bf(torch.randn(rows, d, generator=g, device=cuda)) if with_res else None
    res_out = torch.empty_like(x) if with_res else None
    out = dec.rmsnorm(x, w, 1e-6, residual=res, residual_out=res_out)
    torch.cuda.synchronize()
    s = x.float() + res.float() if with_res else x.float()
    if with_res:
        assert torch.equal(res_out, _bf(s))                     # the bf16 residual stream, bit-exact
        s = _bf(s).float()
    ref = op.rms(s, w.float(), 1e-6)
    assert_close_grad("rmsnorm", to_np(out), to_np(ref))


def test_rmsnorm_in_place_residual(cuda):
    from tokengate_amd import decoder as dec
    g = torch.Generator(device=cuda).manual_seed(3)
    x = _bf(torch.randn(100, 2048, generator=g, device=cuda))
    res = _bf(torch.randn(100, 2048, generator=g, device=cuda))
    w = _bf(torch.ones(2048, device=cuda))
    want_res = _bf(x.float() + res.float())
    ref = op.rms(want_res.float(), w.float(), 1e-6)
    out = dec.rmsnorm(x, w, 1e-6, residual=res, residual_out=res, out=x)   # both aliased
    torch.cuda.synchronize()
    assert torch.equal(res, want_res)
    assert_close_grad("rmsnorm aliased", to_np(out), to_np(ref))


@pytest.mark.parametrize("T,H,Hkv,maxpos,scaled", [(1, 16, 8, 1, False), (333, 16, 8, 4096, True),
                                                    (257, 4, 1, 1 << 17, True), (64, 12, 4, 40000, False)])
def test_qk_norm_rope(cuda, T, H, Hkv, maxpos, scaled):
    from tokengate_amd import decoder as dec
    g = torch.Generator(device=cuda).manual_seed(T * 31 + H)
    D = 128
    shape = dec.DecoderShape(n_layers=1, n_heads=H, n_kv_heads=Hkv, d_model=H * D)
    width = (H + 2 * Hkv) * D
    qkv = _bf(torch.randn(T, width, generator=g, device=cuda) * 2)
    qkv0 = qkv.clone()
    pos = torch.randint(0, maxpos, (T,), generator=g, device=cuda)
    lw = dec.LayerWeights(None, None, _bf(1 + 0.3 * torch.randn(D, generator=g, device=cuda)),
                          _bf(1 + 0.3 * torch.randn(D, generator=g, device=cuda)), None, None, None, None)
    inv = dec.rope_inv_freq(shape, cuda)
    qs = (0.5 + torch.rand(H, generator=g, device=cuda)) if scaled else None
    rs = torch.rand(T, generator=g, device=cuda) if scaled else None      # per-row (scaled-softmax r)
    k = torch.empty(T, Hkv, D, dtype=torch.bfloat16, device=cuda)
    v = torch.empty_like(k)
    q = dec.qk_norm_rope(qkv, pos, lw, shape, inv, k, v, qs, rs)
    torch.cuda.synchronize()
    x = qkv0.float()
    qr = op.rms(x[:, :H * D].view(T, H, D), lw.q_norm.float(), 1e-6)
    kr = op.rms(x[:, H * D:(H + Hkv) * D].view(T, Hkv, D), lw.k_norm.float(), 1e-6)
    cos, sin = op.rope_cos_sin(pos.cpu(), inv.cpu())
    cos, sin = cos.to(cuda)[:, None, :], sin.to(cuda)[:, None, :]
    qr = qr * cos + op.rotate_half(qr) * sin
    kr = kr * cos + op.rotate_half(kr) * sin
    if qs is not None:
        qr = qr * qs[None, :, None] * rs[:, None, None]
    assert_close_grad("q", to_np(q), to_np(qr))
    assert_close_grad("k", to_np(k), to_np(kr))
    assert torch.equal(v.view(T, -1), qkv0[:, (H + Hkv) * D:])
    assert torch.equal(qkv[:, H * D:], qkv0[:, H * D:])          # k/v columns untouched
    assert q.data_ptr() == qkv.data_ptr()                         # q rotated in place
    # k / v rows written to a cache through a row map (rows t -> 3t + 1 of a larger cache)
    rows = torch.arange(T, dtype=torch.int32, device=cuda) * 3 + 1
    kc = torch.zeros(3 * T + 2, Hkv, D, dtype=torch.bfloat16, device=cuda)
    vc = torch.zeros_like(kc)
    qkv2 = qkv0.clone()
    q2 = dec.qk_norm_rope(qkv2, pos, lw, shape, inv, kc, vc, qs, rs, kv_rows=rows)
    torch.cuda.synchronize()
    assert torch.equal(q2, q)
    ri = rows.long()
    assert torch.equal(kc.index_select(0, ri), k) and torch.equal(vc.index_select(0, ri), v)
    others = torch.ones(3 * T + 2, dtype=torch.bool, device=cuda)
    others[ri] = False
    assert bool((kc[others] == 0).all()) and bool((vc[others] == 0).all())


@pytest.mark.parametrize("rows,inter", [(1, 8), (1000, 6144), (37, 1000)])
def test_silu_mul(cuda, rows, inter):
    from tokengate_amd import decoder as dec
    g = torch.Generator(device=cuda).manual_seed(rows + inter)
    gu = _bf(torch.randn(rows, 2 * inter, generator=g, device=cuda) * 3)
    out = dec.silu_mul(gu)
    torch.cuda.synchronize()
    f = gu.float()
    ref = torch.nn.functional.silu(f[:, :inter]) * f[:, inter:]
    assert_close_grad("silu_mul", to_np(out), to_np(ref))


@pytest.mark.parametrize("rows,inter", [(1, 8), (777, 6144), (130, 1000)])
def test_branch_readout(cuda, rows, inter):
    """The scoring branch's readout against torch's own bf16 evaluation of the absorbed branch
    (F.silu and the product in bf16, as an eager bf16 Qwen3MLP computes them; the (1, I) down row
    as an fp32-accumulated dot rounded to bf16): equal up to one bf16 ulp from the summation
    order, and equal on nearly every row."""
    from tokengate_amd import gate as G
    g = torch.Generator(device=cuda).manual_seed(rows + inter)
    gu = _bf(torch.randn(rows, 2 * inter + 16, generator=g, device=cuda) * 2)[:, :2 * inter]   # padded rows
    w = _bf(torch.randn(inter, generator=g, device=cuda) * inter ** -0.5)
    got = G.branch_readout(gu, w)
    torch.cuda.synchronize()
    act = torch.nn.functional.silu(gu[:, :inter]) * gu[:, inter:]          # bf16, torch's roundings
    exact = act.double() @ w.double()
    ref = exact.to(torch.bfloat16).float()
    assert torch.equal(got, got.to(torch.bfloat16).float())                # bf16 values
    ulp = torch.finfo(torch.bfloat16).eps * ref.abs().clamp(min=1e-30)
    assert bool(((got - ref).abs() <= ulp + 1e-6).all())
    assert float((got == ref).float().mean()) >= 0.95    # a skipped bf16 rounding of silu or of the
    #                                                       product moves ~1/4 of the rows by an ulp


@pytest.mark.parametrize("rows,vocab,dim", [(1, 151936, 2048), (3, 1000, 2048), (8, 4099, 512), (2, 777, 2560)])
def test_lm_head(cuda, rows, vocab, dim):
    """The LM head GEMV against the float64 product of the same bf16 inputs rounded to bf16 (what
    F.linear on bf16 tensors returns): within one bf16 ulp (summation order), bf16 values, and
    the argmax of each row equal to torch's bf16 F.linear wherever torch's top two differ."""
    from tokengate_amd import decoder as dec
    g = torch.Generator(device=cuda).manual_seed(rows * 7 + vocab)
    x = _bf(torch.randn(rows, dim + 64, generator=g, device=cuda))[:, :dim]     # padded rows
    w = _bf(torch.randn(vocab, dim, generator=g, device=cuda) * dim ** -0.5)
    got = dec.lm_head(x, w)
    torch.cuda.synchronize()
    assert got.shape == (rows, vocab) and got.dtype == torch.float32
    ref = (x.double() @ w.double().t()).to(torch.bfloat16).float()
    assert torch.equal(got, got.to(torch.bfloat16).float())
    ulp = torch.finfo(torch.bfloat16).eps * ref.abs().clamp(min=1e-30)
    assert bool(((got - ref).abs() <= ulp + 1e-6).all())
    tl = torch.nn.functional.linear(x, w).float()
    top2 = tl.topk(2, dim=-1).values
    clear = top2[:, 0] > top2[:, 1]
    assert torch.equal(got.argmax(-1)[clear], tl.argmax(-1)[clear])


@pytest.mark.parametrize("rows,n_out,dim", [(1, 4096, 2048), (3, 2048, 6144), (8, 12288, 2048), (2, 2048, 1024),
                                          (2, 1000, 4096), (1, 517, 2560)])
def test_linear_rows(cuda, rows, n_out, dim):
    """The decode-step projection GEMV (tg_linear_rows, bf16 out) against the float64 product of
    the same bf16 inputs rounded to bf16 (F.linear on bf16 tensors): within one bf16 ulp
    (summation order), into a strided output view as the decode step writes it."""
    from tokengate_amd import decoder as dec
    g = torch.Generator(device=cuda).manual_seed(rows * 11 + n_out)
    x = _bf(torch.randn(rows, dim + 64, generator=g, device=cuda))[:, :dim]
    w = _bf(torch.randn(n_out, dim, generator=g, device=cuda) * dim ** -0.5)
    buf = torch.zeros(rows, n_out + 32, dtype=torch.bfloat16, device=cuda)
    got = dec.linear_rows(x, w, out=buf[:, :n_out])
    torch.cuda.synchronize()
    assert got.dtype == torch.bfloat16 and got.data_ptr() == buf.data_ptr()
    assert bool((buf[:, n_out:] == 0).all())
    ref = (x.double() @ w.double().t()).to(torch.bfloat16).double()
    ulp = torch.finfo(torch.bfloat16).eps * ref.abs().clamp(min=1e-30)
    err = (got.double() - ref).abs()
    assert bool((err <= ulp + 1e-6).all()), float(err.max())
    print(f"[linear_rows] rows {rows} ({n_out}, {dim}): equal to the rounded float64 product on "
          f"{float((err == 0).double().mean()):.4f} of entries", flush=True)


@pytest.mark.parametrize("rows,n_out,dim", [(1, 4096, 2048), (5, 2048, 1024), (8, 12288, 2048), (2, 1000, 4096),
                                          (3, 517, 2560), (7, 333, 512)])
@pytest.mark.parametrize("with_res", [False, True])
def test_linear_rows_norm_and_swiglu(cuda, rows, n_out, dim, with_res):
    """The fused-input projections equal their two-launch forms bit for bit: RMSNorm (tg_rmsnorm,
    residual add and residual write-back) then tg_linear_rows, and silu_mul then tg_linear_rows;
    the fp32-output form equals the bf16 one converted."""
    from tokengate_amd import decoder as dec
    g = torch.Generator(device=cuda).manual_seed(rows * 7 + n_out + with_res)
    h = _bf(torch.randn(rows, dim, generator=g, device=cuda))
    res = _bf(torch.randn(rows, dim, generator=g, device=cuda)) if with_res else None
    nw = _bf(1.0 + 0.1 * torch.randn(dim, generator=g, device=cuda))
    w = _bf(torch.randn(n_out, dim, generator=g, device=cuda) * dim ** -0.5)
    ro = torch.empty_like(h)
    got = dec.linear_rows_norm(h, nw, 1e-6, w, residual=res, residual_out=ro)
    got32 = dec.linear_rows_norm(h, nw, 1e-6, w, residual=res, out_fp32=True)
    r2 = res.clone() if with_res else None
    normed = dec.rmsnorm(h, nw, 1e-6, residual=r2, residual_out=r2)
    ref = dec.linear_rows(normed, w)
    torch.cuda.synchronize()
    assert torch.equal(got, ref) and torch.equal(got32, ref.float())
    assert torch.equal(ro, r2 if with_res else h)
    gu = _bf(torch.randn(rows, 2 * dim, generator=g, device=cuda))
    wd = _bf(torch.randn(n_out, dim, generator=g, device=cuda) * dim ** -0.5)
    got = dec.linear_rows_swiglu(gu, wd)
    ref = dec.linear_rows(dec.silu_mul(gu), wd)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


@pytest.mark.parametrize("rows,n_out,inter", [(1, 2048, 6144), (2, 2048, 6144), (8, 1000, 6144), (3, 998, 4096)])
def test_linear_rows_swiglu_long_rows(cuda, rows, n_out, inter):
    """The down projection's long rows (split-K form: four waves per 4 output rows): the SwiGLU-fused
    input equals silu_mul then tg_linear_rows bit for bit, at the decoder's 6144 and another length."""
    from tokengate_amd import decoder as dec
    g = torch.Generator(device=cuda).manual_seed(rows * 13 + n_out + inter)
    gu = _bf(torch.randn(rows, 2 * inter, generator=g, device=cuda))
    wd = _bf(torch.randn(n_out, inter, generator=g, device=cuda) * inter ** -0.5)
    got = dec.linear_rows_swiglu(gu, wd)
    ref = dec.linear_rows(dec.silu_mul(gu), wd)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


@pytest.mark.parametrize("rows,V", [(1, 151936), (3, 1001), (8, 151936)])
def test_argmax_rows(cuda, rows, V):
    """tg_argmax_rows against torch.argmax: bf16-valued logits (ties at the top are common), a
    planted tie between two maxima, a NaN row, a row of -inf and a ragged length."""
    from tokengate_amd import decoder as dec
    g = torch.Generator(device=cuda).manual_seed(rows + V)
    pad = 4 - V % 4                               # a padded row stride that is a multiple of 4
    x = torch.randn(rows, V + pad, generator=g, device=cuda).to(torch.bfloat16).float()[:, :V]
    x[0, V // 3] = x[0, V - 1] = float(x[0].max()) + 1.0                      # tie: the lower index wins
    if rows > 1:
        x[1, 5] = float("nan")
        x[1, V - 2] = float("nan")
    if rows > 2:
        x[2] = -float("inf")
    got = dec.argmax_rows(x)
    assert torch.equal(got, x.argmax(-1)), (got, x.argmax(-1))
    assert int(got[0]) == V // 3


def test_decoder_op_errors(cuda):
    from tokengate_amd import decoder as dec
    x = torch.zeros(4, 2050, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        dec.rmsnorm(x[:, :2044], torch.ones(2044, dtype=torch.bfloat16, device=cuda), 1e-6)
    with pytest.raises(RuntimeError, match="inter"):
        dec.silu_mul(torch.zeros(3, 6, dtype=torch.bfloat16, device=cuda))
