"""Shared helpers for the attention tests: seeded inputs and the tolerance check."""
import numpy as np
import torch

# Tolerances against the float64 evaluation of the reference math (bf16 kernels).
MAX_ABS = 2e-2
REL_L2 = 1e-2


def bias_logsigmoid(shape, sigma, gen, device="cpu"):
    """log(sigmoid(z)), z ~ N(0, sigma): the key-bias distribution of the benchmark configs."""
    z = torch.randn(shape, generator=gen, device=device) * sigma
    return torch.nn.functional.logsigmoid(z)


def to_np(t):
    return t.detach().float().cpu().numpy()


def errs(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    fin = np.isfinite(ref)
    assert np.array_equal(fin, np.isfinite(got)), "finite pattern differs"
    d = np.abs(got[fin] - ref[fin])
    max_abs = float(d.max()) if d.size else 0.0
    den = float(np.linalg.norm(ref[fin]))
    rel = float(np.linalg.norm(got[fin] - ref[fin]) / max(den, 1e-30))
    return max_abs, rel


def assert_close(name, got, ref, max_abs=MAX_ABS, rel_l2=REL_L2):
    ma, rl = errs(got, ref)
    assert ma <= max_abs and rl <= rel_l2, f"{name}: max-abs {ma:.3e} (<= {max_abs}), rel-L2 {rl:.3e} (<= {rel_l2})"
    return ma, rl


def assert_close_grad(name, got, ref, max_abs=MAX_ABS, rel_l2=REL_L2, rms_floor=1e-3):
    """Gradient check in bf16 terms: gradients are bf16 tensors whose entries reach magnitudes
    (tens) where one bf16 ulp exceeds 2e-2, so the max-abs bound is taken relative to
    max(1, max|ref|); the rel-L2 bound uses an RMS floor so that gradients that are exactly
    zero in exact arithmetic (a query with a single visible key has dS = 0) are judged by their
    absolute error."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert np.isfinite(got).all(), f"{name}: non-finite values"
    d = np.abs(got - ref)
    scale = max(1.0, float(np.abs(ref).max()) if ref.size else 1.0)
    ma = float(d.max()) / scale if d.size else 0.0
    den = max(float(np.linalg.norm(ref)), rms_floor * np.sqrt(max(ref.size, 1)))
    rl = float(np.linalg.norm(got - ref)) / den
    assert ma <= max_abs and rl <= rel_l2, (f"{name}: max-abs/max(1,|ref|) {ma:.3e} (<= {max_abs}), "
                                            f"rel-L2 {rl:.3e} (<= {rel_l2})")
    return ma, rl


def assert_grad(name, got, ref, fp32_output=False, max_abs=MAX_ABS, rel_l2=REL_L2, big=4.0, rms_floor=1e-3):
    """Attention-gradient check at the stated bound.  fp32 outputs (dBias, softmax_d): absolute
    max-abs <= 2e-2 and rel-L2 <= 1e-2.  bf16 outputs (dQ, dK, dV): absolute max-abs <= 2e-2 on
    entries with |ref| < 4 (where a bf16 half-ulp is at most 1/128) and |err| <= 2e-2 * |ref| / 4
    above that (a bf16 value near 8 is only resolved to 1/32); rel-L2 <= 1e-2.  The rel-L2
    denominator has an RMS floor so that gradients that are zero in exact arithmetic (a query with
    one visible key has dS = 0) are judged by their absolute error.  Prints the absolute figures."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert np.isfinite(got).all(), f"{name}: non-finite values"
    d = np.abs(got - ref)
    ma = float(d.max()) if d.size else 0.0
    den = max(float(np.linalg.norm(ref)), rms_floor * np.sqrt(max(ref.size, 1)))
    rl = float(np.linalg.norm(got - ref)) / den
    if fp32_output:
        ok_abs = ma <= max_abs
        worst = ma
    else:
        a = np.abs(ref)
        small = a < big
        ma_small = float(d[small].max()) if small.any() else 0.0
        ratio_big = float((d[~small] / a[~small]).max()) * big if (~small).any() else 0.0
        ok_abs = ma_small <= max_abs and ratio_big <= max_abs
        worst = max(ma_small, ratio_big)
    print(f"[grad] {name}: max-abs {ma:.3e} (bound-normalised {worst:.3e}), rel-L2 {rl:.3e}, "
          f"max|ref| {float(np.abs(ref).max()) if ref.size else 0.0:.3g}", flush=True)
    assert ok_abs and rl <= rel_l2, (f"{name}: max-abs {ma:.3e} (bound-normalised {worst:.3e} <= {max_abs}), "
                                      f"rel-L2 {rl:.3e} (<= {rel_l2})")
    return ma, rl


def check_bwd(tag, got, exact, faithful=None, names=("dq", "dk", "dv", "dbias_raw", "softmax_d")):
    """Backward parity, two oracles (both with D and P from the forward output and log-sum-exp the
    kernel was given, as the reference's op hands them to its backward):
      * exact — the fp32/float64 evaluation of the math: dBias and softmax_d (fp32 outputs) at
        the absolute bound; dQ/dK/dV at max-abs <= 2e-2 relative to max(1, max|ref|) and rel-L2
        <= 1e-2 (bf16 outputs whose operands P and dS are rounded to bf16 before the MFMA, as in
        the reference's FA2 kernel: their error grows with the magnitude);
      * faithful — the same math with P and dS rounded to bf16 where the reference kernel
        rounds them: dQ/dK/dV at the absolute bound below 4 (assert_grad).
    got / exact / faithful: sequences in `names` order (None entries skipped)."""
    for i, name in enumerate(names):
        if got[i] is None:
            continue
        fp32 = name.startswith("dbias") or name == "softmax_d"
        if fp32:
            assert_grad(f"{name} {tag}", got[i], exact[i], fp32_output=True)
        else:
            ma, rl = errs(got[i], exact[i])
            print(f"[grad exact] {name} {tag}: max-abs {ma:.3e}, rel-L2 {rl:.3e}", flush=True)
            assert_close_grad(f"{name} {tag} (exact)", got[i], exact[i])
            if faithful is not None and faithful[i] is not None:
                assert_grad(f"{name} {tag} (bf16 operands)", got[i], faithful[i])


def qkv(B, Sq, Sk, H, Hkv, gen, device, scale=1.0, D=128):
    q = (torch.randn(B, Sq, H, D, generator=gen, device=device) * scale).to(torch.bfloat16)
    k = (torch.randn(B, Sk, Hkv, D, generator=gen, device=device) * scale).to(torch.bfloat16)
    v = (torch.randn(B, Sk, Hkv, D, generator=gen, device=device) * scale).to(torch.bfloat16)
    return q, k, v


def checked_ratio(ratio, keep, rtol=5e-7):
    """A pipeline's scaled-softmax ratio of one sequence's kept rows (fp32, None without one),
    checked against the float64 closed form r = min(1, ln max(m, 2) / ln max(p + 1, 2)) to a few
    fp32 units, and returned as numpy for the oracle's bf16 chain (oracle.prefill.phase2_tables),
    whose rounding of r to bf16 must follow the pipeline's own fp32 value."""
    if ratio is None:
        return None
    from oracle import gate as og
    got = ratio.float().cpu().numpy().astype(np.float64)
    want = og.ssmax_ratio(np.asarray(keep))
    np.testing.assert_allclose(got, want, rtol=rtol, atol=0)
    return got.astype(np.float32)

