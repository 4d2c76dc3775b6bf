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


def qkv(B, Sq, Sk, H, Hkv, gen, device, scale=1.0, D=128):
    q = (torch.randn(B, Sq, H, D, generator=gen, device=device) * scale).to(torch.bfloat16)
    k = (torch.randn(B, Sk, Hkv, D, generator=gen, device=device) * scale).to(torch.bfloat16)
    v = (torch.randn(B, Sk, Hkv, D, generator=gen, device=device) * scale).to(torch.bfloat16)
    return q, k, v
