"""The threshold selection mode on the CPU (_select_threshold, gate_forward.py:102-125).

* gate.sigmoid_threshold (host logic of the product): the least fp32 b_star with
  torch.sigmoid(b_star) >= tau, so that a kernel evaluates `sigmoid(b) >= tau` as `b >= b_star`.
  Checked against torch.sigmoid itself over every fp32 value within 4096 ulps of b_star, over
  200k random values of every magnitude, and at the special values, for a range of tau (the
  init value 0.5, values near 0 and 1, tau <= 0: everything passes, tau > 1: nothing does).
* oracle.gate.select_threshold (the oracle's restatement, written on b_star) against the reference's
  own expression evaluated with torch: sigmoid(b) >= tau, nonzero, and torch.argmax when nothing
  passes -- random values, ties, NaN, all rejected, the init case b = 0 at tau = 0.5 (every token
  kept), empty spans.
"""
import numpy as np
import pytest
import torch

from oracle import gate as og
from tokengate_amd import gate as G

TAUS = [0.5, 0.3, 0.9, 0.999, 0.9999999, 1.0, 1e-30, 1e-45, 0.0, -1.0, 1.5, 0.7310586, 0.25, 0.6]


def _ordered(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.int64)
    return np.where(u & 0x80000000, (~u) & 0xFFFFFFFF, u | 0x80000000)


def _ref_pass(x, tau):
    return (torch.sigmoid(torch.from_numpy(np.asarray(x, np.float32))) >= tau).numpy()


@pytest.mark.parametrize("tau", TAUS)
def test_sigmoid_threshold_equals_torch_sigmoid(tau):
    b = G.sigmoid_threshold(tau, "cpu")
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(200_000) * 10.0 ** rng.uniform(-40, 3, 200_000)).astype(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45, 3.4e38, -3.4e38, 16.0, 17.0, 88.0, -88.0, -104.0],
                       np.float32)
    vals = [x, special]
    if np.isfinite(b):
        k = _ordered(np.float32(b))
        near = np.arange(k - 4096, k + 4097, dtype=np.int64)
        near = near[(near >= 0x007FFFFF) & (near <= 0xFF800000)]
        vals.append(G._f32_of_keys(near))
    for v in vals:
        with np.errstate(invalid="ignore"):
            got = v >= np.float32(b) if not np.isnan(b) else np.zeros(len(v), bool)
        assert np.array_equal(got, _ref_pass(v, tau)), (tau, b)
    nan = np.array([np.nan], np.float32)
    assert not _ref_pass(nan, tau)[0]                  # NaN never passes, as in the kernel
    if tau <= 0:
        assert b == float("-inf")
    if tau > 1:
        assert np.isnan(b)
    if tau == 0.5:
        assert b <= 0.0 and _ref_pass(np.float32(0.0)[None], tau)[0]


def _ref_threshold(agg, tau):
    """The reference's expression, evaluated with torch (sigmoid, nonzero, argmax)."""
    t = torch.from_numpy(np.asarray(agg, np.float32))
    idx = (torch.sigmoid(t) >= tau).nonzero(as_tuple=True)[0]
    if idx.numel() == 0:
        return t.argmax(dim=0, keepdim=True).numpy()
    return idx.numpy()


@pytest.mark.parametrize("seed", range(40))
def test_oracle_select_threshold_matches_reference_expression(seed):
    rng = np.random.default_rng(100 + seed)
    n = int(rng.integers(1, 3000))
    kind = seed % 5
    agg = (rng.standard_normal(n) * rng.uniform(0.1, 4)).astype(np.float32)
    if kind == 1:
        agg = og.bf16(agg)                                  # ties
    elif kind == 2:
        agg[rng.choice(n, max(1, n // 10), replace=False)] = np.nan
    elif kind == 3:
        agg = np.round(agg * 2).astype(np.float32) / 2      # few values
    elif kind == 4:
        agg = np.zeros(n, np.float32)                       # the init case (W_B = 0)
    tau = float(rng.choice([0.5, 0.2, 0.8, 0.99, 0.999999, 0.5000001, 0.4999999]))
    b = G.sigmoid_threshold(tau, "cpu")
    got = og.select_threshold(agg, b)
    want = _ref_threshold(agg, tau)
    assert np.array_equal(got, want), (seed, tau)


def test_oracle_select_threshold_cases():
    b_half = G.sigmoid_threshold(0.5, "cpu")
    # init: every score 0, tau 0.5 -> every article token kept (the non-strict comparison)
    assert np.array_equal(og.select_threshold(np.zeros(7, np.float32), b_half), np.arange(7))
    # all rejected -> the argmax; ties -> the first; NaN counts as maximal (torch.argmax)
    b_hi = G.sigmoid_threshold(0.999, "cpu")
    for agg in ([1.0, 3.0, 2.0, 3.0], [np.nan, 1.0], [1.0, np.nan, 5.0, np.nan], [-2.0, -2.0]):
        a = np.array(agg, np.float32)
        assert np.array_equal(og.select_threshold(a, b_hi), _ref_threshold(a, 0.999))
    assert og.select_threshold(np.zeros(0, np.float32), b_half).size == 0
    kp = og.threshold_keep_indices(np.array([0.0, -5.0, 2.0], np.float32), b_half, 4, 7, 10)
    assert np.array_equal(kp, [0, 1, 2, 3, 4, 6, 7, 8, 9])


def test_selection_values_is_the_aggregate_chain():
    rng = np.random.default_rng(5)
    raw = og.bf16(rng.standard_normal(500).astype(np.float32))
    gs = rng.standard_normal((3, 16)).astype(np.float32)
    assert np.array_equal(og.selection_values(raw, gs, gain=1.25),
                          og.aggregate(og.gate_bias_layers(raw, gs, gain=1.25)))
