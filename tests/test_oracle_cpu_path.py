"""Pins of oracle/cpu_path.py (the reference's CPU execution restated in torch, timed as the CPU
baseline): the chunked-SDPA attention against the float64 numpy oracle, and the
topk -> sort -> cat -> index_select pruning against the oracle's keep lists and numpy indexing."""
import numpy as np
import pytest
import torch

from oracle import attention as ora
from oracle import cpu_path as cp
from oracle import gate as og


@pytest.mark.parametrize("S,H,Hkv,chunk", [(45, 6, 2, 16), (130, 4, 4, 128), (70, 8, 1, 7)])
def test_sdpa_chunked_matches_numpy_oracle(S, H, Hkv, chunk):
    g = torch.Generator().manual_seed(S + H)
    D = 32
    q = torch.randn(1, S, H, D, generator=g)
    k = torch.randn(1, S, Hkv, D, generator=g)
    v = torch.randn(1, S, Hkv, D, generator=g)
    bias_logit = torch.nn.functional.logsigmoid(torch.randn(1, S, generator=g) * 2)
    scale = D ** -0.5
    ro, _ = ora.keybias_fwd(q.numpy(), k.numpy(), v.numpy(),
                            np.broadcast_to((bias_logit / scale).numpy()[:, None, :], (1, H, S)).copy(), scale, True)
    got = cp.sdpa_chunked(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), bias_logit, chunk=chunk)
    np.testing.assert_allclose(got.transpose(1, 2).numpy(), ro, rtol=1e-4, atol=2e-5)
    # a row range is the same rows of the whole
    part = cp.sdpa_chunked(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), bias_logit, chunk=chunk,
                           rows=range(S - 2 * chunk if S > 2 * chunk else 0, S))
    np.testing.assert_allclose(part.numpy(), got[:, :, -part.shape[2]:].numpy(), rtol=1e-6, atol=1e-7)
    # the bias matters (a plain causal run differs)
    plain = cp.sdpa_chunked(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), None, chunk=chunk)
    assert float((plain - got).abs().max()) > 1e-3


@pytest.mark.parametrize("L,s,e,K", [(1000, 16, 900, 50), (333, 0, 333, 400), (64, 10, 11, 3), (500, 20, 480, 1)])
def test_prune_matches_keep_indices_and_gathers(L, s, e, K):
    rng = np.random.default_rng(L + K)
    sc = rng.permutation(e - s).astype(np.float32) - 7.5            # tie-free
    x = torch.from_numpy(rng.standard_normal((L, 12)).astype(np.float32))
    kv = torch.from_numpy(rng.standard_normal((L, 2, 4)).astype(np.float32))
    keep, (xs, kvs) = cp.prune(torch.from_numpy(sc), K, s, e, L, [x, kv])
    want = og.keep_indices(sc, K, s, e, L)
    assert np.array_equal(keep.numpy(), want)
    assert np.array_equal(xs.numpy(), x.numpy()[want]) and np.array_equal(kvs.numpy(), kv.numpy()[want])
