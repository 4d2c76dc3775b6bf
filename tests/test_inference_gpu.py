"""GPU checks of load_model().generate(): the greedy decode over the pruned caches against the
oracle's teacher-forced decode (oracle.prefill.decode_logits: generated tokens through layers
0..gate over the full prompt and through the layers above over the kept rows, prompt keys
keeping their gate bias), logits within max-abs 2e-2 (relative to max(1, |ref|)) and rel-L2
2e-2 (several bf16 layers; measured values printed); and the generate() contract: first-EOS truncation, the streamer,
kept positions, per-sequence K, prune_below_gate."""
import numpy as np
import pytest
import torch

from oracle import prefill as op
from tests.attn_util import assert_close_grad, to_np

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=4, d_model=2048, n_heads=16, n_kv_heads=8, head_dim=128, d_ff=1024, vocab=512)


def _model(cuda, seed=3, ssmax=False, branch=False):
    from tokengate_amd import decoder as dec
    from tokengate_amd import gate as G
    from tokengate_amd import inference as I
    m = I.load_model(f"random:{seed}", gate_layer=1, device=cuda, shape=dec.DecoderShape(**SMALL))
    if branch:      # the finalized gate: MLP scoring branch, split gate layer
        m.gate = G.random_branch_head(m.weights, 1, seed=seed + 40)
    m.gate.scaled_softmax = ssmax
    if ssmax:   # a visible temperature spread, so r and gamma both matter
        g = torch.Generator(device=cuda).manual_seed(seed)
        m.gate.attn_scale = m.gate.attn_scale + 0.4 * torch.randn(m.gate.attn_scale.shape, generator=g, device=cuda)
    return m


def _prompts(lens, spans, seed):
    from tokengate_amd import inference as I
    g = torch.Generator().manual_seed(seed)
    out = []
    for n, (s, e) in zip(lens, spans):
        ids = torch.randint(3, SMALL["vocab"], (n,), generator=g).tolist()
        out.append(ids[:s] + [I.STATE_START_ID] + ids[s:e] + [I.STATE_END_ID] + ids[e:])
    return out


@pytest.mark.parametrize("prune_below_gate,ssmax,branch,headroom,graph", [
    (False, False, False, True, False), (True, False, False, True, False), (False, True, False, True, False),
    (True, True, True, True, False), (False, True, False, False, False), (True, False, False, False, False),
    (False, False, False, True, True), (True, True, True, True, True), (True, False, False, False, True)])
def test_decode_matches_oracle(cuda, prune_below_gate, ssmax, branch, headroom, graph):
    """Greedy decode steps against the oracle, appending in place to the prefill's caches (headroom)
    or to a copy laid out with room (a prefill without headroom); with graph=True steps 2.. are
    replays of one captured HIP graph of the step."""
    from tokengate_amd import inference as I
    from tokengate_amd.decode import DecodeState
    torch.set_num_threads(min(16, torch.get_num_threads()))
    m = _model(cuda, ssmax=ssmax, branch=branch)
    lens, spans, Ks = [600, 333], [(20, 500), (0, 300)], [64, 1000]
    split = [I.split_state_span(p) for p in _prompts(lens, spans, 5)]
    steps = 4
    pf = m.prefill(split, Ks, prune_below_gate=prune_below_gate, decode_headroom=steps + 1 if headroom else 0)
    st = DecodeState(m.weights, m.gate, m.gate_layer, pf, steps + 1, prune_below_gate, graph=graph)
    assert st.in_place == headroom
    if headroom:
        assert all(st.kv[l].k.data_ptr() == pf.kv[l].k.data_ptr() for l in range(len(st.kv)))
    cur = pf.first_tokens
    toks, logits = [cur], []
    for _ in range(steps):
        cur = st.step(cur)
        toks.append(cur)
        logits.append(st.last_logits.float().cpu())
    torch.cuda.synchronize()
    W = op.Weights(m.weights)
    kp = pf.kept_positions.cpu().numpy()
    for b, (clean, s, e) in enumerate(split):
        keep = kp[pf.cu_kept[b]:pf.cu_kept[b + 1]]
        gen = [int(t[b]) for t in toks[:steps]]      # tokens fed to the decode steps
        ref = op.decode_logits(W, m.gate, clean, s, e, m.gate_layer, keep, gen, prune_below_gate)
        for i in range(steps):
            ma, rl = assert_close_grad(f"seq {b} step {i}", to_np(logits[i][b]), to_np(ref[1 + i]), rel_l2=2e-2)
            print(f"[decode] seq {b} step {i}: logits max-abs/max(1,|ref|) {ma:.2e} rel-L2 {rl:.2e}", flush=True)
            assert int(toks[i + 1][b]) == int(logits[i][b].argmax())
    assert (st._graph is not None) == graph


@pytest.mark.parametrize("seed", [100, 110, 113, 124, 129])
def test_decode_random_geometries(cuda, seed):
    """Seeded random batches (1-4 prompts of up to 900 tokens, state spans down to one token, K
    from 1 to beyond the span, 1-5 greedy steps) over random combinations of prune-below-gate,
    scaled softmax, the finalized gate, in-place headroom and graph replay, against the oracle's
    teacher-forced decode as in test_decode_matches_oracle."""
    from tokengate_amd import inference as I
    from tokengate_amd.decode import DecodeState
    torch.set_num_threads(min(16, torch.get_num_threads()))
    rng = np.random.default_rng(seed)
    lens, spans, Ks = [], [], []
    for _ in range(int(rng.integers(1, 5))):
        L = int(rng.integers(2, 900))
        s = int(rng.integers(0, min(L, 60) + 1))
        e = int(rng.integers(s, L + 1))
        lens.append(L); spans.append((s, e))
        Ks.append(int(rng.choice([1, 16, 64, 300, 5000, int(rng.integers(1, L + 1))])))
    pbg, ssmax, branch, headroom, graph = (bool(rng.random() < p) for p in (0.5, 0.4, 0.3, 0.7, 0.4))
    steps = int(rng.integers(1, 6))
    print(f"[random decode] seed {seed}: lens={lens} spans={spans} K={Ks} prune_below_gate={pbg} ssmax={ssmax} "
          f"branch={branch} headroom={headroom} graph={graph} steps={steps}", flush=True)
    m = _model(cuda, ssmax=ssmax, branch=branch)
    split = [I.split_state_span(p) for p in _prompts(lens, spans, 5 + seed)]
    pf = m.prefill(split, Ks, prune_below_gate=pbg, decode_headroom=steps + 1 if headroom else 0)
    st = DecodeState(m.weights, m.gate, m.gate_layer, pf, steps + 1, pbg, graph=graph)
    assert st.in_place == headroom
    cur = pf.first_tokens
    toks, logits = [cur], []
    for _ in range(steps):
        cur = st.step(cur)
        toks.append(cur)
        logits.append(st.last_logits.float().cpu())
    torch.cuda.synchronize()
    W = op.Weights(m.weights)
    kp = pf.kept_positions.cpu().numpy()
    for b, (clean, s, e) in enumerate(split):
        keep = kp[pf.cu_kept[b]:pf.cu_kept[b + 1]]
        gen = [int(t[b]) for t in toks[:steps]]
        ref = op.decode_logits(W, m.gate, clean, s, e, m.gate_layer, keep, gen, pbg)
        for i in range(steps):
            ma, rl = assert_close_grad(f"seq {b} step {i}", to_np(logits[i][b]), to_np(ref[1 + i]), rel_l2=2e-2)
            print(f"[random decode] seq {b} step {i}: logits max-abs/max(1,|ref|) {ma:.2e} rel-L2 {rl:.2e}", flush=True)
            assert int(toks[i + 1][b]) == int(logits[i][b].argmax())


def test_decode_fused_projections_match_unfused(cuda):
    """The decode step with each RMSNorm folded into the projection after it, the SwiGLU product
    into the down projection and the final norm into the LM head (one launch each) gives the same
    tokens and logits, bit for bit, as the step with separate norm / silu_mul launches."""
    from tokengate_amd import inference as I
    from tokengate_amd.decode import DecodeState
    m = _model(cuda, seed=11, ssmax=True)
    split = [I.split_state_span(p) for p in _prompts([520, 300], [(12, 500), (0, 280)], 4)]
    steps = 5
    pfs = [m.prefill(split, [30, 400], decode_headroom=steps + 1) for _ in range(2)]
    plain = DecodeState(m.weights, m.gate, m.gate_layer, pfs[0], steps + 1, fused=False)
    fused = DecodeState(m.weights, m.gate, m.gate_layer, pfs[1], steps + 1, fused=True)
    cp = cf = pfs[0].first_tokens
    for i in range(steps):
        cp = plain.step(cp)
        cf = fused.step(cf)
        torch.cuda.synchronize()
        assert torch.equal(cp, cf), f"step {i}: tokens differ"
        assert torch.equal(plain.last_logits, fused.last_logits), f"step {i}: logits differ"


def test_decode_graph_replays_match_eager(cuda):
    """Every replay of the captured decode step equals the eager step bit for bit (tokens and
    logits), with eager work and host synchronisations between the replays; the two decodes
    run over two identical prefills (each appends to its own caches)."""
    from tokengate_amd import inference as I
    from tokengate_amd.decode import DecodeState
    m = _model(cuda, seed=6, ssmax=True)
    split = [I.split_state_span(p) for p in _prompts([700, 420, 150], [(30, 640), (0, 400), (10, 140)], 8)]
    steps = 7
    pfs = [m.prefill(split, [40, 200, 1000], decode_headroom=steps + 1) for _ in range(2)]
    eager = DecodeState(m.weights, m.gate, m.gate_layer, pfs[0], steps + 1)
    graph = DecodeState(m.weights, m.gate, m.gate_layer, pfs[1], steps + 1, graph=True)
    ce = cg = pfs[0].first_tokens
    assert torch.equal(pfs[0].first_tokens, pfs[1].first_tokens)
    for i in range(steps):
        ce = eager.step(ce)
        cg = graph.step(cg)
        junk = torch.randn(1 << 20, device=cuda).sum()      # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(ce, cg), f"step {i}: tokens differ"
        assert torch.equal(eager.last_logits, graph.last_logits), f"step {i}: logits differ"
        assert bool(torch.isfinite(junk))
    assert graph._graph is not None and eager._graph is None


class _Tok:
    def __init__(self, eos):
        self.eos_token_id = eos

    def decode(self, ids, skip_special_tokens=True):
        return " ".join(str(i) for i in ids)


class _Streamer:
    def __init__(self):
        self.rows, self.ended = [], False

    def put(self, t):
        self.rows.append(t.clone())

    def end(self):
        self.ended = True


def test_generate_contract(cuda):
    from tokengate_amd import inference as I
    m = _model(cuda, seed=4)
    prompts = _prompts([400, 250], [(10, 380), (5, 240)], 9)
    free = m.generate(prompts, None, max_new_tokens=6, max_kept_prefill_tokens=[50, 10_000])
    assert free.answers == ["", ""] and all(len(t) == 6 for t in free.token_ids)
    assert free.n_state == [370, 235]
    assert free.n_kept == [10 + 50 + 20, 250]
    for b, (clean, s, e) in enumerate(I.split_state_span(p) for p in prompts):
        kp = free.kept_pos[b]
        assert kp == sorted(kp) and kp[:s] == list(range(s)) and kp[len(kp) - (len(clean) - e):] == list(range(e, len(clean)))
    # EOS = the token sequence 0 produced at step 2: its row stops there, the batch runs on
    eos = free.token_ids[0][2]
    streamer = _Streamer()
    out = m.generate(prompts, _Tok(eos), max_new_tokens=6, max_kept_prefill_tokens=[50, 10_000], streamer=streamer)
    assert out.token_ids[0] == free.token_ids[0][:free.token_ids[0].index(eos) + 1]
    assert out.answers[0] == " ".join(str(t) for t in free.token_ids[0][:free.token_ids[0].index(eos)])
    assert streamer.ended and all(r.shape == (2, 1) for r in streamer.rows)
    got = [int(r[0, 0]) for r in streamer.rows]
    assert got == free.token_ids[0][:len(got)] and len(got) > free.token_ids[0].index(eos)
    assert out.prefill_s > 0 and out.decode_s >= 0
    with pytest.raises(ValueError):
        m.generate([[1, 2, 3]], None)
