"""Benchmark: key-bias causal attention forward at 32k context on one MI355X.

One step = one launch of the key-bias attention forward (the drop-in op
recursive_kvs::fa2_keybias_fwd) over the 32k workload: B=1, S=32768, 16 query heads, 8 KV heads,
head_dim 128, bf16, causal; Q/K/V ~ N(0,1)/sqrt(128); per-key bias log(sigmoid(z)), z ~ N(0,3),
forced to 0 on positions [0,64) and [32512,32768), broadcast over heads.  Inputs are generated
on the device before timing (synthetic data).

Before the W warmup steps the forward runs untimed for about 0.15 s (`clock_warmup_launches`): a
per-dispatch clock profile (profiles/prefill_32k_phase1_clock.txt) shows the part's clock ramping
over the first ~10 launches from idle, so without it the timed steps would measure the ramp.

Prints ONE JSON line with the bench contract fields plus:
  roofline     — the attention kernel's algorithmic TFLOP/s (2*B*H*D*S*(S+1) per launch over
                 the mean launch time from HIP events on the launch stream) against the bf16
                 dense MFMA peak; traffic = HBM bytes per launch from the committed rocprofv3
                 counter summary when present;
  cpu_baseline — the reference's CPU attention path (its SDPA compatibility prefill: chunks of 128
                 query rows, an additive float mask, GQA by repeating K/V) restated in float32 torch
                 on the host's threads, timed on a bounded sample of the same workload (the last
                 query chunks, each over every key it sees); `cores` is the thread count used and
                 `affinity_cores` the cores this process may run on;
  extra        — secondary measurements: the 4k forward, the B4 x 8192 backward (TFLOP/s of
                 5*B*H*D*S*(S+1)), the 32k and ragged 8 x 16k-128k gate paths (scoring, top-K,
                 pack, and the whole score -> select -> pack chain in one graph; the short gate
                 launches are timed as replays of a captured HIP graph), and the pruned-prefill
                 time to first token of a Qwen3-1.7B-shaped decoder at 32k (K = 100, 2000, all)
                 and on 8 ragged prompts of 16k-128k tokens.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--cpu-seconds 10]
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA peak
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E


def causal_flops(b, h, s, d=128):
    return 2.0 * b * h * d * s * (s + 1)


def make_inputs(S, H, Hkv, sigma, seed, device, prefix=64, suffix=256, qkv_scale=None):
    import torch
    D = 128
    g = torch.Generator(device=device).manual_seed(seed)
    sc = qkv_scale if qkv_scale is not None else 1.0
    q = (torch.randn(1, S, H, D, generator=g, device=device) * sc).to(torch.bfloat16)
    k = (torch.randn(1, S, Hkv, D, generator=g, device=device) * sc).to(torch.bfloat16)
    v = (torch.randn(1, S, Hkv, D, generator=g, device=device) * sc).to(torch.bfloat16)
    z = torch.randn(1, S, generator=g, device=device) * sigma
    kb = torch.nn.functional.logsigmoid(z)
    if prefix:
        kb[:, :prefix] = 0.0
    if suffix:
        kb[:, S - suffix:] = 0.0
    scale = D ** -0.5
    bias_raw = (kb[:, None, :].expand(1, H, S).float() / scale).contiguous()
    return q, k, v, bias_raw, scale


CLOCK_WARMUP_LAUNCHES = 40


def time_fwd(q, k, v, bias_raw, scale, steps, warmup, clock_warmup=0):
    """Returns (ms_per_step from the bracketing host clock, mean kernel ms from HIP events).
    clock_warmup: untimed launches before the warmup steps (the clock's ramp from idle)."""
    import torch
    op = torch.ops.recursive_kvs.fa2_keybias_fwd
    for _ in range(clock_warmup):
        op(q, k, v, bias_raw, scale, True)
    for _ in range(warmup):
        op(q, k, v, bias_raw, scale, True)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        ev[i][0].record(stream)
        op(q, k, v, bias_raw, scale, True)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    kern_ms = sum(a.elapsed_time(b) for a, b in ev) / steps
    return (t1 - t0) * 1e3 / steps, kern_ms


def time_events(fn, iters, warmup=3):
    """Mean milliseconds of fn() between HIP events on the current stream."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for _ in range(iters):
        fn()
    b.record(st)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters


def time_graph(fn, iters=20, reps=5):
    """Mean milliseconds of fn() with `iters` calls captured in one HIP graph and replayed `reps`
    times: the device time of short launches without the host's launch latency."""
    import torch
    fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(iters):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for _ in range(reps):
        graph.replay()
    b.record(st)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / (iters * reps)


def bench_bwd(dev, iters=5):
    """Backward at B=4, S=8192, 16/8 heads (preprocess + dQ + dK/dV/dBias launches)."""
    import torch
    from tokengate_amd.fa2bias.keybias import ext
    B, S, H, Hkv = 4, 8192, 16, 8
    g = torch.Generator(device=dev).manual_seed(4)
    q = torch.randn(B, S, H, 128, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(B, S, Hkv, 128, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(B, S, Hkv, 128, generator=g, device=dev).to(torch.bfloat16)
    kb = torch.nn.functional.logsigmoid(torch.randn(B, S, generator=g, device=dev) * 2.0)
    scale = 128 ** -0.5
    bias_raw = (kb[:, None, :].expand(B, H, S) / scale).contiguous()
    dout = torch.randn(B, S, H, 128, generator=g, device=dev).to(torch.bfloat16)
    out, lse, _, _ = ext().fwd(q, k, v, None, bias_raw, 0.0, scale, True, -1, -1, 0.0, False, None)
    ms = time_events(lambda: ext().bwd(dout, q, k, v, out, lse, None, None, None, bias_raw, 0.0, scale, True,
                                       -1, -1, 0.0, False, None, None), iters, warmup=2)
    flops = 5.0 * B * H * 128 * S * (S + 1)
    tf = flops / (ms * 1e-3) / 1e12
    return {"ms": round(ms, 4), "tflops": round(tf, 2), "frac_mfma": round(tf / PEAK_BF16_TFLOPS, 4),
            "flop": flops, "shape": "B4 S8192 H16/8 D128 causal, bias [4,8192] broadcast"}


def bench_gate(dev, iters=50):
    """Scoring + top-K + pack on the 32k gate workload: hidden [1,32768,2048], state span 64..32511,
    synthetic head Linear(2048->256)->SiLU->Linear(256->1) (Xavier, seed 5), K/V of 2 layers."""
    import torch
    from tokengate_amd import gate
    S, d, s, e = 32768, 2048, 64, 32512
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(S, d, generator=g, device=dev).to(torch.bfloat16)
    a1 = math.sqrt(6.0 / (d + 256))
    w1 = ((torch.rand(256, d, generator=g, device=dev) * 2 - 1) * a1).to(torch.bfloat16)
    w2 = (torch.rand(256, generator=g, device=dev) * 2 - 1) * math.sqrt(6.0 / 257)
    b1 = torch.zeros(256, device=dev)
    kv = [torch.randn(S, 8, 128, generator=g, device=dev).to(torch.bfloat16) for _ in range(4)]
    scores = torch.empty(S, dtype=torch.float32, device=dev)
    n_art = e - s
    w1k = gate.ktile_w1(w1)   # the head's k-step-major W1 (gate.ScoringHead streams this copy)
    ms_score = time_graph(lambda: gate.score_mlp(x[s:e], w1, b1, w2, 0.0, out=scores[s:e], w1_ktiled=w1k))
    ms_score_rm = time_graph(lambda: gate.score_mlp(x[s:e], w1, b1, w2, 0.0, out=scores[s:e]))
    score_bytes = n_art * d * 2 + w1.numel() * 2 + n_art * 4
    score_flop = 2.0 * n_art * d * 256
    res = {"score": {"ms": round(ms_score, 4), "gbs": round(score_bytes / (ms_score * 1e-3) / 1e9, 1),
                     "frac_hbm": round(score_bytes / (ms_score * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                     "tflops": round(score_flop / (ms_score * 1e-3) / 1e12, 1),
                     "frac_mfma": round(score_flop / (ms_score * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4), "rows": n_art,
                     "ms_w1_row_major": round(ms_score_rm, 4)}}
    for K in (100, 500, 2000):
        p = gate.plan([0], [S], [s], [e], [K], dev)
        T = p.total_kept
        outs = [torch.empty(T, d, dtype=torch.bfloat16, device=dev)] + \
               [torch.empty(T, 8, 128, dtype=torch.bfloat16, device=dev) for _ in kv]
        pos = torch.empty(T, dtype=torch.int64, device=dev)
        bias = torch.empty(T, dtype=torch.float32, device=dev)
        keep = torch.empty(T, dtype=torch.int64, device=dev)
        ss = torch.empty(1, dtype=torch.float32, device=dev)
        pairs = list(zip([x] + kv, outs))
        ms_topk = time_graph(lambda: gate.select_keep(scores, p, keep_out=keep, sumsq_out=ss))
        ms_pack = time_graph(lambda: gate.pack(keep, p, pairs, positions=pos, bias_src=scores, sumsq=ss,
                                               bias_out=bias))
        # the pair as the prefill runs it: both launches back to back in one graph
        ms_pair = time_graph(lambda: (gate.select_keep(scores, p, keep_out=keep, sumsq_out=ss),
                                      gate.pack(keep, p, pairs, positions=pos, bias_src=scores, sumsq=ss,
                                                bias_out=bias)))
        pack_bytes = 2 * T * (d * 2 + 4 * 8 * 128 * 2) + T * (8 + 8 + 4 + 4)
        topk_bytes = n_art * 4 + T * 8
        both = (pack_bytes + topk_bytes) / ((ms_topk + ms_pack) * 1e-3) / 1e9
        pair = (pack_bytes + topk_bytes) / (ms_pair * 1e-3) / 1e9
        # the prefill's path: multi-workgroup selection, then the pack (gate.select_pack)
        ms_sel = time_graph(lambda: gate.select_pack(scores, p, [], positions=pos, bias_out=bias, keep_out=keep))
        ms_sp = time_graph(lambda: gate.select_pack(scores, p, pairs, positions=pos, bias_out=bias, keep_out=keep))
        sp = (pack_bytes + topk_bytes) / (ms_sp * 1e-3) / 1e9
        # the whole chain from the hidden states: scoring head, selection, pack (one graph)
        ms_chain = time_graph(lambda: (gate.score_mlp(x[s:e], w1, b1, w2, 0.0, out=scores[s:e], w1_ktiled=w1k),
                                       gate.select_pack(scores, p, pairs, positions=pos, bias_out=bias,
                                                        keep_out=keep)))
        chain = (score_bytes + pack_bytes + topk_bytes) / (ms_chain * 1e-3) / 1e9
        res[f"K{K}"] = {"kept": T, "topk_ms": round(ms_topk, 4), "pack_ms": round(ms_pack, 4),
                        "pack_gbs": round(pack_bytes / (ms_pack * 1e-3) / 1e9, 1),
                        "pack_frac_hbm": round(pack_bytes / (ms_pack * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                        "topk_plus_pack_gbs": round(both, 1),
                        "topk_plus_pack_frac_hbm": round(both / PEAK_HBM_GBS, 4),
                        "topk_pack_one_graph_ms": round(ms_pair, 4),
                        "topk_pack_one_graph_frac_hbm": round(pair / PEAK_HBM_GBS, 4),
                        "select_multi_wg_ms": round(ms_sel, 4),
                        "select_pack_ms": round(ms_sp, 4), "select_pack_gbs": round(sp, 1),
                        "select_pack_frac_hbm": round(sp / PEAK_HBM_GBS, 4),
                        "score_select_pack_ms": round(ms_chain, 4),
                        "score_select_pack_frac_hbm": round(chain / PEAK_HBM_GBS, 4),
                        "bytes": pack_bytes + topk_bytes}
    return res


def bench_gate_ragged8(dev):
    """Top-K + pack at the ragged prefill's scale: 8 prompts of 16k-128k tokens (prefix 64, suffix
    256), K from {100, 500, 2000, 4000}, bf16-valued scores, the hidden rows (2048 bf16) and 2 layers
    of K/V (8 x 128 bf16) gathered.  Single-workgroup top-K + pack against the multi-workgroup
    selection + pack (gate.select_pack); graph-replayed."""
    import torch
    from tokengate_amd import gate
    lens = [114517, 57946, 113394, 80391, 42386, 123699, 106754, 74151]
    Ks = [2000, 4000, 100, 4000, 100, 100, 4000, 500]
    starts, ends = [64] * 8, [L - 256 for L in lens]
    R = sum(lens)
    row0 = [sum(lens[:b]) for b in range(8)]
    g = torch.Generator(device=dev).manual_seed(8)
    scores = torch.randn(R, generator=g, device=dev).to(torch.bfloat16).float()
    x = torch.randn(R, 2048, generator=g, device=dev).to(torch.bfloat16)
    kv = [torch.randn(R, 8, 128, generator=g, device=dev).to(torch.bfloat16) for _ in range(4)]
    # the scoring head over all rows of the batch (the 256-row workgroup form at this size)
    a1 = math.sqrt(6.0 / (2048 + 256))
    w1 = ((torch.rand(256, 2048, generator=g, device=dev) * 2 - 1) * a1).to(torch.bfloat16)
    w2 = (torch.rand(256, generator=g, device=dev) * 2 - 1) * math.sqrt(6.0 / 257)
    b1 = torch.zeros(256, device=dev)
    sc_out = torch.empty(R, dtype=torch.float32, device=dev)
    w1k = gate.ktile_w1(w1)
    ms_score = time_graph(lambda: gate.score_mlp(x, w1, b1, w2, 0.0, out=sc_out, w1_ktiled=w1k))
    ms_score_rm = time_graph(lambda: gate.score_mlp(x, w1, b1, w2, 0.0, out=sc_out))
    score_bytes = R * 2048 * 2 + w1.numel() * 2 + R * 4
    p = gate.plan(row0, lens, starts, ends, Ks, dev)
    T = p.total_kept
    outs = [torch.empty(T, 2048, dtype=torch.bfloat16, device=dev)] + \
           [torch.empty(T, 8, 128, dtype=torch.bfloat16, device=dev) for _ in kv]
    pos = torch.empty(T, dtype=torch.int64, device=dev)
    bias = torch.empty(T, dtype=torch.float32, device=dev)
    keep = torch.empty(T, dtype=torch.int64, device=dev)
    ss = torch.empty(8, dtype=torch.float32, device=dev)
    pairs = list(zip([x] + kv, outs))
    ms_old = time_graph(lambda: (gate.select_keep(scores, p, keep_out=keep, sumsq_out=ss),
                                 gate.pack(keep, p, pairs, positions=pos, bias_src=scores, sumsq=ss, bias_out=bias)))
    ms_topk = time_graph(lambda: gate.select_keep(scores, p, keep_out=keep, sumsq_out=ss))
    ms_sel = time_graph(lambda: gate.select_pack(scores, p, [], positions=pos, bias_out=bias, keep_out=keep))
    ms_new = time_graph(lambda: gate.select_pack(scores, p, pairs, positions=pos, bias_out=bias, keep_out=keep))
    # the whole chain from the hidden states: scoring head over every row, selection, pack (one graph)
    ms_chain = time_graph(lambda: (gate.score_mlp(x, w1, b1, w2, 0.0, out=sc_out, w1_ktiled=w1k),
                                   gate.select_pack(sc_out, p, pairs, positions=pos, bias_out=bias, keep_out=keep)))
    n_art = sum(e - s for s, e in zip(starts, ends))
    byts = 2 * T * (2048 * 2 + 4 * 8 * 128 * 2) + T * (8 + 8 + 4 + 4) + n_art * 4
    gbs = lambda ms: byts / (ms * 1e-3) / 1e9
    score_flop = 2.0 * R * 2048 * 256
    return {"score": {"rows": R, "ms": round(ms_score, 4), "gbs": round(score_bytes / (ms_score * 1e-3) / 1e9, 1),
                      "frac_hbm": round(score_bytes / (ms_score * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                      "tflops": round(score_flop / (ms_score * 1e-3) / 1e12, 1),
                      "frac_mfma": round(score_flop / (ms_score * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                      "ms_w1_row_major": round(ms_score_rm, 4)},
            "kept": T, "lens": lens, "K": Ks, "bytes": byts,
            "topk_single_wg_ms": round(ms_topk, 4), "topk_pack_ms": round(ms_old, 4),
            "topk_pack_frac_hbm": round(gbs(ms_old) / PEAK_HBM_GBS, 4),
            "select_multi_wg_ms": round(ms_sel, 4), "select_pack_ms": round(ms_new, 4),
            "select_pack_gbs": round(gbs(ms_new), 1), "select_pack_frac_hbm": round(gbs(ms_new) / PEAK_HBM_GBS, 4),
            "score_select_pack_ms": round(ms_chain, 4),
            "score_select_pack_frac_hbm": round((byts + score_bytes) / (ms_chain * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}


def bench_ttft(dev, reps=5):
    """Pruned-prefill time to first token (tokengate_amd.prefill.prefill_batch) on a random-init
    Qwen3-1.7B-shaped decoder (28 layers, d 2048, 16/8 heads, head_dim 128, FFN 6144, vocab 151936,
    RoPE theta 1e6, bf16), gate at layer 1 (scoring head Linear(2048->256)->SiLU->Linear(256->1)),
    prompts of uniform random ids already on the device, state span = prompt minus a 64-token
    prefix and a 256-token suffix.  Protocol of the reference's TTFT bench: sync, perf_counter,
    prefill through the first token, sync; median of `reps` after one warmup.  The "_branch" line
    runs the finalized gate instead: the MLP scoring branch (a copy of the gate layer's SwiGLU, I
    6144, with an absorbed (1, I) readout row) on the gate layer's attention boundary, the gate
    layer's MLP on the kept rows only, scaled softmax in Phase 2.  decode_ms_per_token (32k, K=2000
    and K=all, ragged8): greedy decode steps after a prefill run with 16 rows of decode headroom in
    every cache, median of 8 after 2 warmup steps."""
    import statistics
    import torch
    from tokengate_amd import decoder as dec
    from tokengate_amd import gate as G
    from tokengate_amd import prefill as P
    shape = dec.QWEN3_1P7B
    wts = dec.random_decoder(shape, seed=0, device=dev)
    head = G.random_head(shape.n_layers - 2, shape.n_heads, seed=5, device=dev)
    g = torch.Generator().manual_seed(7)
    out = {}

    branch = G.random_branch_head(wts, 1, seed=5)

    def decode_ms(r, head, steps=8, warmup=2, graph=True):
        """Greedy decode after the prefill r (tokengate_amd.decode.DecodeState.step, all 28 layers,
        attention over the pruned caches; graph=True: steps after the first replay one captured
        HIP graph of the step): median milliseconds per token over `steps` steps."""
        from tokengate_amd.decode import DecodeState
        st = DecodeState(wts, head, 1, r, steps + warmup + 1, graph=graph)
        cur = r.first_tokens
        ts = []
        for i in range(steps + warmup):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            cur = st.step(cur)
            torch.cuda.synchronize()
            if i >= warmup:
                ts.append((time.perf_counter() - t0) * 1e3)
        del st
        return round(statistics.median(ts), 3)

    def run(name, lens, Ks, head=head, decode=False):
        ids = [torch.randint(0, shape.vocab, (n,), generator=g).to(dev) for n in lens]
        starts = [64] * len(lens)
        ends = [n - 256 for n in lens]
        fn = lambda: P.prefill_batch(wts, head, ids, starts, ends, 1, Ks)
        times = P.ttft_ms(fn, reps=reps, warmup=1)
        # the measured prefill leaves decode headroom in every cache (decode appends in place)
        r = P.prefill_batch(wts, head, ids, starts, ends, 1, Ks, phase_timing=True,
                            decode_headroom=16 if decode else 0)
        out[name] = {"ttft_ms": round(statistics.median(times), 3), "reps_ms": [round(t, 3) for t in times],
                     "prompt_tokens": sum(lens), "kept_tokens": r.cu_kept[-1],
                     "phase_ms": {k: round(v, 3) for k, v in r.phase_ms.items()}}
        if decode:
            out[name]["decode_ms_per_token"] = decode_ms(r, head)
            out[name]["decode_eager_ms_per_token"] = decode_ms(r, head, graph=False)
        if r.cu_kept[-1] <= 32768:
            # Phase 2 replayed from a captured graph (captured during the warm-up call)
            graphs = P.Phase2Graphs()
            fg = lambda: P.prefill_batch(wts, head, ids, starts, ends, 1, Ks, phase2_graphs=graphs)
            tg = P.ttft_ms(fg, reps=reps, warmup=1)
            rg = P.prefill_batch(wts, head, ids, starts, ends, 1, Ks, phase_timing=True, phase2_graphs=graphs)
            out[name]["ttft_ms_phase2_graph"] = round(statistics.median(tg), 3)
            out[name]["phase2_ms_graph"] = round(rg.phase_ms["phase2"], 3)
            del graphs, rg
        if len(lens) > 1:
            out[name]["lens"] = lens
            out[name]["K"] = Ks
        del r
        torch.cuda.empty_cache()

    for K in (100, 2000):
        run(f"32k_K{K}", [32768], [K], decode=K == 2000)
    run("32k_Kall", [32768], [10_000_000], decode=True)
    run("32k_K2000_branch", [32768], [2000], head=branch)
    rng = torch.Generator().manual_seed(17)
    lens = [int(x) for x in torch.randint(16384, 131073, (8,), generator=rng)]
    Ks = [[100, 500, 2000, 4000][int(i)] for i in torch.randint(0, 4, (8,), generator=rng)]
    run("ragged8", lens, Ks, decode=True)
    del wts
    torch.cuda.empty_cache()
    return out


def prefill_trace_run(dev, runs=8):
    """The 32k / K=2000 gated prefill of bench_ttft (same decoder, head and prompt generator), run
    `runs` times back to back with no other work, for a per-kernel trace of one prefill."""
    import torch
    from tokengate_amd import decoder as dec
    from tokengate_amd import gate as G
    from tokengate_amd import prefill as P
    shape = dec.QWEN3_1P7B
    wts = dec.random_decoder(shape, seed=0, device=dev)
    head = G.random_head(shape.n_layers - 2, shape.n_heads, seed=5, device=dev)
    g = torch.Generator().manual_seed(7)
    ids = [torch.randint(0, shape.vocab, (32768,), generator=g).to(dev)]
    for i in range(runs):
        P.prefill_batch(wts, head, ids, [64], [32768 - 256], 1, [2000])
        torch.cuda.synchronize()
        print(f"prefill {i + 1}/{runs} done", flush=True)


def clock_study_run(dev, runs=3):
    """The 32k key-bias forward alone (10 launches, the benchmark's inputs), then `runs` gated
    prefills at 32k / K=2000 (prefill_trace_run's), then the forward alone again (5 launches): a
    per-dispatch GRBM_GUI_ACTIVE / duration profile compares the clock of the forward with that of
    the prefill's own Phase-1 attention launches."""
    import torch
    S, H, Hkv = 32768, 16, 8
    q, k, v, bias_raw, scale = make_inputs(S, H, Hkv, 3.0, 2, dev, qkv_scale=1.0 / math.sqrt(128))
    op = torch.ops.recursive_kvs.fa2_keybias_fwd
    for _ in range(10):
        op(q, k, v, bias_raw, scale, True)
    torch.cuda.synchronize()
    print("clock study: forward alone x10 done", flush=True)
    prefill_trace_run(dev, runs=runs)
    for _ in range(5):
        op(q, k, v, bias_raw, scale, True)
    torch.cuda.synchronize()
    print("clock study: forward alone x5 done", flush=True)


def decode_trace_run(dev, steps=30):
    """Greedy decode after the 32k / K=2000 gated prefill of prefill_trace_run (graph replay of the
    whole step after the first), for a per-kernel trace of the decode step; prints ms per token."""
    import statistics
    import torch
    from tokengate_amd import decoder as dec
    from tokengate_amd import gate as G
    from tokengate_amd import prefill as P
    from tokengate_amd.decode import DecodeState
    shape = dec.QWEN3_1P7B
    wts = dec.random_decoder(shape, seed=0, device=dev)
    head = G.random_head(shape.n_layers - 2, shape.n_heads, seed=5, device=dev)
    g = torch.Generator().manual_seed(7)
    ids = [torch.randint(0, shape.vocab, (32768,), generator=g).to(dev)]
    r = P.prefill_batch(wts, head, ids, [64], [32768 - 256], 1, [2000], decode_headroom=steps + 4)
    st = DecodeState(wts, head, 1, r, steps + 3, graph=True)
    cur = r.first_tokens
    ts = []
    for i in range(steps + 2):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        cur = st.step(cur)
        torch.cuda.synchronize()
        if i >= 2:
            ts.append((time.perf_counter() - t0) * 1e3)
    print(json.dumps({"decode_ms_per_token": round(statistics.median(ts), 3), "steps": steps}), flush=True)


def cpu_model() -> str:
    """The host CPU's model name (from /proc/cpuinfo), or 'unknown'."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def gate_counter_run(dev, reps=5):
    """Eager launches of the gate kernels for a per-dispatch counter profile: scoring at 32k and over
    the ragged8 batch's rows; at 32k for K in {100, 500, 2000} and on the ragged8 batch, the
    single-workgroup top-K, the pack, and
    the multi-workgroup selection + pack (gate.select_pack), `reps` times each; then three plain
    1 GiB device copies (counter calibration)."""
    import torch
    from tokengate_amd import gate
    S, d, s, e = 32768, 2048, 64, 32512
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(S, d, generator=g, device=dev).to(torch.bfloat16)
    a1 = math.sqrt(6.0 / (d + 256))
    w1 = ((torch.rand(256, d, generator=g, device=dev) * 2 - 1) * a1).to(torch.bfloat16)
    w2 = (torch.rand(256, generator=g, device=dev) * 2 - 1) * math.sqrt(6.0 / 257)
    b1 = torch.zeros(256, device=dev)
    scores = torch.zeros(S, dtype=torch.float32, device=dev)
    w1k = gate.ktile_w1(w1)
    for _ in range(reps):
        gate.score_mlp(x[s:e], w1, b1, w2, 0.0, out=scores[s:e], w1_ktiled=w1k)
    torch.cuda.synchronize()
    print("gate counters: scoring done", flush=True)
    kv = [torch.randn(S, 8, 128, generator=g, device=dev).to(torch.bfloat16) for _ in range(4)]

    def one(sc, p, srcs, tag):
        T = p.total_kept
        outs = [torch.empty(T, *t.shape[1:], dtype=t.dtype, device=dev) for t in srcs]
        pos = torch.empty(T, dtype=torch.int64, device=dev)
        bias = torch.empty(T, dtype=torch.float32, device=dev)
        pairs = list(zip(srcs, outs))
        for _ in range(reps):
            keep, ss = gate.select_keep(sc, p)
            gate.pack(keep, p, pairs, positions=pos, bias_src=sc, sumsq=ss, bias_out=bias)
        for _ in range(reps):
            gate.select_pack(sc, p, pairs, positions=pos, bias_out=bias)
        torch.cuda.synchronize()
        print(f"gate counters: {tag} done ({T} kept)", flush=True)

    for K in (100, 500, 2000):
        one(scores, gate.plan([0], [S], [s], [e], [K], dev), [x] + kv, f"32k K{K}")
    del x, kv
    lens = [114517, 57946, 113394, 80391, 42386, 123699, 106754, 74151]
    Ks = [2000, 4000, 100, 4000, 100, 100, 4000, 500]
    R = sum(lens)
    sc8 = torch.randn(R, generator=g, device=dev).to(torch.bfloat16).float()
    x8 = torch.randn(R, 2048, generator=g, device=dev).to(torch.bfloat16)
    kv8 = [torch.randn(R, 8, 128, generator=g, device=dev).to(torch.bfloat16) for _ in range(4)]
    sc8_head = torch.empty(R, dtype=torch.float32, device=dev)
    for _ in range(reps):
        gate.score_mlp(x8, w1, b1, w2, 0.0, out=sc8_head, w1_ktiled=w1k)
    torch.cuda.synchronize()
    print("gate counters: ragged8 scoring done", flush=True)
    p8 = gate.plan([sum(lens[:b]) for b in range(8)], lens, [64] * 8, [L - 256 for L in lens], Ks, dev)
    one(sc8, p8, [x8] + kv8, "ragged8")
    del x8, kv8
    src = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("gate counters: calibration copies done", flush=True)


def cpu_threads() -> int:
    """Host threads for the CPU legs: the job's CPU share (OMP_NUM_THREADS when the environment
    sets it, as on a machine shared by several jobs), else every core this process may run on
    (len(os.sched_getaffinity(0))); the report gives both counts."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    n = len(os.sched_getaffinity(0))
    return max(1, min(n, int(env))) if env.isdigit() and int(env) > 0 else n


def _median_s(fn, reps=3, warmup=1):
    import statistics
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_prune_baseline():
    """The reference's CPU pruning path (oracle.cpu_path.prune: torch.topk -> sort -> cat ->
    index_select, gate_forward.py:1396-1470) at the 32k gate workload for each K: the state span's
    fp32 scores, the hidden rows (32768 x 2048 bf16) and 2 layers of K/V (32768 x 8 x 128 bf16)
    gathered; torch on the host's threads, median of 3 after 1 warmup."""
    import torch
    from oracle import cpu_path as cp
    threads = cpu_threads()
    torch.set_num_threads(threads)
    S, s, e = 32768, 64, 32512
    g = torch.Generator().manual_seed(5)
    sc = torch.randn(e - s, generator=g)
    hid = torch.randn(S, 2048, generator=g).to(torch.bfloat16)
    kvs = [torch.randn(S, 8, 128, generator=g).to(torch.bfloat16) for _ in range(4)]
    res = {}
    for K in (100, 500, 2000):
        t = _median_s(lambda: cp.prune(sc, K, s, e, S, [hid] + kvs))
        res[f"K{K}_ms"] = round(t * 1e3, 3)
    res.update({"cores": threads, "affinity_cores": len(os.sched_getaffinity(0)), "kind": "port",
                "cpu_model": cpu_model(),
                "sample": "reference CPU pruning path restated in torch (topk, sort, cat, index_select of "
                          "hidden + 2 layers' K/V), 32k / K in {100, 500, 2000}, median of 3"})
    return res


def cpu_baseline(seconds):
    """The reference's CPU attention path (oracle.cpu_path.sdpa_chunked: the SDPA compatibility
    prefill, chunks of 128 query rows, additive float mask = key bias + causal -inf, K/V heads
    repeated for GQA; sdpa_compat.py:6-37) in float32 on the host's threads.  value: a bounded
    sample of the 32k workload -- the last query chunks (each over every key it sees), as many as
    fit in about `seconds` -- in causal-counted TFLOP/s; c1: the whole 4k workload (batch 1, 16/8
    heads, bias log(sigmoid(z)) z~N(0,2)), median of 3 after 1 warmup."""
    import torch
    from oracle import cpu_path as cp
    threads = cpu_threads()
    torch.set_num_threads(threads)
    H, Hkv, D = 16, 8, 128

    def inputs(S, sigma, seed):
        g = torch.Generator().manual_seed(seed)
        q = torch.randn(1, H, S, D, generator=g) / math.sqrt(D)
        k = torch.randn(1, Hkv, S, D, generator=g) / math.sqrt(D)
        v = torch.randn(1, Hkv, S, D, generator=g)
        b = torch.nn.functional.logsigmoid(torch.randn(1, S, generator=g) * sigma)
        return q, k, v, b

    q, k, v, b = inputs(4096, 2.0, 0)
    t1 = _median_s(lambda: cp.sdpa_chunked(q, k, v, b))
    c1 = {"ms": round(t1 * 1e3, 1), "tflops": round(causal_flops(1, H, 4096) / t1 / 1e12, 4)}
    S = 32768
    q, k, v, b = inputs(S, 3.0, 2)
    chunk, done, flop = 128, 0, 0.0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds and done < S:
        hi = S - done
        cp.sdpa_chunked(q, k, v, b, rows=range(hi - chunk, hi))
        flop += 4.0 * H * D * sum(r + 1 for r in range(hi - chunk, hi))
        done += chunk
    dt = time.perf_counter() - t0
    return {"value": round(flop / dt / 1e12, 6), "unit": "TFLOP/s", "cores": threads,
            "affinity_cores": len(os.sched_getaffinity(0)), "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"reference CPU attention path restated in torch (chunked SDPA, float mask, GQA by "
                      f"repeat), float32: the last {done} query rows of the 32k causal workload in "
                      f"{dt:.1f} s ({flop:.3e} causal FLOP)",
            "c1_4k_whole": c1}


def traffic_from_profile():
    """HBM bytes per launch of the forward kernel at the 32k workload, from the committed
    rocprofv3 counter summary (line 'hbm_bytes_per_launch: N'), or None."""
    path = os.path.join(ROOT, "profiles", "keybias_fwd_32k_hbm_counters.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("hbm_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run three plain 1 GiB device copies (counter calibration for HBM bytes)")
    ap.add_argument("--gate-counters", action="store_true",
                    help="only run eager launches of the gate kernels (for a per-dispatch counter profile)")
    ap.add_argument("--bwd-only", action="store_true",
                    help="only run the B4 x 8192 backward (for a per-dispatch counter profile)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only run greedy decode steps after one 32k / K=2000 prefill (for a kernel trace)")
    ap.add_argument("--ttft-only", action="store_true",
                    help="only run 8 back-to-back gated prefills at 32k / K=2000 (for a kernel trace)")
    ap.add_argument("--clock-study", action="store_true",
                    help="only run the 32k forward alone, 3 gated prefills at 32k / K=2000, then the forward "
                         "alone again (for a per-dispatch clock profile)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the path is timed on one GPU's share of the work, with no "
              "collectives (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    from tokengate_amd.fa2bias import keybias  # noqa: F401  (registers the custom ops)
    dev = torch.device("cuda:0")
    if args.ttft_only:
        prefill_trace_run(dev)
        return
    if args.clock_study:
        clock_study_run(dev)
        return
    if args.gate_counters:
        gate_counter_run(dev)
        return
    if args.decode_only:
        decode_trace_run(dev)
        return
    if args.bwd_only:
        print(json.dumps({"bwd_8k_b4": bench_bwd(dev, iters=3)}), flush=True)
        return

    S, H, Hkv = 32768, 16, 8
    q, k, v, bias_raw, scale = make_inputs(S, H, Hkv, 3.0, 2, dev, qkv_scale=1.0 / math.sqrt(128))
    flops = causal_flops(1, H, S)
    ms_step, kern_ms = time_fwd(q, k, v, bias_raw, scale, args.steps, args.warmup,
                                clock_warmup=CLOCK_WARMUP_LAUNCHES)
    value = flops / (ms_step * 1e-3) / 1e12
    achieved = flops / (kern_ms * 1e-3) / 1e12

    extra = {"kernel_ms_32k": round(kern_ms, 4), "clock_warmup_launches": CLOCK_WARMUP_LAUNCHES}
    if not args.no_extra:
        q1, k1, v1, b1, s1 = make_inputs(4096, H, Hkv, 2.0, 0, dev, prefix=0, suffix=0)
        _, k1ms = time_fwd(q1, k1, v1, b1, s1, 20, 5)
        extra["fwd_4k_tflops"] = round(causal_flops(1, H, 4096) / (k1ms * 1e-3) / 1e12, 2)
        extra["fwd_4k_kernel_ms"] = round(k1ms, 4)
        del q1, k1, v1, b1
        extra["bwd_8k_b4"] = bench_bwd(dev)
        extra["gate_32k"] = bench_gate(dev)
        extra["gate_ragged8"] = bench_gate_ragged8(dev)
        if args.cpu_seconds > 0:
            extra["gate_32k"]["cpu_prune_baseline"] = cpu_prune_baseline()
        extra["ttft"] = bench_ttft(dev)

    if args.calib_copy:
        src = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    del q, k, v, bias_raw
    cpu = cpu_baseline(args.cpu_seconds) if args.cpu_seconds > 0 else None
    line = {
        "metric": "key-bias attn TFLOP/s at 32k bf16 (% MFMA peak); pruned-prefill TTFT ms",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "key-bias attention forward, causal GQA, 32k context",
                   "batch": 1, "seq_len": S, "heads": H, "kv_heads": Hkv, "head_dim": 128,
                   "bias": "log(sigmoid(z)), z~N(0,3), 0 on [0,64) and [32512,32768), broadcast over heads",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic_from_profile()},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
