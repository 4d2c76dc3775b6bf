"""Gated prefill of a ragged batch: Phase 1 -> score -> top-K keep -> pack -> Phase 2 -> first token.

Follows prefill_batch_for_decode (tokengate/e2e_gate/gate_module/gate_forward.py:1280-1580):
layers 0..gate_layer run over every prompt token (:1334-1366); the gate scores the gate layer's
hidden state and keeps, per sequence, its prefix, the K_clamped = max(1, min(K, n_art))
highest-scoring state tokens in original order, and its suffix (:1378-1421); the kept hidden rows,
their original positions and their gate bias are gathered (:1435-1470); layers gate_layer+1..
run on the kept rows with RoPE at the original positions and the per-(layer, head) gate bias
(:1478-1560, _apply_gate_bias :588-662); the first token is the argmax of the LM head at each
sequence's last row (:1560-1580).  Layers at or below the gate keep their full Phase-1 KV cache
(prune_below_gate=False, the reference default); prune_below_gate=True packs it down to the kept
rows in the same launch that packs the hidden states.  With the finalized gate's MLP scoring
branch (gate.BranchHead) the gate layer is split (split_gate_layer_mlp, gate_forward.py:345-357,
:1362-1372): Phase 1 ends at the gate layer's attention residual, the branch scores that boundary,
and the gate layer's own MLP runs on the packed kept rows only, at Phase-2 entry (:1476-1478).

MI355X layout: the batch is never padded.  Phase 1 packs all prompts back to back (cu_seqlens)
and runs one varlen attention launch per layer; the keep lists of all sequences come from one
multi-workgroup selection (gate.select_pack: every state span cut into chunks of 4096 scores) and
every gather from one pack launch; Phase 2 runs the packed kept rows, with
the -1e9 pad-slot bias of the reference replaced by the cu_seqlens boundaries.  Every size is
known on the host from the prompt lengths, spans and K, so nothing synchronises before the
first token.
"""
import math
import time
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import torch

from tokengate_amd import gate as G
from tokengate_amd.decoder import (CacheGap, DecoderWeights, LayerKV, Ragged, Workspace, alloc_kv, argmax_rows, h2d,
                                   logits_last, mlp_sublayer, run_layers)


@dataclass
class PrefillResult:
    first_tokens: torch.Tensor        # (B,) int64 on the device
    logits: torch.Tensor              # (B, vocab) bf16: the LM head at each sequence's last kept row
    kept_positions: torch.Tensor      # (total_kept,) int64, packed (cu_kept layout)
    cu_kept: List[int]
    n_kept: List[int]
    k_clamped: List[int]
    kv: List[LayerKV]                 # per layer: Phase-1 rows (cu_prompt) at/below the gate, kept rows above
    cu_prompt: List[int]
    kept_bias: torch.Tensor           # (total_kept,) fp32 normalised gate score (0 on prefix / suffix)
    kept_ratio: Optional[torch.Tensor] = None   # (total_kept,) fp32 scaled-softmax ratio r (ssmax heads)
    phase2_bias: Optional[torch.Tensor] = None  # (L2, H, total_kept) fp32 raw-unit key bias of each Phase-2 layer
    phase_ms: Dict[str, float] = field(default_factory=dict)
    capture: Optional[dict] = None
    # decode headroom: every layer's cache keeps `decode_headroom` free rows after each sequence
    # (cache_below: layers at / below the gate, cache_above: Phase-2 layers); phase2_bias_seq
    # (L2, B, H, max_kept + decode_headroom) fp32 is each Phase-2 layer's key bias by sequence and
    # key index, 0 past the kept rows (the generated keys' bias)
    decode_headroom: int = 0
    cache_below: Optional[CacheGap] = None
    cache_above: Optional[CacheGap] = None
    phase2_bias_seq: Optional[torch.Tensor] = None


def _cat_ids(ids_list: Sequence, device) -> torch.Tensor:
    if all(torch.is_tensor(x) for x in ids_list):
        return torch.cat([x.reshape(-1).to(device=device, dtype=torch.long) for x in ids_list])
    flat = [int(t) for ids in ids_list for t in (ids.tolist() if torch.is_tensor(ids) else ids)]
    return h2d(torch.tensor(flat, dtype=torch.long), device)


class Phase2Graphs:
    """Captured HIP graphs of the Phase-2 layer loop (the reference's whole-loop graph replay,
    phase2_graph.py:170-223, with bucketed sizes as set_phase2_bucket, gate_forward.py:531-546).

    One graph per (number of sequences, rows rounded up to `bucket_rows`, longest sequence rounded
    up to `bucket_len`): its static inputs are the packed kept rows, their positions, cu_seqlens,
    the per-layer bias table and the per-layer query scales; the varlen attention reads
    cu_seqlens from device memory, so every batch of that geometry replays the same graph.  Rows
    past the last sequence are zero and belong to no sequence (attention never visits them).
    Replays are stream-ordered on the current stream; the returned tensors are views of the
    graph's static buffers, valid until the next replay of the same graph."""

    def __init__(self, bucket_rows: int = 64, bucket_len: int = 64):
        self.bucket_rows = bucket_rows
        self.bucket_len = bucket_len
        self.graphs = {}

    @staticmethod
    def _up(n: int, b: int) -> int:
        return (n + b - 1) // b * b

    def run(self, wts: DecoderWeights, layer_ids: List[int], hs: torch.Tensor, positions: torch.Tensor,
            cu_dev: torch.Tensor, biases_all: torch.Tensor, q_head: Optional[torch.Tensor], mlp_rows: int,
            q_row: Optional[torch.Tensor] = None, cu_kept: Optional[List[int]] = None, gap: int = 0):
        """biases_all (L2, nseq, H, >= max_kept) fp32 raw-unit key bias; q_head (L2, H) / q_row (T2,)
        the query factors (None when absent); gap > 0: the caches keep `gap` free rows after each
        sequence (cu_kept, the host copy of cu_dev, is then required) and are returned whole."""
        dev = hs.device
        nseq = cu_dev.numel() - 1
        T2 = hs.shape[0]
        max_kept = max(cu_kept[b + 1] - cu_kept[b] for b in range(nseq)) if cu_kept is not None \
            else biases_all.shape[-1]
        Tb, Lb = self._up(T2, self.bucket_rows), self._up(max_kept, self.bucket_len)
        if gap and cu_kept is None:
            raise ValueError("Phase2Graphs.run: a cache gap needs the host cu_kept")
        # the graph reads the weights' and workspaces' memory: a key per weights object (held
        # alive by the entry) and per MLP chunking
        key = (id(wts), nseq, Tb, Lb, tuple(layer_ids), q_head is not None, q_row is not None, int(mlp_rows),
               int(gap))
        ent = self.graphs.get(key)
        if ent is None:
            ent = self._capture(wts, layer_ids, nseq, Tb, Lb, q_head is not None, q_row is not None, mlp_rows, dev,
                                int(gap))
            ent["wts"] = wts
            self.graphs[key] = ent
        if q_row is not None:
            ent["rs"][:T2].copy_(q_row)
        ent["x"][:T2].copy_(hs)
        ent["x"][T2:].zero_()
        ent["pos"][:T2].copy_(positions)
        ent["pos"][T2:].zero_()
        ent["cu"].copy_(cu_dev)
        ent["bias"][..., :max_kept].copy_(biases_all[..., :max_kept])
        if q_head is not None:
            ent["qs"].copy_(q_head)
        if gap:
            cg = CacheGap.build(cu_kept, gap, dev, pad_rows=Tb - T2)
            sc = ent["cache"]
            sc.seg_dev.copy_(cg.seg_dev)
            sc.used_dev.copy_(cg.used_dev)
            sc.rows_dev.copy_(cg.rows_dev)
        ent["graph"].replay()
        if gap:
            return ent["out"][:T2], {l: ent["kv"][l] for l in layer_ids}
        return ent["out"][:T2], {l: LayerKV(ent["kv"][l].k[:T2], ent["kv"][l].v[:T2]) for l in layer_ids}

    def _capture(self, wts, layer_ids, nseq, Tb, Lb, with_qs, with_rs, mlp_rows, dev, gap=0):
        shape = wts.shape
        L2 = len(layer_ids)
        x = torch.zeros(Tb, shape.d_model, dtype=torch.bfloat16, device=dev)
        pos = torch.zeros(Tb, dtype=torch.int64, device=dev)
        cu = torch.zeros(nseq + 1, dtype=torch.int32, device=dev)
        cu[-1] = Tb
        bias = torch.zeros(L2, nseq, shape.n_heads, Lb, dtype=torch.float32, device=dev)
        qs = torch.ones(L2, shape.n_heads, dtype=torch.float32, device=dev) if with_qs else None
        rs = torch.ones(Tb, dtype=torch.float32, device=dev) if with_rs else None
        cache = None
        if gap:
            # static cache geometry, as the static cu (every row in the last sequence) until a
            # replay copies the batch's own; the caches hold the bucket's rows plus every gap
            cache = CacheGap.build([0] * nseq + [Tb], gap, dev)
        kv: List[Optional[LayerKV]] = [None] * shape.n_layers
        for l in layer_ids:
            kv[l] = alloc_kv(shape, Tb + nseq * gap, dev)
        ws = Workspace(shape, Tb, dev, mlp_rows=mlp_rows)
        geo = Ragged([0, Tb], cu, pos, Lb, cache=cache)
        biases = {l: bias[j] for j, l in enumerate(layer_ids)}
        q_scales = {l: qs[j] for j, l in enumerate(layer_ids)} if with_qs else None
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            run_layers(wts, layer_ids, x, geo, ws, kv, biases=biases, q_scales=q_scales, q_row_scale=rs)   # warm-up
        torch.cuda.current_stream(dev).wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = run_layers(wts, layer_ids, x, geo, ws, kv, biases=biases, q_scales=q_scales, q_row_scale=rs)
        return dict(graph=g, x=x, pos=pos, cu=cu, bias=bias, qs=qs, rs=rs, kv=kv, ws=ws, out=out, cache=cache)


@torch.no_grad()
def prefill_batch(wts: DecoderWeights, head, ids_list: Sequence, art_starts: Sequence[int],
                  art_ends: Sequence[int], gate_layer: int, K, prune_below_gate: bool = False,
                  phase_timing: bool = False, capture: bool = False, mlp_rows: int = 131072,
                  phase2_graphs: Optional[Phase2Graphs] = None, decode_headroom: int = 0) -> PrefillResult:
    """ids_list: B prompts (lists of ints or 1-D tensors); the state span of prompt b is
    [art_starts[b], art_ends[b]); K: scalar or per-prompt list; head: gate.ScoringHead or
    gate.BranchHead (split gate layer).  phase2_graphs: replay Phase 2
    from captured graphs (captured on first use per geometry); the Phase-2 KV caches are then views
    of the graph's buffers, valid until its next replay.  decode_headroom: every layer's KV cache
    is laid out with that many free rows after each sequence (written there by the prefill's own
    launches and the pack), so that decode appends in place.  Raises RuntimeError (after queueing
    every launch, when the selection's launches have finished) if the keep-list selection reported
    an error: the result would be built on invalid keep lists."""
    shape = wts.shape
    dev = wts.device
    B = len(ids_list)
    if B == 0:
        raise ValueError("empty batch")
    n_layers = shape.n_layers
    if not 0 <= gate_layer < n_layers - 1:
        raise ValueError(f"gate_layer {gate_layer} must leave at least one layer above it")
    if head.gate_scale.shape != (n_layers - gate_layer - 1, shape.n_heads):
        raise ValueError("head.gate_scale must be (layers above the gate, num_heads)")
    lens = [int(x.numel()) if torch.is_tensor(x) else len(x) for x in ids_list]
    if min(lens) < 1:
        raise ValueError("every prompt needs at least one token")
    gap = int(decode_headroom)
    if gap < 0:
        raise ValueError("decode_headroom must be >= 0")
    ev = [] if phase_timing else None

    def mark(name):
        if ev is not None:
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            ev.append((name, e))

    cap = {"phase1": [], "phase2": []} if capture else None
    mark("phase1")
    ids = _cat_ids(ids_list, dev)
    geo1 = Ragged.from_lengths(lens, dev)
    if gap and not prune_below_gate:    # the Phase-1 caches are the decode caches of these layers
        geo1.cache = CacheGap.build(geo1.cu, gap, dev)
    T = geo1.total
    x = torch.nn.functional.embedding(ids, wts.embed)
    ws1 = Workspace(shape, T, dev, mlp_rows=mlp_rows)
    kv: List[Optional[LayerKV]] = [None] * n_layers
    for i in range(gate_layer + 1):
        kv[i] = alloc_kv(shape, geo1.kv_rows, dev)
    split = bool(getattr(head, "split_gate_layer", False))
    h = run_layers(wts, range(gate_layer + 1), x, geo1, ws1, kv, capture=cap["phase1"] if cap else None,
                   attn_only_last=split)
    del x

    mark("score")
    if split:
        scores = head.scores_from_boundary(h, wts.layers[gate_layer].ln2, shape.rms_eps, normed=ws1.normed,
                                           chunk_rows=mlp_rows)
    else:
        scores = head.scores(h)

    mark("select+pack")
    threshold = getattr(head, "selection_mode", "topk") == "threshold"
    if threshold:
        # sample-dependent kept counts (one host synchronisation); K is unused, as in the reference
        p, sel_scores, _, sel_sumsq, _ = G.threshold_plan(scores, geo1.cu[:-1], lens, art_starts, art_ends, head,
                                                           dev)
    else:
        p = G.plan(geo1.cu[:-1], lens, art_starts, art_ends, K, dev)
    T2 = p.total_kept
    hs = torch.empty(T2, shape.d_model, dtype=h.dtype, device=dev)
    kept_pos = torch.empty(T2, dtype=torch.int64, device=dev)
    kept_bias = torch.empty(T2, dtype=torch.float32, device=dev)
    pairs = [(h, hs)]
    B_ = len(lens)
    if prune_below_gate:
        for i in range(gate_layer + 1):
            nk = alloc_kv(shape, T2 + B_ * gap, dev)
            pairs += [(kv[i].k, nk.k, gap), (kv[i].v, nk.v, gap)]
            kv[i] = nk
    # the selection's error word comes back with an asynchronous copy; it is checked once every
    # launch of the prefill is queued (the GPU then never waits for the host)
    err_host = torch.zeros(1, dtype=torch.int32, pin_memory=True)
    if threshold:
        keep = G.select_pack(sel_scores, p, pairs, positions=kept_pos, error_out=err_host)
        G.pack(keep, p, [], bias_src=scores, sumsq=sel_sumsq, bias_out=kept_bias)
    else:
        keep = G.select_pack(scores, p, pairs, positions=kept_pos, bias_out=kept_bias, error_out=err_host)
    err_ev = torch.cuda.Event()
    err_ev.record()
    sel_stream = torch.cuda.current_stream().cuda_stream
    if cap is not None:
        cap["h1"] = h
    del h, ws1, pairs

    mark("phase2")
    ws2 = None
    if split:                       # the gate layer's MLP on the kept rows (Phase-2 entry)
        ws2 = Workspace(shape, T2, dev, mlp_rows=mlp_rows)
        if cap is not None:
            cap["hs_boundary"] = hs
        hs = mlp_sublayer(wts, gate_layer, hs, ws2)
    max_kept = max(p.n_kept)
    ratio = G.ssmax_ratio_rows(kept_pos, p.cu_kept) if head.ssmax else None   # (T2,)
    bias_rows, q_head, q_row = head.phase2_tables(kept_bias, ratio, 1.0 / math.sqrt(shape.head_dim))
    # per-sequence view of the packed rows' bias: row b, column t <- packed row cu_kept[b] + t,
    # 0 past the sequence's kept rows (the decode's generated keys; Phase 2 never reads them)
    W = max_kept + gap
    t_ = torch.arange(W, dtype=torch.int64)[None, :]
    st = torch.tensor(p.cu_kept[:-1], dtype=torch.int64)[:, None]
    nk_ = torch.tensor(p.n_kept, dtype=torch.int64)[:, None]
    idx_d = h2d(torch.where(t_ < nk_, st + t_, T2), dev)                      # T2: the zero column
    bias_z = torch.cat([bias_rows, bias_rows.new_zeros(bias_rows.shape[0], bias_rows.shape[1], 1)], -1)
    biases_all = bias_z[:, :, idx_d].permute(0, 2, 1, 3).contiguous()          # (L2, B, H, W)
    cu2_dev = h2d(torch.tensor(p.cu_kept, dtype=torch.int32), dev)
    above = list(range(gate_layer + 1, n_layers))
    cache2 = None
    if phase2_graphs is not None and cap is None:
        h2, kv2 = phase2_graphs.run(wts, above, hs, kept_pos, cu2_dev, biases_all, q_head, mlp_rows, q_row,
                                    cu_kept=p.cu_kept, gap=gap)
        for l in above:
            kv[l] = kv2[l]
        if gap:
            cache2 = CacheGap.build(p.cu_kept, gap, dev)
    else:
        cache2 = CacheGap.build(p.cu_kept, gap, dev) if gap else None
        geo2 = Ragged(p.cu_kept, cu2_dev, kept_pos, max_kept, cache=cache2)
        biases = {l: biases_all[j] for j, l in enumerate(above)}
        qs = {l: q_head[j] for j, l in enumerate(above)} if q_head is not None else None
        for l in above:
            kv[l] = alloc_kv(shape, geo2.kv_rows, dev)
        ws2 = ws2 if ws2 is not None else Workspace(shape, T2, dev, mlp_rows=mlp_rows)
        h2 = run_layers(wts, above, hs, geo2, ws2, kv, biases=biases, q_scales=qs,
                        capture=cap["phase2"] if cap else None, q_row_scale=q_row)

    mark("head")
    last = h2d(torch.tensor(p.cu_kept[1:], dtype=torch.int64).sub_(1), dev)
    logits = logits_last(wts, h2, last)
    first = argmax_rows(logits)
    mark("end")
    err_ev.synchronize()
    G.raise_select_error(int(err_host[0]), dev, sel_stream)
    phase_ms = {}
    if ev is not None:
        torch.cuda.synchronize()
        for (n0, e0), (_, e1) in zip(ev[:-1], ev[1:]):
            phase_ms[n0] = e0.elapsed_time(e1)
    if cap is not None:
        cap.update(scores=scores, keep=keep, hs_packed=hs, h2=h2, logits=logits, biases_all=biases_all,
                   q_head=q_head, q_row=q_row)
    cache1 = None
    if gap:
        cache1 = geo1.cache if not prune_below_gate else CacheGap.build(p.cu_kept, gap, dev)
    return PrefillResult(first, logits, kept_pos, p.cu_kept, p.n_kept, p.k_clamped, kv, geo1.cu, kept_bias, ratio,
                         bias_rows, phase_ms, cap, gap, cache1, cache2, biases_all if gap else None)


def ttft_ms(fn, reps: int = 5, warmup: int = 1) -> List[float]:
    """Time-to-first-token protocol of the reference's TTFT bench (bench_ttft.py:312-359): device
    sync, perf_counter, the whole prefill, device sync; warmup calls first, then `reps` timed
    calls back to back.  Returns every repeat in ms."""
    for _ in range(warmup):
        fn()
    out = []
    for _ in range(reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        out.append((time.perf_counter() - t0) * 1e3)
    return out
