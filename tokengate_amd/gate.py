"""Gate path host API: scoring, order-preserving top-K keep lists and the ragged pack.

Mirrors the selection and prune/pack steps of prefill_batch_for_decode
(tokengate/e2e_gate/gate_module/gate_forward.py:1384-1522) — K_clamped = max(1, min(K, n_art))
(:1409-1410), keep = [0, s) + s + sort(topk) + [e, seq_len) (:1417-1421, _keep_indices :77-81),
hidden/KV row gathers at the kept positions (:1454-1522), kept positions (:1457) and the kept rows'
gate bias (build_gate_bias_vectorized :968-1036) — on the gfx950 kernels of csrc/gate.hip.

Differences from the reference, by design: kept rows of all sequences are packed back to back
(cu_seqlens layout) rather than right-padded to the longest; score ties go to the lower position
(torch.topk leaves the order unspecified).  The per-sequence Python loop of the reference becomes
one launch per step for the whole batch.  The threshold selection mode (_select_threshold
:102-125) runs as a count launch, one host synchronisation for the sample-dependent kept counts,
then the same top-K selection over a derived score (threshold_plan).
"""
import ctypes
from dataclasses import dataclass, field
from typing import ClassVar, List, Optional, Sequence, Tuple

import numpy as np
import torch

from tokengate_amd import _lib

RMS_EPS = 1e-6   # E2EGate's normalisation epsilon (e2e_gate_module.py:74)


class PackStream(ctypes.Structure):
    """C layout of tg_pack_stream (include/tokengate_hip.h)."""
    _fields_ = [("src", ctypes.c_void_p), ("dst", ctypes.c_void_p), ("src_row_stride", ctypes.c_int64),
                ("dst_row_stride", ctypes.c_int64), ("src_chunk_stride", ctypes.c_int64),
                ("chunk_bytes", ctypes.c_int32), ("n_chunks", ctypes.c_int32), ("dst_seq_gap", ctypes.c_int64)]


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def k_clamped(K: int, n_art: int) -> int:
    return 0 if n_art <= 0 else max(1, min(int(K), int(n_art)))


@dataclass
class KeepPlan:
    """Host-known geometry of one selection step (no device synchronisation needed)."""
    geom_host: torch.Tensor        # (nseq, 6) int32: row_start, seq_len, art_start, art_end, k_clamped, kept_start
    geom: torch.Tensor             # same, on the device
    n_kept: List[int]
    k_clamped: List[int]
    cu_kept: List[int]             # nseq + 1 (the packed Phase-2 cu_seqlens)
    max_article: int
    sel_kpt: int = 0               # select_pack: keys per thread (0: spans too long for it)
    sel_starts: Optional[List[int]] = None        # select_pack: first chunk of each sequence (nseq + 1)
    sel_starts_dev: Optional[torch.Tensor] = None   # the same, on the device

    @property
    def total_kept(self) -> int:
        return self.cu_kept[-1]


def plan(row_starts: Sequence[int], seq_lens: Sequence[int], art_starts: Sequence[int],
         art_ends: Sequence[int], Ks, device) -> KeepPlan:
    """Geometry of a batch: sequence b's rows are rows row_starts[b] .. + seq_lens[b] of the packed
    score / source tensors; its state span is [art_starts[b], art_ends[b]); it keeps
    K_clamped = max(1, min(K_b, n_art)) state tokens plus its prefix and suffix."""
    n = len(seq_lens)
    Ks = list(Ks) if isinstance(Ks, (list, tuple)) else [int(Ks)] * n
    rows, n_kept, kcs, cu = [], [], [], [0]
    for b in range(n):
        s, e, L = int(art_starts[b]), int(art_ends[b]), int(seq_lens[b])
        if not (0 <= s <= e <= L):
            raise ValueError(f"sequence {b}: state span [{s}, {e}) outside [0, {L}]")
        kc = k_clamped(Ks[b], e - s)
        nk = s + kc + (L - e)
        rows.append([int(row_starts[b]), L, s, e, kc, cu[-1]])
        n_kept.append(nk)
        kcs.append(kc)
        cu.append(cu[-1] + nk)
    if cu[-1] >= 2 ** 31:
        raise ValueError("more than 2^31 kept rows")
    gh = torch.tensor(rows, dtype=torch.int32).reshape(n, 6)
    max_art = max((int(art_ends[b]) - int(art_starts[b]) for b in range(n)), default=0)
    kpt, starts = _select_layout([r[3] - r[2] for r in rows])
    # one host-to-device copy: the geometry table and select_pack's chunk starts
    both = torch.cat([gh.reshape(-1), torch.tensor(starts if starts else [0], dtype=torch.int32)])
    bd = both.pin_memory().to(device, non_blocking=True) if torch.device(device).type == "cuda" else both
    gd = bd[:6 * n].view(n, 6)
    return KeepPlan(gh, gd, n_kept, kcs, cu, max_art, kpt, starts, bd[6 * n:] if starts else None)


def select_keep(scores: torch.Tensor, p: KeepPlan, with_sumsq: bool = True,
                keep_out: Optional[torch.Tensor] = None,
                sumsq_out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Keep lists of every sequence, packed: keep[cu_kept[b] + t] = the t-th kept position of
    sequence b (int64, ascending within a sequence).  Also the per-sequence sum of squared
    article scores (for the RMS-normalised gate bias).  keep_out / sumsq_out: optional
    preallocated outputs (int64 of at least total_kept, float32 of at least num_seqs)."""
    if scores.dtype != torch.float32 or scores.dim() != 1 or not scores.is_contiguous():
        raise RuntimeError("scores must be a contiguous 1-D float32 tensor")
    keep = keep_out if keep_out is not None else torch.empty(p.total_kept, dtype=torch.int64, device=scores.device)
    if keep.dtype != torch.int64 or keep.numel() < p.total_kept or not keep.is_contiguous():
        raise RuntimeError("keep_out must be contiguous int64 with room for every kept row")
    if sumsq_out is not None:
        if sumsq_out.dtype != torch.float32 or sumsq_out.numel() < len(p.n_kept):
            raise RuntimeError("sumsq_out must be float32 with one entry per sequence")
        sumsq = sumsq_out
    else:
        sumsq = torch.empty(len(p.n_kept), dtype=torch.float32, device=scores.device) if with_sumsq else None
    if p.n_kept:
        _lib.call("tg_gate_topk_keep", scores.data_ptr(), p.geom.data_ptr(), len(p.n_kept), p.max_article,
                  keep.data_ptr(), sumsq.data_ptr() if sumsq is not None else None, _stream(scores))
    return keep, sumsq


_SEL_WS = {}          # (device index, stream) -> zero-initialised select-pack workspace (uint8)
_SEL_KPT = (8, 16, 32)
_SEL_MAX_CHUNKS = 64
# Small batches take 4 keys per thread (chunks of 2048 scores): every span at most 32768 scores and
# at most 64 chunks in all.  There the selection's latency chain is shorter with the chunks halved
# (graph replays: one 8k / 32k span 13.4 -> 11.9 / 14.3 -> 13.4 us, 32 spans of 4k 14.7 -> 13.8 us);
# with longer spans or more chunks the last arrival's reads over twice the chunks cost more than the
# shorter first pass saves (one 128k span 17.7 -> 19.3 us, three of 100k 20.3 -> 22.8 us).
_SEL_SMALL_KPT = 4
_SEL_SMALL_SPAN = 32768
_SEL_SMALL_CHUNKS = 64


def _chunk_starts(n_art: Sequence[int], kpt: int) -> List[int]:
    chunk = 512 * kpt
    starts = [0]
    for n in n_art:
        starts.append(starts[-1] + ((n + chunk - 1) // chunk if n > 0 else 0))
    return starts


def _select_layout(n_art: Sequence[int]):
    """Keys per thread and per-sequence chunk starts of tg_gate_select_pack for spans of these
    lengths, or (0, None) when a span needs more than 64 chunks of the largest size."""
    if max(n_art, default=0) <= _SEL_SMALL_SPAN:
        starts = _chunk_starts(n_art, _SEL_SMALL_KPT)
        if starts[-1] <= _SEL_SMALL_CHUNKS:
            return _SEL_SMALL_KPT, starts
    for kpt in _SEL_KPT:
        chunk = 512 * kpt
        if max(n_art, default=0) <= _SEL_MAX_CHUNKS * chunk:
            return kpt, _chunk_starts(n_art, kpt)
    return 0, None


def _sel_workspace(device, stream: int, nseq: int, n_chunks: int):
    """(workspace, seq_capacity, chunk_capacity) for this device and stream, zero-filled when
    created.  Its layout depends on the capacities alone and the kernels leave its counters
    zeroed after every call, so it is reused as is while the batch fits; a larger batch gets a
    new zeroed one with doubled capacities."""
    key = (torch.device(device).index, stream)
    ent = _SEL_WS.get(key)
    if ent is None or ent[1] < nseq or ent[2] < n_chunks:
        seq_cap = max(64, nseq, 2 * ent[1] if ent else 0)
        chunk_cap = max(512, n_chunks, 2 * ent[2] if ent else 0)
        nbytes = int(_lib.load().tg_gate_select_pack_workspace_size(seq_cap, chunk_cap))
        ent = (torch.zeros(nbytes, dtype=torch.uint8, device=device), seq_cap, chunk_cap)
        _SEL_WS[key] = ent
    return ent


def select_pack(scores: torch.Tensor, p: KeepPlan, pairs: Sequence[tuple] = (),
                positions: Optional[torch.Tensor] = None, bias_out: Optional[torch.Tensor] = None,
                keep_out: Optional[torch.Tensor] = None, rms_eps: float = RMS_EPS,
                check: bool = False, error_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """select_keep and pack with the keep lists selected by many workgroups per state span
    (tg_gate_select_pack): the keep lists of every sequence (returned, int64, packed), the rows of
    every (src, dst) pair gathered at them, the kept positions and the kept rows' RMS-normalised
    gate bias.  Spans beyond its limits (more than 64 x 16384 scores) run select_keep then pack.
    The launches' error word (a failed look-back wait, an overrun count, or a kept position outside
    its sequence) stays set in the stream's workspace until reported:
    check: read it back (a host synchronisation), and if set clear it and raise;
    error_out: a (1,) int32 pinned host tensor that receives it by an asynchronous copy after the
    launches (0 when these launches use no workspace); see raise_select_error."""
    if scores.dtype != torch.float32 or scores.dim() != 1 or not scores.is_contiguous():
        raise RuntimeError("scores must be a contiguous 1-D float32 tensor")
    keep = keep_out if keep_out is not None else torch.empty(p.total_kept, dtype=torch.int64, device=scores.device)
    if keep.dtype != torch.int64 or keep.numel() < p.total_kept or not keep.is_contiguous():
        raise RuntimeError("keep_out must be contiguous int64 with room for every kept row")
    if len(pairs) > 16:
        raise RuntimeError("select_pack: at most 16 row streams per launch")
    for t, dt in ((positions, torch.int64), (bias_out, torch.float32)):
        if t is not None and (t.dtype != dt or not t.is_contiguous()):
            raise RuntimeError("select_pack: positions must be contiguous int64, bias_out contiguous float32")
    arr = _streams(pairs, p)
    if error_out is not None:
        if error_out.dtype != torch.int32 or error_out.device.type != "cpu" or error_out.numel() != 1:
            raise RuntimeError("select_pack: error_out must be a (1,) int32 host tensor")
        error_out.zero_()
    if p.total_kept == 0:
        return keep
    if not p.sel_kpt:
        k2, sumsq = select_keep(scores, p, keep_out=keep)
        pack(k2, p, pairs, positions=positions, bias_src=scores, sumsq=sumsq, bias_out=bias_out, rms_eps=rms_eps)
        return k2
    kpt, starts, st_d = p.sel_kpt, p.sel_starts, p.sel_starts_dev
    nseq = len(p.n_kept)
    stream = _stream(scores)
    ws, seq_cap, chunk_cap = _sel_workspace(scores.device, stream, nseq, starts[-1])
    _lib.call("tg_gate_select_pack", scores.data_ptr(), p.geom.data_ptr(), st_d.data_ptr(), nseq, starts[-1], kpt,
              ctypes.cast(arr, ctypes.c_void_p), len(pairs), p.total_kept, keep.data_ptr(),
              positions.data_ptr() if positions is not None else None,
              bias_out.data_ptr() if bias_out is not None else None, float(rms_eps), ws.data_ptr(), seq_cap, chunk_cap,
              stream)
    flag = _error_word(ws)
    if error_out is not None:
        error_out.copy_(flag, non_blocking=True)
    if check:
        raise_select_error(int(flag.item()), scores.device, stream)
    return keep


_SELECT_ERRORS = {1: "a look-back wait timed out", 2: "a chunk's kept count overran its sequence",
                  3: "the gather met a kept position outside its sequence"}


def _error_word(ws: torch.Tensor) -> torch.Tensor:
    off = _lib.SELECT_PACK_ERROR_OFFSET
    return ws[off:off + 4].view(torch.int32)


def raise_select_error(code: int, device, stream: int) -> None:
    """If `code` (the error word select_pack reported) is nonzero, zero the workspace of (device,
    stream) -- the word, and any counter a failed wait left mid-count -- so that the next call starts
    clean, and raise RuntimeError: the keep lists and packed rows of the calls since it was last
    cleared are not valid."""
    if not code:
        return
    ent = _SEL_WS.get((torch.device(device).index, stream))
    if ent is not None:   # (an error path: the device is drained around the clear)
        torch.cuda.synchronize(device)
        ent[0].zero_()
        torch.cuda.synchronize(device)
    raise RuntimeError(f"tg_gate_select_pack: error word {code} "
                       f"({_SELECT_ERRORS.get(code, 'unknown')}); the keep lists are not valid")


_BSTAR: dict = {}


def _f32_of_keys(keys: np.ndarray) -> np.ndarray:
    """fp32 values of ordered keys (the order-preserving uint32 map of non-NaN floats)."""
    k = keys.astype(np.uint64)
    u = np.where(k >= 0x80000000, k - 0x80000000, (~k) & 0xFFFFFFFF).astype(np.uint32)
    return u.view(np.float32)


def sigmoid_threshold(tau: float, device) -> float:
    """b_star: the least fp32 value x with torch.sigmoid(x) >= tau on `device` -- the exact form of
    _select_threshold's `torch.sigmoid(b) >= tau` (gate_forward.py:102-125) that a kernel evaluates
    without a transcendental: b >= b_star.  -inf when every non-NaN value passes, NaN when none does.
    Found over the ordered fp32 values by grid refinement (65537 sigmoid evaluations per step, three
    steps), which relies on torch.sigmoid being non-decreasing; cached per (tau, device)."""
    dev = torch.device(device)
    ck = (float(tau), dev.type, dev.index)
    if ck in _BSTAR:
        return _BSTAR[ck]

    def passes(keys):
        x = torch.from_numpy(_f32_of_keys(keys).copy()).to(dev)
        return (torch.sigmoid(x) >= tau).cpu().numpy()

    lo, hi = 0x007FFFFF, 0xFF800000          # the keys of -inf and +inf
    if passes(np.array([lo]))[0]:
        out = float("-inf")
    elif not passes(np.array([hi]))[0]:
        out = float("nan")
    else:
        while hi - lo > 1:                   # passes(lo) is False, passes(hi) is True
            step = -(-(hi - lo) // 65536)
            grid = np.minimum(lo + step * np.arange(65537, dtype=np.int64), hi)
            j = int(np.argmax(passes(grid)))
            lo, hi = int(grid[j - 1]), int(grid[j])
        out = float(_f32_of_keys(np.array([hi]))[0])
    _BSTAR[ck] = out
    return out


def threshold_plan(scores: torch.Tensor, row_starts: Sequence[int], seq_lens: Sequence[int],
                   art_starts: Sequence[int], art_ends: Sequence[int], head, device,
                   rms_eps: float = RMS_EPS):
    """The threshold mode's selection (_select_threshold via _select_indices, gate_forward.py:102-143)
    for a batch: tg_gate_threshold_select computes every state token's selection value agg
    (aggregate of E2EGate.forward's bias, e2e_gate_module.py:363-399) and the per-sequence count of
    tokens with sigmoid(agg) >= head.tau; one host synchronisation reads the counts.  Returns
    (plan with K_b = max(count_b, 1) -- the argmax fallback when nothing passes --, sel: the scores
    whose top-K_b are exactly the kept tokens, agg, sumsq (per sequence, for the kept rows' gate
    bias), counts).  K is the reference's sample-dependent kept count; the caller's K is unused,
    as in the reference."""
    if scores.dtype != torch.float32 or scores.dim() != 1 or not scores.is_contiguous():
        raise RuntimeError("scores must be a contiguous 1-D float32 tensor")
    n = len(seq_lens)
    p0 = plan(row_starts, seq_lens, art_starts, art_ends, [1] * n, device)
    hs = head.selection_head_scale()
    b_star = sigmoid_threshold(float(head.tau), scores.device)
    agg = torch.empty_like(scores)
    sel = torch.empty_like(scores)
    counts = torch.empty(n, dtype=torch.int32, device=scores.device)
    sumsq = torch.empty(n, dtype=torch.float32, device=scores.device)
    hs_arr = (ctypes.c_float * len(hs))(*hs)
    _lib.call("tg_gate_threshold_select", scores.data_ptr(), p0.geom.data_ptr(), n, ctypes.cast(hs_arr, ctypes.c_void_p),
              len(hs), float(getattr(head, "bias_gain", 1.0)), float(rms_eps), float(b_star), agg.data_ptr(),
              sel.data_ptr(), counts.data_ptr(), sumsq.data_ptr(), _stream(scores))
    ch = counts.cpu().tolist()
    p = plan(row_starts, seq_lens, art_starts, art_ends, [max(1, c) for c in ch], device)
    return p, sel, agg, sumsq, ch


def _streams(pairs, p: KeepPlan):
    """PackStream array of (src, dst) or (src, dst, gap) entries: with a gap, kept row j of
    sequence b goes to dst row j + b * gap (a cache with `gap` free rows after each sequence)."""
    arr = (PackStream * max(1, len(pairs)))()
    nseq = len(p.n_kept)
    for i, pr in enumerate(pairs):
        src, dst = pr[0], pr[1]
        gap = int(pr[2]) if len(pr) > 2 else 0
        if gap < 0:
            raise RuntimeError("pack: negative destination gap")
        if dst.shape[0] < p.total_kept + gap * max(0, nseq - 1):
            raise RuntimeError("pack: destination has fewer rows than kept tokens")
        arr[i] = _row_stream(src, dst, gap)
    return arr


def _row_stream(src: torch.Tensor, dst: torch.Tensor, gap: int = 0) -> PackStream:
    """A (rows, ...) source / destination pair.  The source may be (rows, chunks, chunk_elems) with
    any row and chunk strides (head-major caches); everything after the row axis of dst, and the
    chunk axis of src, must be contiguous."""
    if src.dtype != dst.dtype:
        raise RuntimeError("pack: source and destination dtypes differ")
    es = src.element_size()
    if src.dim() == 3 and not src[0].is_contiguous():
        if src.stride(2) != 1:
            raise RuntimeError("pack: the innermost source axis must be contiguous")
        n_chunks, chunk = src.shape[1], src.shape[2] * es
        chunk_stride = src.stride(1) * es
    else:
        if not src[0].is_contiguous():
            raise RuntimeError("pack: source rows must be contiguous (or (rows, chunks, elems))")
        n_chunks, chunk, chunk_stride = 1, src[0].numel() * es, 0
    if not dst[0].is_contiguous() or dst[0].numel() * dst.element_size() != n_chunks * chunk:
        raise RuntimeError("pack: destination rows must be contiguous and as long as a source row")
    return PackStream(src.data_ptr(), dst.data_ptr(), src.stride(0) * es, dst.stride(0) * es, chunk_stride,
                      chunk, n_chunks, gap)


def pack(keep: torch.Tensor, p: KeepPlan, pairs: Sequence[tuple],
         positions: Optional[torch.Tensor] = None, bias_src: Optional[torch.Tensor] = None,
         sumsq: Optional[torch.Tensor] = None, bias_out: Optional[torch.Tensor] = None,
         rms_eps: float = RMS_EPS) -> None:
    """One launch: dst[j] = src[row_start[b] + keep[j]] for every (src, dst) pair (or dst[j + b * gap]
    for a (src, dst, gap) entry); positions[j] =
    keep[j]; bias_out[j] = RMS-normalised bias_src score of kept article rows, 0 elsewhere."""
    if len(pairs) > 16:
        raise RuntimeError("pack: at most 16 row streams per launch")
    arr = _streams(pairs, p)
    for t, dt in ((positions, torch.int64), (bias_src, torch.float32), (sumsq, torch.float32),
                  (bias_out, torch.float32)):
        if t is not None and (t.dtype != dt or not t.is_contiguous()):
            raise RuntimeError("pack: positions must be contiguous int64, bias / sumsq contiguous float32")
    if p.total_kept == 0:
        return
    _lib.call("tg_gate_pack", ctypes.cast(arr, ctypes.c_void_p), len(pairs), keep.data_ptr(), p.geom.data_ptr(),
              len(p.n_kept), p.total_kept, positions.data_ptr() if positions is not None else None,
              bias_src.data_ptr() if bias_src is not None else None,
              sumsq.data_ptr() if sumsq is not None else None, float(rms_eps),
              bias_out.data_ptr() if bias_out is not None else None, _stream(keep))


def ktile_w1(w1: torch.Tensor) -> torch.Tensor:
    """W1 (256, 2048) stored k-step major, (64, 256, 32): each 32-input step of the scoring kernel's
    weight stream is then 16 KiB contiguous (tg_gate_score_mlp_ktiled)."""
    d_h, d_in = w1.shape
    return w1.reshape(d_h, d_in // 32, 32).transpose(0, 1).contiguous()


def score_mlp(x: torch.Tensor, w1: torch.Tensor, b1: torch.Tensor, w2: torch.Tensor, b2: float,
              out: Optional[torch.Tensor] = None, w1_ktiled: Optional[torch.Tensor] = None) -> torch.Tensor:
    """scores[r] = w2 . silu(W1 x_r + b1) + b2 for every row of x (rows, 2048) bf16;
    W1 (256, 2048) bf16; b1, w2 (256,) float32.  With w1_ktiled = ktile_w1(W1) the kernel streams
    that copy instead (the same results, bit for bit)."""
    if x.dtype != torch.bfloat16 or w1.dtype != torch.bfloat16 or x.dim() != 2 or x.stride(1) != 1:
        raise RuntimeError("score_mlp: x (rows, 2048) and W1 (256, 2048) must be bf16 with contiguous rows")
    if not w1.is_contiguous() or b1.dtype != torch.float32 or w2.dtype != torch.float32:
        raise RuntimeError("score_mlp: W1 contiguous bf16, b1 / w2 float32")
    if w1_ktiled is not None and (w1_ktiled.dtype != torch.bfloat16 or not w1_ktiled.is_contiguous() or
                                  w1_ktiled.shape != (w1.shape[1] // 32, w1.shape[0], 32)):
        raise RuntimeError("score_mlp: w1_ktiled must be ktile_w1(W1)")
    n = x.shape[0]
    out = out if out is not None else torch.empty(n, dtype=torch.float32, device=x.device)
    if n:
        fn, w = ("tg_gate_score_mlp", w1) if w1_ktiled is None else ("tg_gate_score_mlp_ktiled", w1_ktiled)
        _lib.call(fn, x.data_ptr(), n, x.stride(0), x.shape[1], w1.shape[0], w.data_ptr(),
                  b1.contiguous().data_ptr(), w2.contiguous().data_ptr(), float(b2), out.data_ptr(), _stream(x))
    return out


def keep_indices(scores_art: torch.Tensor, K: int, article_start: int, article_end: int, seq_len: int) -> torch.Tensor:
    """Single-sequence form of the reference's keep construction (gate_forward.py:1417-1421):
    [0, s) + s + sort(topk(scores_art, K_c)) + [e, seq_len).  scores_art holds the article's scores."""
    n = article_end - article_start
    if scores_art.numel() != n:
        raise ValueError("scores_art must hold exactly the article's scores")
    full = torch.zeros(seq_len, dtype=torch.float32, device=scores_art.device)
    full[article_start:article_end] = scores_art.float()
    p = plan([0], [seq_len], [article_start], [article_end], [K], scores_art.device)
    keep, _ = select_keep(full, p, with_sumsq=False)
    return keep


def branch_readout(gu: torch.Tensor, w_row: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """scores[r] = bf16(w_row . bf16(bf16(silu(gu[r, :I])) * gu[r, I:])) as float32 for the fused
    gate/up rows gu (rows, 2I) bf16 of the scoring branch; w_row (I,) bf16."""
    if gu.dtype != torch.bfloat16 or w_row.dtype != torch.bfloat16 or gu.dim() != 2 or gu.stride(1) != 1:
        raise RuntimeError("branch_readout: gu (rows, 2I) and w_row (I,) must be bf16 with contiguous rows")
    n, inter = gu.shape[0], gu.shape[1] // 2
    if w_row.numel() != inter or not w_row.is_contiguous():
        raise RuntimeError("branch_readout: w_row must be contiguous with I = gu.shape[1] / 2 entries")
    out = out if out is not None else torch.empty(n, dtype=torch.float32, device=gu.device)
    if out.dtype != torch.float32 or out.numel() < n or not out.is_contiguous():
        raise RuntimeError("branch_readout: out must be contiguous float32 with one entry per row")
    if n:
        _lib.call("tg_gate_branch_readout", gu.data_ptr(), gu.stride(0), n, inter, w_row.data_ptr(), out.data_ptr(),
                  _stream(gu))
    return out


class _BiasScales:
    """Per-(Phase-2 layer, head) bias magnitude and temperature shared by the scoring heads:
    gate_scale (L2, H) and attn_scale (L2, H) or None, both pre-softplus, scaled_softmax flag and
    the normalisation gain bias_gain.  selection_mode / tau: E2EGate's selection (e2e_gate_module.py
    :216-266): "topk" keeps K state tokens, "threshold" keeps those with sigmoid(agg) >= tau
    (threshold_plan)."""
    bias_gain: float = 1.0
    selection_mode: str = "topk"
    tau: float = 0.5

    def selection_head_scale(self) -> List[float]:
        """softplus(gate_scale) of the first Phase-2 layer, fp32, as host floats: the per-head factors
        of the selection value agg (aggregate, e2e_gate_module.py:387-399)."""
        return torch.nn.functional.softplus(self.gate_scale[0].float()).cpu().tolist()

    @property
    def ssmax(self) -> bool:
        return self.scaled_softmax and self.attn_scale is not None

    def phase2_tables(self, kept_bias: torch.Tensor, ratio: Optional[torch.Tensor], softmax_scale: float
                      ) -> Tuple[torch.Tensor, Optional[torch.Tensor], Optional[torch.Tensor]]:
        """The Phase-2 constants of the packed kept rows, in the reference's own arithmetic.

        kept_bias (T2,) fp32: each kept row's RMS-normalised score (0 on prefix / suffix rows);
        ratio (T2,) fp32: each kept row's scaled-softmax ratio r, or None.  The stored bias is
        gb[l, j, h] = bf16(fp32(bias_gain * kept_bias_j) * softplus(gate_scale[l, h])) (E2EGate.forward
        e2e_gate_module.py:363-385, kept in the model dtype by build_gate_bias_vectorized
        gate_forward.py:995-1008, :1450); the key bias and query multiplier follow _phase2_q_bias
        (qwen3_flex_attention.py:433-473) in bf16: scaled softmax s_eff = bf16(bf16(gamma_h) *
        bf16(r)), bias' = bf16(gb * bf16(mean_h s_eff)); per-head temperature bias' =
        bf16(gb * bf16(gamma_h)), gamma = softplus(attn_scale) (attn_scale_eff :302-305).

        Returns (bias_raw (L2, H, T2) fp32 = bias' / softmax_scale, the kernel's raw-score units as
        flash_attn_key_bias forms them (kernels/fa2bias/keybias.py:86); q_head (L2, H) and q_row
        (T2,) fp32 bf16 values, or None: the factors tg_qk_norm_rope multiplies (s = bf16(q_head *
        q_row)))."""
        bf = torch.bfloat16
        gs = torch.nn.functional.softplus(self.gate_scale.float())              # (L2, H)
        bn = kept_bias.float()
        if self.bias_gain != 1.0:
            bn = bn * float(self.bias_gain)
        gb = (bn[None, :, None] * gs[:, None, :]).to(bf)                        # (L2, T2, H)
        q_head = q_row = None
        if self.attn_scale is None:
            bias = gb
        else:
            temp = torch.nn.functional.softplus(self.attn_scale.float()).to(bf)  # (L2, H)
            q_head = temp.float().contiguous()
            if self.ssmax:
                if ratio is None:
                    raise RuntimeError("phase2_tables: scaled softmax needs the kept rows' ratio")
                rb = ratio.to(bf)
                s_eff = temp[:, :, None] * rb[None, None, :]                     # (L2, H, T2) bf16
                bias = gb * s_eff.mean(1)[:, :, None]
                q_row = rb.float()
            else:
                bias = gb * temp[:, None, :]
        return (bias.float().permute(0, 2, 1) / softmax_scale).contiguous(), q_head, q_row

    def decode_query_head(self) -> Optional[torch.Tensor]:
        """q_head for a decode step: the new token's multiplier is bf16(gamma_h * r) from fp32
        factors in scaled-softmax mode (FormDecodeState.step, qwen3_flex_attention.py:1090-1101,
        applied at :400), bf16(gamma_h) with a per-head temperature; None without one."""
        if self.attn_scale is None:
            return None
        temp = torch.nn.functional.softplus(self.attn_scale.float())
        return (temp if self.ssmax else temp.to(torch.bfloat16).float()).contiguous()


@dataclass
class ScoringHead(_BiasScales):
    """The gate's parameters for one prefill.

    Scoring: score_j = w2 . silu(W1 x_j + b1) + b2 on the gate layer's hidden state (the
    Linear(2048->256) -> SiLU -> Linear(256->1) head of the 32k gate workload).  Bias: the kept
    article rows' scores RMS-normalised over the article (E2EGate.forward,
    e2e_gate_module.py:348-385, eps 1e-6 :74), times softplus(gate_scale[l, h]) per Phase-2 layer
    l and query head h; the attention temperature softplus(attn_scale[l, h]) (attn_scale_eff
    :302-305) multiplies both the query and the bias (_phase2_q_bias,
    qwen3_flex_attention.py:433-473, per-head branch).  Top-K ranks the raw score: the
    reference's selection key (aggregate :387-399) is a positive multiple of it."""
    w1: torch.Tensor            # (256, 2048) bf16
    b1: torch.Tensor            # (256,) fp32
    w2: torch.Tensor            # (256,) fp32
    b2: float
    gate_scale: torch.Tensor    # (n_phase2_layers, H) fp32, pre-softplus
    attn_scale: Optional[torch.Tensor] = None   # (n_phase2_layers, H) fp32, pre-softplus
    # scaled-softmax mode (E2EGate.scaled_softmax_scale, e2e_gate_module.py:229): the temperature
    # becomes gamma_h * r_q per query and the bias is scaled by mean_h(gamma) * r_k per key, with
    # r = min(1, ln max(slot, 2) / ln max(position + 1, 2)) (_ssmax_ratio, gate_forward.py:574-585;
    # _phase2_q_bias, qwen3_flex_attention.py:433-473).  Needs attn_scale.
    scaled_softmax: bool = False
    split_gate_layer: ClassVar[bool] = False      # scores the gate layer's full output
    _w1k: Optional[tuple] = field(default=None, init=False, repr=False, compare=False)

    def scores(self, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        # the k-step-major copy of W1 the kernel streams, made once (and again if w1 is replaced)
        if self._w1k is None or self._w1k[0] is not self.w1:
            self._w1k = (self.w1, ktile_w1(self.w1))
        return score_mlp(x, self.w1, self.b1, self.w2, self.b2, out=out, w1_ktiled=self._w1k[1])


@dataclass
class BranchHead(_BiasScales):
    """The finalized gate (E2EGate, e2e_gate_module.py:204-399) with its MLP scoring branch.

    Scoring (gate_branch_hs, gate_forward.py:491-524, absorbed readout without residual): on the
    gate layer's attention boundary a_j, z = post_attention_layernorm(a_j) of the gate layer and
    score_j = w_row . (silu(W_gate z) * (W_up z)) in bf16 — a clone of the gate layer's Qwen3MLP
    whose down projection is the single absorbed row w_row (build_gate_branch :261-342; load_gate
    e2e_gate_module.py:497-514).  Its presence splits the gate layer (split_gate_layer_mlp
    :345-357): Phase 1 ends at a_j, and the gate layer's own MLP runs on the kept rows only at
    Phase-2 entry (gate_layer_mlp :422-437, applied at :1476-1478).  Bias: the bf16 score,
    RMS-normalised over the state span in float32 with gain bias_gain (b_norm, :296-300), times
    softplus(gate_scale[l, h]) (forward :348-385); scaled softmax is the finalized default
    (scaled_softmax_scale :229).  Top-K ranks the bf16 score: the selection key (aggregate,
    mean over heads of layer 0's bias, :387-399) is a non-decreasing function of it."""
    w_gu: torch.Tensor          # (2I, d) bf16: the branch's gate_proj rows, then its up_proj rows
    w_row: torch.Tensor         # (I,) bf16: the absorbed down_proj row
    gate_scale: torch.Tensor    # (n_phase2_layers, H) fp32, pre-softplus
    attn_scale: Optional[torch.Tensor] = None
    scaled_softmax: bool = True
    bias_gain: float = 1.0
    split_gate_layer: ClassVar[bool] = True

    @property
    def inter(self) -> int:
        return self.w_row.numel()

    def scores_from_boundary(self, a: torch.Tensor, ln2: torch.Tensor, eps: float,
                             out: Optional[torch.Tensor] = None, normed: Optional[torch.Tensor] = None,
                             chunk_rows: int = 65536) -> torch.Tensor:
        """bf16-valued float32 scores of every row of the boundary a (T, d) bf16; ln2: the gate
        layer's post_attention_layernorm weight.  The branch's gate/up GEMM runs in row chunks of
        chunk_rows (the reference bounds its MLP workspace the same way, gate_forward.py:418-437)."""
        from tokengate_amd.decoder import rmsnorm
        T, d = a.shape
        if self.w_gu.shape != (2 * self.inter, d):
            raise RuntimeError("BranchHead: w_gu must be (2 * len(w_row), d_model)")
        out = out if out is not None else torch.empty(T, dtype=torch.float32, device=a.device)
        if T == 0:
            return out
        normed = normed[:T] if normed is not None else torch.empty_like(a)
        rmsnorm(a, ln2, eps, out=normed)
        cr = max(1, min(T, int(chunk_rows)))
        gu = torch.empty(cr, 2 * self.inter, dtype=torch.bfloat16, device=a.device)
        for r0 in range(0, T, cr):
            r1 = min(T, r0 + cr)
            torch.matmul(normed[r0:r1], self.w_gu.t(), out=gu[:r1 - r0])
            branch_readout(gu[:r1 - r0], self.w_row, out=out[r0:r1])
        return out


def ssmax_ratio_rows(kept_pos: torch.Tensor, cu_kept: Sequence[int]) -> torch.Tensor:
    """r per packed kept row: min(1, ln max(m, 2) / ln max(p + 1, 2)), m the row's 1-based slot
    within its sequence and p its original position (_ssmax_ratio, gate_forward.py:574-585);
    fp32 on the rows' device, built without a host synchronisation."""
    dev = kept_pos.device
    T = int(cu_kept[-1])
    n = torch.tensor([cu_kept[b + 1] - cu_kept[b] for b in range(len(cu_kept) - 1)], dtype=torch.int64)
    st = torch.tensor(list(cu_kept[:-1]), dtype=torch.int64)
    if dev.type == "cuda":
        n, st = n.pin_memory().to(dev, non_blocking=True), st.pin_memory().to(dev, non_blocking=True)
    slot = torch.arange(T, device=dev) - torch.repeat_interleave(st, n, output_size=T) + 1
    m = slot.to(torch.float32).clamp(min=2.0)
    pos = (kept_pos.to(torch.float32) + 1.0).clamp(min=2.0)
    return (torch.log(m) / torch.log(pos)).clamp(max=1.0)


def random_head(n_layers: int, n_heads: int, seed: int = 5, device="cuda", d_in: int = 2048, d_hidden: int = 256,
                gate_scale: Optional[float] = None, temperature: bool = True,
                scaled_softmax: bool = False) -> ScoringHead:
    """Seeded head: Xavier-uniform W1 / w2, zero b1 / b2; gate_scale = softplus^-1(1.0) (or a
    given value) plus a small seeded spread per (layer, head); attn_scale = softplus^-1(1), the
    identity temperature E2EGate starts from."""
    import math
    g = torch.Generator(device=device).manual_seed(seed)
    a1 = math.sqrt(6.0 / (d_in + d_hidden))
    w1 = ((torch.rand(d_hidden, d_in, generator=g, device=device) * 2 - 1) * a1).to(torch.bfloat16)
    w2 = (torch.rand(d_hidden, generator=g, device=device) * 2 - 1) * math.sqrt(6.0 / (d_hidden + 1))
    b1 = torch.zeros(d_hidden, device=device)
    base = math.log(math.expm1(1.0)) if gate_scale is None else gate_scale
    gs = base + 0.1 * torch.randn(n_layers, n_heads, generator=g, device=device)
    at = torch.full((n_layers, n_heads), math.log(math.expm1(1.0)), device=device) if temperature else None
    return ScoringHead(w1, b1, w2, 0.0, gs, at, scaled_softmax)


def random_branch_head(wts, gate_layer: int, seed: int = 5, gate_scale: Optional[float] = None,
                       row_std: Optional[float] = None) -> BranchHead:
    """Seeded finalized-gate head on decoder weights wts: the branch starts as a copy of the gate
    layer's gate/up projections (build_gate_branch, gate_forward.py:261-342); the absorbed row,
    zero at initialisation there, is a seeded normal row of std row_std (default I^-1/2) standing
    in for a trained one; gate_scale as random_head; attn_scale = softplus^-1(1) plus a seeded
    spread; scaled softmax on."""
    import math
    dev = wts.device
    shape = wts.shape
    n_layers = shape.n_layers - gate_layer - 1
    g = torch.Generator(device=dev).manual_seed(seed)
    w_gu = wts.layers[gate_layer].w_gu.clone()
    inter = w_gu.shape[0] // 2
    std = row_std if row_std is not None else inter ** -0.5
    w_row = (torch.randn(inter, generator=g, device=dev) * std).to(torch.bfloat16)
    base = math.log(math.expm1(1.0)) if gate_scale is None else gate_scale
    gs = base + 0.1 * torch.randn(n_layers, shape.n_heads, generator=g, device=dev)
    at = math.log(math.expm1(1.0)) + 0.1 * torch.randn(n_layers, shape.n_heads, generator=g, device=dev)
    return BranchHead(w_gu, w_row, gs, at, True)
