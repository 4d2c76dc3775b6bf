"""Gate path host API: scoring, order-preserving top-K keep lists and the ragged pack.

Mirrors the selection and prune/pack steps of prefill_batch_for_decode
(tokengate/e2e_gate/gate_module/gate_forward.py:1384-1522) — K_clamped = max(1, min(K, n_art))
(:1409-1410), keep = [0, s) + s + sort(topk) + [e, seq_len) (:1417-1421, _keep_indices :77-81),
hidden/KV row gathers at the kept positions (:1454-1522), kept positions (:1457) and the kept rows'
gate bias (build_gate_bias_vectorized :968-1036) — on the gfx950 kernels of csrc/gate.hip.

Differences from the reference, by design: kept rows of all sequences are packed back to back
(cu_seqlens layout) rather than right-padded to the longest; score ties go to the lower position
(torch.topk leaves the order unspecified).  The per-sequence Python loop of the reference becomes
one launch per step for the whole batch.
"""
import ctypes
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import torch

from tokengate_amd import _lib

RMS_EPS = 1e-6   # E2EGate's normalisation epsilon (e2e_gate_module.py:74)


class PackStream(ctypes.Structure):
    """C layout of tg_pack_stream (include/tokengate_hip.h)."""
    _fields_ = [("src", ctypes.c_void_p), ("dst", ctypes.c_void_p), ("src_row_stride", ctypes.c_int64),
                ("dst_row_stride", ctypes.c_int64), ("src_chunk_stride", ctypes.c_int64),
                ("chunk_bytes", ctypes.c_int32), ("n_chunks", ctypes.c_int32)]


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
    gd = gh.pin_memory().to(device, non_blocking=True) if torch.device(device).type == "cuda" else gh
    max_art = max((int(art_ends[b]) - int(art_starts[b]) for b in range(n)), default=0)
    return KeepPlan(gh, gd, n_kept, kcs, cu, max_art)


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


def _row_stream(src: torch.Tensor, dst: torch.Tensor) -> PackStream:
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
                      chunk, n_chunks)


def pack(keep: torch.Tensor, p: KeepPlan, pairs: Sequence[Tuple[torch.Tensor, torch.Tensor]],
         positions: Optional[torch.Tensor] = None, bias_src: Optional[torch.Tensor] = None,
         sumsq: Optional[torch.Tensor] = None, bias_out: Optional[torch.Tensor] = None,
         rms_eps: float = RMS_EPS) -> None:
    """One launch: dst[j] = src[row_start[b] + keep[j]] for every (src, dst) pair; positions[j] =
    keep[j]; bias_out[j] = RMS-normalised bias_src score of kept article rows, 0 elsewhere."""
    if len(pairs) > 16:
        raise RuntimeError("pack: at most 16 row streams per launch")
    arr = (PackStream * max(1, len(pairs)))()
    for i, (s, d) in enumerate(pairs):
        if d.shape[0] < p.total_kept:
            raise RuntimeError("pack: destination has fewer rows than kept tokens")
        arr[i] = _row_stream(s, d)
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


def score_mlp(x: torch.Tensor, w1: torch.Tensor, b1: torch.Tensor, w2: torch.Tensor, b2: float,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """scores[r] = w2 . silu(W1 x_r + b1) + b2 for every row of x (rows, 2048) bf16;
    W1 (256, 2048) bf16; b1, w2 (256,) float32."""
    if x.dtype != torch.bfloat16 or w1.dtype != torch.bfloat16 or x.dim() != 2 or x.stride(1) != 1:
        raise RuntimeError("score_mlp: x (rows, 2048) and W1 (256, 2048) must be bf16 with contiguous rows")
    if not w1.is_contiguous() or b1.dtype != torch.float32 or w2.dtype != torch.float32:
        raise RuntimeError("score_mlp: W1 contiguous bf16, b1 / w2 float32")
    n = x.shape[0]
    out = out if out is not None else torch.empty(n, dtype=torch.float32, device=x.device)
    if n:
        _lib.call("tg_gate_score_mlp", x.data_ptr(), n, x.stride(0), x.shape[1], w1.shape[0], w1.data_ptr(),
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


@dataclass
class ScoringHead:
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

    def scores(self, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        return score_mlp(x, self.w1, self.b1, self.w2, self.b2, out=out)

    @property
    def ssmax(self) -> bool:
        return self.scaled_softmax and self.attn_scale is not None

    def layer_coefficients(self, softmax_scale: float) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        """(bias coefficient in raw-score units, per-head query scale) per (layer, head):
        raw bias of key j = normalised score_j * coef[l, h] (* r_j in scaled-softmax mode), where
        coef = softplus(gate_scale) * temperature / softmax_scale; the temperature is
        softplus(attn_scale) per head, or its mean over heads in scaled-softmax mode."""
        coef = torch.nn.functional.softplus(self.gate_scale.float())
        qs = None
        if self.attn_scale is not None:
            qs = torch.nn.functional.softplus(self.attn_scale.float()).contiguous()
            coef = coef * (qs.mean(1, keepdim=True) if self.scaled_softmax else qs)
        return (coef / softmax_scale).contiguous(), qs


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
