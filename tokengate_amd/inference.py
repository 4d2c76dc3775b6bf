"""Public inference API with the names of tokengate.inference (tokengate/inference.py:1-180).

    from tokengate_amd.inference import load_model, apply_chat_template
    model = load_model("random", gate_layer=1)            # or a local Qwen3 checkpoint directory
    ids = apply_chat_template(tok, "Answer using the article.\\n{state}\\nAnswer:", state=text)
    out = model.generate([ids], tok, max_kept_prefill_tokens=1000, max_new_tokens=64)

generate() is the gated prefill of tokengate_amd.prefill (one ragged batch: Phase 1 over every
prompt token, gate, top-K keep, pack, Phase 2 on the kept rows) followed by greedy decode
(tokengate_amd.decode).  The prompt ids carry the state span as the sentinel ids
STATE_START_ID / STATE_END_ID, exactly as the reference's apply_chat_template produces them.

Model sources (no network here): "random" / "random:<seed>" builds a seeded Qwen3-1.7B-shaped
decoder with a seeded scoring head; a local directory holding a transformers Qwen3 checkpoint
(config.json + *.safetensors) loads the base model's weights (safetensors only, nothing
unpickled) with a seeded head, or the head saved by save_head() when `gate_path` is given.
"""
import glob
import json
import os
import re
import time
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple, Union

import torch

from tokengate_amd import decoder as dec
from tokengate_amd import gate as G
from tokengate_amd import prefill as P

# Sentinel ids marking the state span inside prompt ids (gate_forward.py:669-670).
STATE_START_ID = -1001
STATE_END_ID = -1002
# K meaning "keep every state token" (inference.py:35).
_NO_PRUNING = 10_000_000


def split_state_span(ids: List[int]) -> Tuple[List[int], int, int]:
    """(clean_ids, start, end) from ids carrying exactly one STATE_START_ID followed by one
    STATE_END_ID (gate_forward.py:673-689); ValueError otherwise."""
    starts = [i for i, t in enumerate(ids) if t == STATE_START_ID]
    ends = [i for i, t in enumerate(ids) if t == STATE_END_ID]
    if len(starts) != 1 or len(ends) != 1 or starts[0] >= ends[0]:
        raise ValueError("ids carry no valid state span: expected exactly one STATE_START_ID followed by one "
                         f"STATE_END_ID (use apply_chat_template(state=...)); found starts={starts} ends={ends}")
    s, e = starts[0], ends[0]
    return ids[:s] + ids[s + 1:e] + ids[e + 1:], s, e - 1


def find_article_boundaries(full_ids: List[int], empty_ids: List[int]) -> Tuple[int, int]:
    """(common prefix length, common suffix length) of the prompt rendered with and without the
    state (gate_forward.py: find_article_boundaries)."""
    pre = 0
    for a, b in zip(full_ids, empty_ids):
        if a != b:
            break
        pre += 1
    post = 0
    for i in range(1, min(len(full_ids), len(empty_ids)) - pre + 1):
        if full_ids[-i] != empty_ids[-i]:
            break
        post = i
    return pre, post


def compute_prunable_span(full_ids: List[int], empty_ids: List[int]) -> Tuple[int, int]:
    pre, post = find_article_boundaries(full_ids, empty_ids)
    return pre, len(full_ids) - post


def apply_chat_template(tokenizer, prompt: str, use_chat_template: bool = True, state: str = None) -> List[int]:
    """Token ids of `prompt` (chat-templated unless use_chat_template=False); with `state`, the
    prompt holds "{state}" exactly once and the state's token span is marked by the sentinels
    (gate_forward.py:692-770)."""
    if state is not None:
        if prompt.count("{state}") != 1:
            raise ValueError("apply_chat_template(state=...) requires the prompt to contain the placeholder "
                             f"'{{state}}' exactly once; found {prompt.count('{state}')} occurrences.")
        full = apply_chat_template(tokenizer, prompt.replace("{state}", state), use_chat_template)
        empty = apply_chat_template(tokenizer, prompt.replace("{state}", ""), use_chat_template)
        s, e = compute_prunable_span(full, empty)
        return full[:s] + [STATE_START_ID] + full[s:e] + [STATE_END_ID] + full[e:]
    if not use_chat_template:
        ids = tokenizer.encode(prompt, add_special_tokens=False)
        return list(ids.tolist() if hasattr(ids, "tolist") else ids)
    msgs = [{"role": "user", "content": prompt}]
    try:
        ids = tokenizer.apply_chat_template(msgs, add_generation_prompt=True, tokenize=True, enable_thinking=False)
    except TypeError:
        ids = tokenizer.apply_chat_template(msgs, add_generation_prompt=True, tokenize=True)
    if hasattr(ids, "input_ids"):
        ids = ids.input_ids
    if hasattr(ids, "tolist"):
        ids = ids.tolist()
    if ids and isinstance(ids[0], list):
        ids = ids[0]
    return list(ids)


_THINK_RE = re.compile(r"<think>.*?</think>", re.DOTALL)
_THINK_OPEN_RE = re.compile(r"<think>.*", re.DOTALL)


def _strip_thinking(text: str) -> str:
    return _THINK_OPEN_RE.sub("", _THINK_RE.sub("", text)).strip()


@dataclass
class GenerateOutput:
    """Result of TokenGateModel.generate, one entry per input sequence (inference.py:60-69)."""
    answers: List[str]
    n_kept: List[int]
    n_state: List[int]
    kept_pos: List[List[int]]
    prefill_s: float
    decode_s: float
    token_ids: List[List[int]]


def _sync():
    torch.cuda.synchronize()


class TokenGateModel:
    """Decoder weights + scoring head + gate layer behind one object (inference.py:72-150)."""

    def __init__(self, weights: dec.DecoderWeights, head, gate_layer: int, base_model: str):
        self.weights = weights
        self.gate = head
        self.gate_layer = gate_layer
        self.base_model = base_model

    @property
    def config(self) -> dec.DecoderShape:
        return self.weights.shape

    @property
    def device(self) -> torch.device:
        return self.weights.device

    def prefill(self, ids: Sequence, max_kept_prefill_tokens=None, prune_below_gate: bool = False,
                decode_headroom: int = 0):
        """Gated prefill of already-split prompts: ids = [(clean_ids, start, end), ...];
        decode_headroom: free cache rows left after each sequence for the decode to append to."""
        k = _NO_PRUNING if max_kept_prefill_tokens is None else max_kept_prefill_tokens
        return P.prefill_batch(self.weights, self.gate, [x[0] for x in ids], [x[1] for x in ids],
                               [x[2] for x in ids], self.gate_layer, k, prune_below_gate=prune_below_gate,
                               decode_headroom=decode_headroom)

    @torch.no_grad()
    def generate(self, ids: Union[List[int], List[List[int]]], tokenizer=None, *, max_new_tokens: int = 20,
                 max_kept_prefill_tokens: Optional[int] = None, streamer=None,
                 prune_below_gate: bool = False) -> GenerateOutput:
        """Gated prefill + greedy decode (TokenGateModel.generate, inference.py:85-124).  ids: one
        sequence or a batch, each carrying the state sentinels.  max_kept_prefill_tokens: the K of
        the paper (None keeps every state token); a list gives one K per sequence.  tokenizer:
        provides eos_token_id and decode(); without one, no EOS stops generation and answers are
        empty strings.  streamer: optional object with put(cpu (B, 1) int64) and end()."""
        from tokengate_amd.decode import DecodeState
        if max_new_tokens < 1:
            raise ValueError("max_new_tokens must be positive")
        if ids and isinstance(ids[0], int):
            ids = [ids]
        split = [split_state_span(list(seq)) for seq in ids]
        _sync()
        t0 = time.perf_counter()
        pf = self.prefill(split, max_kept_prefill_tokens, prune_below_gate,
                          decode_headroom=max_new_tokens if max_new_tokens > 1 else 0)
        first = pf.first_tokens
        _sync()
        prefill_s = time.perf_counter() - t0
        B = len(split)
        eos_id = getattr(tokenizer, "eos_token_id", None) if tokenizer is not None else None
        gen = [first]
        if streamer is not None:
            streamer.put(first.detach().cpu().view(B, 1))
        t0 = time.perf_counter()
        if max_new_tokens > 1:
            st = DecodeState(self.weights, self.gate, self.gate_layer, pf, max_new_tokens, prune_below_gate,
                             graph=True)
            cur = first
            done = torch.zeros(B, dtype=torch.bool, device=first.device)
            for _ in range(max_new_tokens - 1):
                if eos_id is not None:
                    done |= cur == eos_id
                    if bool(done.all()):
                        break
                cur = st.step(cur)
                gen.append(cur)
                if streamer is not None:
                    streamer.put(cur.detach().cpu().view(B, 1))
        _sync()
        decode_s = time.perf_counter() - t0
        if streamer is not None:
            streamer.end()
        toks = torch.stack(gen, 1).cpu().tolist()
        answers, token_ids = [], []
        for row in toks:
            if eos_id is not None and eos_id in row:
                end = row.index(eos_id)
                token_ids.append(row[:end + 1])
                row = row[:end]
            else:
                token_ids.append(row)
            answers.append(_strip_thinking(tokenizer.decode(row, skip_special_tokens=True))
                           if tokenizer is not None and row else "")
        kp = pf.kept_positions.cpu()
        kept_pos = [kp[pf.cu_kept[b]:pf.cu_kept[b + 1]].tolist() for b in range(B)]
        return GenerateOutput(answers, list(pf.n_kept), [e - s for _, s, e in split], kept_pos, prefill_s, decode_s,
                              token_ids)


# ---- loading --------------------------------------------------------------------------------

def _load_hf_qwen3(path: str, device) -> Tuple[dec.DecoderWeights, str]:
    """Weights of a transformers Qwen3ForCausalLM checkpoint directory (config.json +
    *.safetensors), fused into this package's layout (q|k|v and gate|up projections)."""
    from safetensors.torch import load_file
    with open(os.path.join(path, "config.json")) as f:
        cfg = json.load(f)
    if cfg.get("attention_bias", False):
        raise ValueError("attention projections with bias are not supported")
    H = cfg["num_attention_heads"]
    D = cfg.get("head_dim") or cfg["hidden_size"] // H
    shape = dec.DecoderShape(n_layers=cfg["num_hidden_layers"], d_model=cfg["hidden_size"], n_heads=H,
                             n_kv_heads=cfg["num_key_value_heads"], head_dim=D, d_ff=cfg["intermediate_size"],
                             vocab=cfg["vocab_size"], rms_eps=cfg.get("rms_norm_eps", 1e-6),
                             rope_theta=cfg.get("rope_theta", (cfg.get("rope_parameters") or {}).get("rope_theta", 1e6)),
                             tie_embeddings=cfg.get("tie_word_embeddings", False))
    sd = {}
    for fn in sorted(glob.glob(os.path.join(path, "*.safetensors"))):
        sd.update(load_file(fn, device="cpu"))
    if not sd:
        raise FileNotFoundError(f"no *.safetensors in {path}")
    bf = torch.bfloat16

    def t(name):
        if name not in sd:
            raise KeyError(f"{path}: missing tensor {name}")
        return sd[name].to(device=device, dtype=bf)

    layers = []
    for i in range(shape.n_layers):
        p = f"model.layers.{i}."
        layers.append(dec.LayerWeights(
            t(p + "input_layernorm.weight"),
            torch.cat([t(p + "self_attn.q_proj.weight"), t(p + "self_attn.k_proj.weight"),
                       t(p + "self_attn.v_proj.weight")]).contiguous(),
            t(p + "self_attn.q_norm.weight"), t(p + "self_attn.k_norm.weight"), t(p + "self_attn.o_proj.weight"),
            t(p + "post_attention_layernorm.weight"),
            torch.cat([t(p + "mlp.gate_proj.weight"), t(p + "mlp.up_proj.weight")]).contiguous(),
            t(p + "mlp.down_proj.weight")))
    embed = t("model.embed_tokens.weight")
    lm_head = embed if shape.tie_embeddings or "lm_head.weight" not in sd else t("lm_head.weight")
    w = dec.DecoderWeights(shape, embed, layers, t("model.norm.weight"), lm_head, dec.rope_inv_freq(shape, device))
    return w, path


def save_head(head, path: str) -> None:
    """Writes a scoring head as safetensors: the synthetic head (w1, b1, w2, b2) or the branch
    head (w_gu, w_row, bias_gain), with gate_scale[, attn_scale] and the scaled-softmax flag."""
    from safetensors.torch import save_file
    if isinstance(head, G.BranchHead):
        t = {"w_gu": head.w_gu.cpu(), "w_row": head.w_row.cpu(), "bias_gain": torch.tensor([float(head.bias_gain)])}
    else:
        t = {"w1": head.w1.cpu(), "b1": head.b1.cpu(), "w2": head.w2.cpu(), "b2": torch.tensor([head.b2])}
    t["gate_scale"] = head.gate_scale.cpu()
    if head.attn_scale is not None:
        t["attn_scale"] = head.attn_scale.cpu()
    t["scaled_softmax"] = torch.tensor([1 if head.scaled_softmax else 0], dtype=torch.int32)
    save_file({k: v.contiguous() for k, v in t.items()}, path)


def load_head(path: str, device):
    """A head written by save_head."""
    from safetensors.torch import load_file
    t = load_file(path, device="cpu")
    gs = t["gate_scale"].to(device, torch.float32)
    at = t["attn_scale"].to(device, torch.float32) if "attn_scale" in t else None
    if "w_gu" in t:
        return G.BranchHead(t["w_gu"].to(device, torch.bfloat16), t["w_row"].to(device, torch.bfloat16), gs, at,
                            bool(int(t["scaled_softmax"].item())) if "scaled_softmax" in t else True,
                            float(t["bias_gain"].item()) if "bias_gain" in t else 1.0)
    return G.ScoringHead(t["w1"].to(device, torch.bfloat16), t["b1"].to(device, torch.float32),
                         t["w2"].to(device, torch.float32), float(t["b2"].item()), gs, at,
                         bool(int(t["scaled_softmax"].item())) if "scaled_softmax" in t else False)


def _is_gate_checkpoint(checkpoint: str) -> bool:
    if checkpoint.endswith(".pt"):
        return True
    return os.path.isdir(checkpoint) and any(glob.glob(os.path.join(checkpoint, pat))
                                             for pat in ("swa_gate_*.pt", "gate_final.pt", "gate_step*.pt"))


def load_model(checkpoint: str = "random", base_model: Optional[str] = None, gate_layer: Optional[int] = None,
               gate_attn: str = "fa2", dtype=None, *, gate_path: Optional[str] = None, device="cuda",
               shape: Optional[dec.DecoderShape] = None) -> TokenGateModel:
    """One model object (load_model, inference.py:137-180).

    checkpoint: a trained gate in the reference's format — a gate *.pt file or a local run
    directory holding gate_*.pt (swa_gate_* > gate_final > gate_step*) — whose metadata names
    base_model and gate_layer (arguments override them); base_model must then be a local Qwen3
    checkpoint directory, and the adapter saved beside the gate is folded into its weights.
    Otherwise checkpoint is "random[:seed]" (a seeded Qwen3-1.7B-shaped decoder, or `shape`) or a
    local Qwen3 directory, with the synthetic scoring head or the head saved by save_head at
    gate_path; gate_layer defaults to 1 there.  gate_attn: "fa2" (this package's key-bias
    kernels; the reference's "flex" / "sdpa" paths do not exist here); dtype: bfloat16 only.
    Nothing is downloaded."""
    if dtype is not None and dtype != torch.bfloat16:
        raise ValueError("this library runs the decoder in torch.bfloat16 only")
    if gate_attn != "fa2":
        raise ValueError(f"gate_attn={gate_attn!r}: only 'fa2' (the key-bias HIP kernels) is available")
    if not checkpoint.startswith("random") and _is_gate_checkpoint(checkpoint):
        from tokengate_amd import checkpoint as C
        gpath = C.resolve_gate_path(checkpoint)
        head, meta = C.load_gate(gpath, device)
        base_model = base_model or meta.get("base_model")
        if not base_model:
            raise ValueError(f"{gpath} records no base_model in its metadata; pass base_model= explicitly")
        if gate_layer is None:
            gate_layer = meta.get("gate_layer")
            if gate_layer is None:
                raise ValueError(f"{gpath} records no gate_layer in its metadata; pass gate_layer= explicitly")
        gate_layer = int(gate_layer)
        if not os.path.isdir(base_model):
            raise FileNotFoundError(f"base_model {base_model!r} is not a local checkpoint directory "
                                    "(nothing is downloaded)")
        w, name = _load_hf_qwen3(base_model, device)
        C.load_adapter_for(w, gpath, meta)
        n2 = w.shape.n_layers - gate_layer - 1
        if tuple(head.gate_scale.shape) != (n2, w.shape.n_heads):
            raise ValueError(f"{gpath}: gate_scale {tuple(head.gate_scale.shape)} does not match (layers above "
                             f"gate layer {gate_layer}, heads) = ({n2}, {w.shape.n_heads})")
        if head.w_gu.shape[1] != w.shape.d_model:
            raise ValueError(f"{gpath}: scoring branch width {head.w_gu.shape[1]} != d_model {w.shape.d_model}")
        return TokenGateModel(w, head, gate_layer, name)
    gate_layer = 1 if gate_layer is None else int(gate_layer)
    src = base_model or checkpoint
    if src.startswith("random"):
        seed = int(src.split(":", 1)[1]) if ":" in src else 0
        w = dec.random_decoder(shape or dec.QWEN3_1P7B, seed=seed, device=device)
        name = f"random-init {'Qwen3-1.7B-shaped' if shape is None else 'custom'} decoder (seed {seed})"
    elif os.path.isdir(src):
        w, name = _load_hf_qwen3(src, device)
    else:
        raise FileNotFoundError(f"{src}: not 'random[:seed]' and not a local checkpoint directory "
                                "(nothing is downloaded)")
    n2 = w.shape.n_layers - gate_layer - 1
    if n2 < 1:
        raise ValueError(f"gate_layer {gate_layer} leaves no layer above it")
    head = load_head(gate_path, device) if gate_path else G.random_head(n2, w.shape.n_heads, device=device)
    if tuple(head.gate_scale.shape) != (n2, w.shape.n_heads):
        raise ValueError("the head's gate_scale does not match (layers above the gate, heads)")
    return TokenGateModel(w, head, gate_layer, name)
