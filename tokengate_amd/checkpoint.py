"""Trained TokenGate gate checkpoints in the reference's own file format.

A gate checkpoint is the dict that save_gate writes with torch.save
(tokengate/e2e_gate/gate_module/e2e_gate_module.py:402-430): the E2EGate state_dict (gate_scale,
attn_scale, b_norm.weight, agg_weights and the scoring branch gate_branch.{gate,up,down}_proj.weight
in float32), the architecture fields and a metadata dict (base_model, gate_layer, adapter_type,
lora_start_layer, lora_alpha, ...).  It is read here with torch.load(weights_only=True), which
builds tensors and plain containers only.

load_gate follows the reference's load_gate (:433-525): the finalized architecture is the only one
accepted, research variants are rejected by name, and the branch must be present.  Its weights are
float32 storage whose compute runs in the input dtype (CastLinear, :89-141), so the bf16 copies
kept here are exactly the weights the reference multiplies with.

The backbone adapter paired with a gate by file name (find_adapter_path, lora.py:262-284) is folded
into the decoder weights at load time: a delta adapter computes F.linear(x, W + bf16(delta))
(DeltaLinear, lora.py:83-116), so W' = bf16(W + bf16(delta)) is the same weight; a LoRA adapter adds
(x A B) * alpha / rank in bf16 (LoRALinear, :49-80), folded as W' = bf16(W + (A B)^T alpha / rank),
which differs from the unmerged evaluation at the bf16-ulp level (the reference's own
merge_adapters_into_layers, :196-229, makes the same trade).
"""
import glob
import os
import re
from typing import Dict, Optional, Tuple

import torch

from tokengate_amd import gate as G

# (key, required value, default when absent): load_gate's _require list (e2e_gate_module.py:459-477)
_FINALIZED = [
    ("n_input_layers", 1, 1), ("score_source", "hidden", "hidden"), ("learned_agg", False, False),
    ("tanh_gate", False, False), ("qk_norm_scale", False, False), ("softplus_sss", False, False),
    ("sss_frozen_gate_scale", False, False), ("ste_factor", 0.0, 0.0), ("normed_gate", True, True),
    ("use_attn_scale", True, True), ("scaled_softmax_scale", True, True), ("softplus_gate_scale", True, True),
    ("shared_readout", True, True), ("absorbed_readout", True, True), ("readout_residual", False, False),
    ("gate_branch_mode", "mlp", "mlp"), ("head_agg", "avg", "avg"), ("per_layer_gate", True, True),
    ("learnable_sss_scale", True, True),
]


def resolve_gate_path(checkpoint: str) -> str:
    """A gate .pt path, or a local run directory where the newest-stage gate wins:
    swa_gate_* > gate_final > gate_step* (_resolve_gate_path, tokengate/inference.py:38-59).
    Nothing is downloaded: a Hub id that is not a local directory raises."""
    if checkpoint.endswith(".pt"):
        if not os.path.isfile(checkpoint):
            raise FileNotFoundError(f"gate checkpoint not found: {checkpoint}")
        return checkpoint
    if not os.path.isdir(checkpoint):
        raise FileNotFoundError(f"{checkpoint}: not a gate .pt file or a local run directory "
                                "(nothing is downloaded)")
    for pat in ("swa_gate_*.pt", "gate_final.pt", "gate_step*.pt"):
        hits = sorted(glob.glob(os.path.join(checkpoint, pat)))
        if hits:
            return hits[-1]
    raise FileNotFoundError(f"no gate checkpoint (gate_*.pt) in {checkpoint}")


def read_checkpoint(path: str) -> dict:
    """The saved dict, through the loader that builds tensors and plain containers only."""
    obj = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(obj, dict) or "state_dict" not in obj:
        raise ValueError(f"{path}: not a gate checkpoint (a dict with a state_dict)")
    return obj


def load_gate(path: str, device="cuda") -> Tuple[G.BranchHead, Dict]:
    """(BranchHead, metadata) of a saved finalized gate (load_gate, e2e_gate_module.py:433-525)."""
    obj = read_checkpoint(path)
    for key, want, default in _FINALIZED:
        got = obj.get(key, default)
        if got != want:
            raise ValueError(f"Checkpoint {path} has {key}={got!r}; the finalized gate requires {key}={want!r}")
    gc = obj.get("gate_cond", "none")
    if gc not in ("none", None) or obj.get("use_boundary_cond", False):
        raise ValueError(f"Checkpoint {path} uses removed gate_cond={gc!r}; only gate_cond='none' gates are supported")
    mode = obj.get("selection_mode", "topk")
    if mode not in ("topk", "threshold"):
        raise ValueError(f"selection_mode must be 'topk' or 'threshold', got {mode!r}")
    sd = obj["state_dict"]
    if "post_proj.weight" in sd:
        raise ValueError(f"checkpoint {path!r} carries post_proj.weight (removed post-top-K projection)")
    names = ("gate_branch.gate_proj.weight", "gate_branch.up_proj.weight", "gate_branch.down_proj.weight")
    if not any(k.startswith("gate_branch.") for k in sd):
        raise ValueError(f"checkpoint {path!r} carries no gate_branch.* weights — the finalized gate "
                         "scores through the 'mlp' branch")
    for n in names:
        if n not in sd:
            raise ValueError(f"checkpoint {path!r}: missing {n}")
    gp, up, dp = (sd[n] for n in names)
    inter, d = gp.shape
    if up.shape != (inter, d) or dp.shape != (1, inter):
        raise ValueError(f"checkpoint {path!r}: branch shapes gate {tuple(gp.shape)}, up {tuple(up.shape)}, "
                         f"down {tuple(dp.shape)} are not (I, d), (I, d), (1, I)")
    if int(obj.get("d_model", d)) != d:
        raise ValueError(f"checkpoint {path!r}: d_model {obj.get('d_model')} != branch width {d}")
    H, L2 = int(obj.get("n_heads", 1)), int(obj.get("n_layers_bias", 0))
    gs, at = sd["gate_scale"].float(), sd["attn_scale"].float()
    if L2 <= 0 or gs.shape != (L2, H) or at.shape != (L2, H):
        raise ValueError(f"checkpoint {path!r}: gate_scale / attn_scale must be (n_layers_bias, n_heads) = ({L2}, {H})")
    agg = sd.get("agg_weights")
    if agg is not None and not torch.allclose(agg.float(), torch.full((H,), 1.0 / H)):
        raise ValueError(f"checkpoint {path!r}: agg_weights are not the uniform head mean")
    gain = sd.get("b_norm.weight")
    bf = torch.bfloat16
    head = G.BranchHead(torch.cat([gp, up]).to(device=device, dtype=bf).contiguous(),
                        dp[0].to(device=device, dtype=bf).contiguous(), gs.to(device), at.to(device), True,
                        float(gain.reshape(-1)[0]) if gain is not None else 1.0)
    # E2EGate(selection_mode=..., tau=...) as load_gate restores them (e2e_gate_module.py:482-488)
    head.selection_mode = mode
    head.tau = float(obj.get("tau", 0.5))
    return head, dict(obj.get("metadata", {}) or {})


def find_adapter_path(gate_path: str) -> Optional[str]:
    """The adapter saved with a gate, by name, in the same directory: gate_X.pt -> lora_X.pt,
    swa_gate_X.pt -> swa_lora_X.pt (lora.py:262-284); None when absent."""
    d = os.path.dirname(os.path.abspath(gate_path))
    base = os.path.basename(gate_path)
    if base.startswith("swa_gate_"):
        cand = "swa_lora_" + base[len("swa_gate_"):]
    elif base.startswith("gate_"):
        cand = "lora_" + base[len("gate_"):]
    else:
        raise ValueError(f"cannot infer the paired adapter file for gate checkpoint name {base!r} "
                         "(expected gate_*.pt or swa_gate_*.pt)")
    p = os.path.join(d, cand)
    return p if os.path.exists(p) else None


def lora_alpha_for(gate_path: str, meta: Dict) -> float:
    """alpha from the gate metadata, else the run's params.json (_lora_alpha_for,
    benchmark_gate_e2e.py:603-617)."""
    if meta.get("lora_alpha"):
        return float(meta["lora_alpha"])
    pj = os.path.join(os.path.dirname(os.path.abspath(gate_path)), "params.json")
    if os.path.exists(pj):
        import json
        with open(pj) as f:
            la = json.load(f).get("lora_alpha")
        if la:
            return float(la)
    raise ValueError(f"lora_alpha not in gate meta and no params.json with it next to {gate_path}")


_KEY = re.compile(r"(?:^|\.)layers\.(\d+)\.(self_attn\.[qkvo]_proj|mlp\.(?:gate|up|down)_proj)\."
                  r"(delta|delta_bias|lora_A|lora_B)$")


def _slot(weights, layer: int, target: str):
    """(tensor holding the target's rows, row offset) in the fused layout."""
    s = weights.shape
    lw = weights.layers[layer]
    qd, kd = s.n_heads * s.head_dim, s.n_kv_heads * s.head_dim
    return {"self_attn.q_proj": (lw.w_qkv, 0), "self_attn.k_proj": (lw.w_qkv, qd),
            "self_attn.v_proj": (lw.w_qkv, qd + kd), "self_attn.o_proj": (lw.w_o, 0),
            "mlp.gate_proj": (lw.w_gu, 0), "mlp.up_proj": (lw.w_gu, s.d_ff),
            "mlp.down_proj": (lw.w_down, 0)}[target]


@torch.no_grad()
def fold_adapter(weights, sd: Dict[str, torch.Tensor], adapter_type: str, alpha: Optional[float] = None) -> int:
    """Adds a delta or LoRA adapter state dict into the decoder weights in place; returns the
    number of linears changed.  Every adapter key must land on a linear of the decoder."""
    groups: Dict[Tuple[int, str], Dict[str, torch.Tensor]] = {}
    for k, v in sd.items():
        m = _KEY.search(k)
        if m is None:
            if k.rsplit(".", 1)[-1] in ("delta", "delta_bias", "lora_A", "lora_B"):
                raise ValueError(f"adapter key {k!r} names no decoder linear")
            continue
        groups.setdefault((int(m.group(1)), m.group(2)), {})[m.group(3)] = v
    n_layers = weights.shape.n_layers
    for (layer, target), parts in sorted(groups.items()):
        if layer >= n_layers:
            raise ValueError(f"adapter covers layer {layer}; the decoder has {n_layers}")
        if "delta_bias" in parts:
            raise ValueError("adapter carries delta_bias; the decoder's linears have no bias")
        w, r0 = _slot(weights, layer, target)
        if adapter_type == "delta":
            if "delta" not in parts:
                raise ValueError(f"layer {layer} {target}: delta adapter without a delta tensor")
            dl = parts["delta"].to(w.device)
            rows = w[r0:r0 + dl.shape[0]]
            if dl.shape != rows.shape:
                raise ValueError(f"layer {layer} {target}: delta {tuple(dl.shape)} vs weight {tuple(rows.shape)}")
            rows.copy_(rows + dl.to(w.dtype))                   # bf16(W + bf16(delta)), as DeltaLinear
        elif adapter_type == "lora":
            if alpha is None:
                raise ValueError("a LoRA adapter needs alpha")
            A, B = parts["lora_A"].float().to(w.device), parts["lora_B"].float().to(w.device)
            upd = (A @ B).t() * (float(alpha) / B.shape[0])     # (out, in), scaling = alpha / rank
            rows = w[r0:r0 + upd.shape[0]]
            if upd.shape != rows.shape:
                raise ValueError(f"layer {layer} {target}: LoRA update {tuple(upd.shape)} vs weight "
                                 f"{tuple(rows.shape)}")
            rows.copy_((rows.float() + upd).to(w.dtype))
        else:
            raise ValueError(f"adapter_type {adapter_type!r}: 'delta' or 'lora'")
    return len(groups)


def load_adapter_for(weights, gate_path: str, meta: Dict) -> Optional[str]:
    """Folds the adapter paired with gate_path into weights (load_gate_model,
    benchmark_gate_e2e.py:661-697); returns its path, or None when the gate has none.  A gate whose
    metadata names an adapter_type without the paired file raises."""
    p = find_adapter_path(gate_path)
    if p is None:
        if meta.get("adapter_type"):
            raise FileNotFoundError(f"{gate_path} was trained with adapter_type={meta['adapter_type']!r} but no "
                                    "paired adapter file exists next to it")
        return None
    sd = torch.load(p, map_location="cpu", weights_only=True)
    kind = meta.get("adapter_type") or "lora"
    fold_adapter(weights, sd, kind, lora_alpha_for(gate_path, meta) if kind == "lora" else None)
    return p
