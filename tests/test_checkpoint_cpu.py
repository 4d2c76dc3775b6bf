"""Trained-gate checkpoints in the reference's file format (tokengate_amd.checkpoint), on the CPU.

The fixtures are written here in the layout save_gate produces (e2e_gate_module.py:402-430: the
finalized constants, the E2EGate state_dict with the float32 MLP scoring branch whose down_proj
is the absorbed (1, I) row, a metadata dict) and in the adapter layout of
collect_lora_state_dict (lora.py:247-259: model.layers.N.<module path>.delta / lora_A / lora_B).
Checked: the loaded head holds the bf16 images of the float32 weights (what CastLinear multiplies
with); every research variant load_gate rejects is rejected; gate-file resolution and adapter
pairing by name; a delta adapter folds into exactly the weight DeltaLinear evaluates, a LoRA adapter
into W + (A B)^T alpha / rank; load_model wires a gate .pt, a local Qwen3 directory and the
paired adapter together (no kernel is called).
"""
import json
import math
import os

import pytest
import numpy as np
import torch
import torch.nn.functional as F

from tokengate_amd import checkpoint as C
from tokengate_amd import decoder as dec
from tokengate_amd import gate as G

SHAPE = dec.DecoderShape(n_layers=3, d_model=64, n_heads=4, n_kv_heads=2, head_dim=16, d_ff=96, vocab=50)


def _gate_obj(shape=SHAPE, gate_layer=1, seed=0, **over):
    g = torch.Generator().manual_seed(seed)
    L2, H, d, inter = shape.n_layers - gate_layer - 1, shape.n_heads, shape.d_model, shape.d_ff
    sd = {"gate_scale": torch.randn(L2, H, generator=g), "attn_scale": torch.randn(L2, H, generator=g),
          "b_norm.weight": torch.tensor([1.25]), "agg_weights": torch.full((H,), 1.0 / H),
          "gate_branch.gate_proj.weight": torch.randn(inter, d, generator=g) * 0.1,
          "gate_branch.up_proj.weight": torch.randn(inter, d, generator=g) * 0.1,
          "gate_branch.down_proj.weight": torch.randn(1, inter, generator=g) * 0.1}
    obj = {"state_dict": sd, "d_model": d, "n_heads": H, "n_layers_bias": L2, "selection_mode": "topk",
           "tau": 0.5, "head_agg": "avg", "per_layer_gate": True, "learnable_sss_scale": True,
           "normed_gate": True, "use_attn_scale": True, "scaled_softmax_scale": True,
           "softplus_gate_scale": True, "shared_readout": True, "absorbed_readout": True,
           "readout_residual": False, "ste_factor": 0.0, "gate_branch_mode": "mlp",
           "metadata": {"gate_layer": gate_layer}}
    obj.update(over)
    return obj


def test_load_gate_holds_bf16_images(tmp_path):
    obj = _gate_obj()
    p = str(tmp_path / "gate_final.pt")
    torch.save(obj, p)
    head, meta = C.load_gate(p, device="cpu")
    sd = obj["state_dict"]
    assert isinstance(head, G.BranchHead) and head.split_gate_layer and head.scaled_softmax
    assert torch.equal(head.w_gu, torch.cat([sd["gate_branch.gate_proj.weight"],
                                             sd["gate_branch.up_proj.weight"]]).to(torch.bfloat16))
    assert torch.equal(head.w_row, sd["gate_branch.down_proj.weight"][0].to(torch.bfloat16))
    assert torch.equal(head.gate_scale, sd["gate_scale"]) and torch.equal(head.attn_scale, sd["attn_scale"])
    assert head.bias_gain == 1.25 and meta == {"gate_layer": 1}
    # the Phase-2 constants of the loaded gate follow the reference's bf16 chain (oracle.gate)
    from oracle import gate as og
    g = torch.Generator().manual_seed(3)
    T2 = 300
    kept = torch.randn(T2, generator=g)
    kept[:5] = 0                                                    # prefix rows
    ratio = torch.rand(T2, generator=g) * 0.5 + 0.5
    bias_raw, q_head, q_row = head.phase2_tables(kept, ratio, 0.25)
    temp = og.softplus32(sd["attn_scale"].numpy())
    b = (np.float32(1.25) * kept.numpy()).astype(np.float32)[:, None, None] * og.softplus32(sd["gate_scale"].numpy())[None]
    gb = og.bf16(b.astype(np.float32))
    for l in range(gb.shape[1]):
        want = og.phase2_bias(gb[:, l, :], temp[l], ratio.numpy()).T / np.float32(0.25)
        assert np.array_equal(bias_raw[l].numpy(), want.astype(np.float32))
        s_want = og.phase2_query_scale(temp[l], ratio.numpy())
        s_got = (q_head[l][:, None] * q_row[None, :]).to(torch.bfloat16).float().numpy()
        assert np.array_equal(s_got, s_want)


@pytest.mark.parametrize("over,match", [
    (dict(readout_residual=True), "readout_residual"), (dict(absorbed_readout=False), "absorbed_readout"),
    (dict(tanh_gate=True), "tanh_gate"), (dict(head_agg="learned"), "head_agg"),
    (dict(gate_cond="film"), "gate_cond"), (dict(selection_mode="adaptive"), "selection_mode"),
])
def test_load_gate_rejects_variants(tmp_path, over, match):
    p = str(tmp_path / "gate_final.pt")
    torch.save(_gate_obj(**over), p)
    with pytest.raises(ValueError, match=match):
        C.load_gate(p, device="cpu")


def test_load_gate_selection_mode(tmp_path):
    """selection_mode / tau are restored as E2EGate keeps them (load_gate, e2e_gate_module.py:482-488):
    top-K by default, the threshold mode with its tau."""
    p = str(tmp_path / "gate_final.pt")
    torch.save(_gate_obj(), p)
    head, _ = C.load_gate(p, device="cpu")
    assert head.selection_mode == "topk"
    torch.save(_gate_obj(selection_mode="threshold", tau=0.625), p)
    head, _ = C.load_gate(p, device="cpu")
    assert head.selection_mode == "threshold" and head.tau == 0.625
    obj = _gate_obj(selection_mode="threshold")
    del obj["tau"]
    torch.save(obj, p)
    assert C.load_gate(p, device="cpu")[0].tau == 0.5


def test_load_gate_rejects_missing_branch_and_post_proj(tmp_path):
    obj = _gate_obj()
    obj["state_dict"] = {k: v for k, v in obj["state_dict"].items() if not k.startswith("gate_branch.")}
    p = str(tmp_path / "gate_a.pt")
    torch.save(obj, p)
    with pytest.raises(ValueError, match="gate_branch"):
        C.load_gate(p, device="cpu")
    obj = _gate_obj()
    obj["state_dict"]["post_proj.weight"] = torch.zeros(2, 2)
    torch.save(obj, p)
    with pytest.raises(ValueError, match="post_proj"):
        C.load_gate(p, device="cpu")
    obj = _gate_obj()
    obj["state_dict"]["gate_branch.down_proj.weight"] = torch.zeros(SHAPE.d_model, SHAPE.d_ff)
    torch.save(obj, p)
    with pytest.raises(ValueError, match="branch shapes"):
        C.load_gate(p, device="cpu")


def test_resolve_and_adapter_pairing(tmp_path):
    d = str(tmp_path)
    for n in ("gate_step100.pt", "gate_step200.pt"):
        open(os.path.join(d, n), "wb").close()
    assert C.resolve_gate_path(d).endswith("gate_step200.pt")
    open(os.path.join(d, "gate_final.pt"), "wb").close()
    assert C.resolve_gate_path(d).endswith("gate_final.pt")
    open(os.path.join(d, "swa_gate_final.pt"), "wb").close()
    assert C.resolve_gate_path(d).endswith("swa_gate_final.pt")
    with pytest.raises(FileNotFoundError):
        C.resolve_gate_path(os.path.join(d, "nope.pt"))
    with pytest.raises(FileNotFoundError):
        C.resolve_gate_path("someone/some-hub-repo")
    assert C.find_adapter_path(os.path.join(d, "gate_final.pt")) is None
    open(os.path.join(d, "lora_final.pt"), "wb").close()
    open(os.path.join(d, "swa_lora_final.pt"), "wb").close()
    assert C.find_adapter_path(os.path.join(d, "gate_final.pt")).endswith("/lora_final.pt")
    assert C.find_adapter_path(os.path.join(d, "swa_gate_final.pt")).endswith("/swa_lora_final.pt")
    assert C.find_adapter_path(os.path.join(d, "gate_step100.pt")) is None     # never lora_final
    with pytest.raises(ValueError):
        C.find_adapter_path(os.path.join(d, "model.pt"))


def _delta_sd(shape, layers, seed=1):
    g = torch.Generator().manual_seed(seed)
    H, Hkv, D, d, f = shape.n_heads, shape.n_kv_heads, shape.head_dim, shape.d_model, shape.d_ff
    dims = {"self_attn.q_proj": (H * D, d), "self_attn.k_proj": (Hkv * D, d), "self_attn.v_proj": (Hkv * D, d),
            "self_attn.o_proj": (d, H * D), "mlp.gate_proj": (f, d), "mlp.up_proj": (f, d),
            "mlp.down_proj": (d, f)}
    return {f"model.layers.{i}.{t}.delta": torch.randn(*s, generator=g) * 0.003
            for i in layers for t, s in dims.items()}, dims


def test_delta_adapter_folds_to_the_evaluated_weight():
    """W' equals DeltaLinear's W + delta.to(W.dtype) bit for bit, so every projection is unchanged."""
    w = dec.random_decoder(SHAPE, seed=3, device="cpu")
    base = dec.random_decoder(SHAPE, seed=3, device="cpu")
    sd, dims = _delta_sd(SHAPE, [0, 2])
    assert C.fold_adapter(w, sd, "delta") == 14
    x = torch.randn(5, SHAPE.d_model).to(torch.bfloat16)
    for i in (0, 2):
        lw, lb = w.layers[i], base.layers[i]
        q = sd[f"model.layers.{i}.self_attn.q_proj.delta"]
        k = sd[f"model.layers.{i}.self_attn.k_proj.delta"]
        up = sd[f"model.layers.{i}.mlp.up_proj.delta"]
        Hd, Kd, f = SHAPE.n_heads * SHAPE.head_dim, SHAPE.n_kv_heads * SHAPE.head_dim, SHAPE.d_ff
        assert torch.equal(F.linear(x, lw.w_qkv[:Hd]), F.linear(x, lb.w_qkv[:Hd] + q.to(torch.bfloat16)))
        assert torch.equal(lw.w_qkv[Hd:Hd + Kd], lb.w_qkv[Hd:Hd + Kd] + k.to(torch.bfloat16))
        assert torch.equal(lw.w_gu[f:], lb.w_gu[f:] + up.to(torch.bfloat16))
        assert torch.equal(lw.w_down, lb.w_down + sd[f"model.layers.{i}.mlp.down_proj.delta"].to(torch.bfloat16))
    assert torch.equal(w.layers[1].w_qkv, base.layers[1].w_qkv)            # untouched layer


def test_lora_adapter_folds_within_bf16_rounding():
    w = dec.random_decoder(SHAPE, seed=4, device="cpu")
    base = dec.random_decoder(SHAPE, seed=4, device="cpu")
    g = torch.Generator().manual_seed(5)
    r, alpha, d = 4, 8.0, SHAPE.d_model
    Hd = SHAPE.n_heads * SHAPE.head_dim
    A = torch.randn(d, r, generator=g) * 0.1
    B = torch.randn(r, Hd, generator=g) * 0.1
    sd = {"model.layers.1.self_attn.q_proj.lora_A": A, "model.layers.1.self_attn.q_proj.lora_B": B}
    C.fold_adapter(w, sd, "lora", alpha)
    x = torch.randn(7, d)
    want = x @ base.layers[1].w_qkv[:Hd].float().t() + (x @ A @ B) * (alpha / r)
    got = x @ w.layers[1].w_qkv[:Hd].float().t()
    assert float((got - want).norm() / want.norm()) < 1e-2
    assert not torch.equal(w.layers[1].w_qkv[:Hd], base.layers[1].w_qkv[:Hd])
    with pytest.raises(ValueError, match="alpha"):
        C.fold_adapter(w, sd, "lora", None)
    with pytest.raises(ValueError, match="names no decoder linear"):
        C.fold_adapter(w, {"model.layers.1.self_attn.rotary.delta": torch.zeros(1)}, "delta")


def _write_hf_dir(path, shape, seed=7):
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(seed)
    H, Hkv, D, d, f = shape.n_heads, shape.n_kv_heads, shape.head_dim, shape.d_model, shape.d_ff
    sd = {"model.embed_tokens.weight": torch.randn(shape.vocab, d, generator=g),
          "model.norm.weight": torch.ones(d)}
    for i in range(shape.n_layers):
        p = f"model.layers.{i}."
        for n, s in (("self_attn.q_proj", (H * D, d)), ("self_attn.k_proj", (Hkv * D, d)),
                     ("self_attn.v_proj", (Hkv * D, d)), ("self_attn.o_proj", (d, H * D)),
                     ("mlp.gate_proj", (f, d)), ("mlp.up_proj", (f, d)), ("mlp.down_proj", (d, f))):
            sd[p + n + ".weight"] = torch.randn(*s, generator=g) * 0.02
        for n, s in (("input_layernorm", d), ("post_attention_layernorm", d), ("self_attn.q_norm", D),
                     ("self_attn.k_norm", D)):
            sd[p + n + ".weight"] = torch.ones(s)
    save_file({k: v.to(torch.bfloat16).contiguous() for k, v in sd.items()}, os.path.join(path, "model.safetensors"))
    cfg = dict(num_hidden_layers=shape.n_layers, hidden_size=d, num_attention_heads=H, num_key_value_heads=Hkv,
               head_dim=D, intermediate_size=f, vocab_size=shape.vocab, rms_norm_eps=1e-6, rope_theta=1e6,
               tie_word_embeddings=True)
    with open(os.path.join(path, "config.json"), "w") as fh:
        json.dump(cfg, fh)


def test_load_model_from_gate_checkpoint(tmp_path):
    from tokengate_amd import inference as I
    base = tmp_path / "qwen3"
    base.mkdir()
    _write_hf_dir(str(base), SHAPE)
    run = tmp_path / "run"
    run.mkdir()
    obj = _gate_obj(gate_layer=0)
    obj["metadata"] = {"base_model": str(base), "gate_layer": 0, "adapter_type": "delta"}
    torch.save(obj, str(run / "gate_final.pt"))
    sd, _ = _delta_sd(SHAPE, [0])
    with pytest.raises(FileNotFoundError, match="adapter"):
        I.load_model(str(run), device="cpu")           # adapter_type recorded, file missing
    torch.save(sd, str(run / "lora_final.pt"))
    m = I.load_model(str(run), device="cpu")
    assert m.gate_layer == 0 and isinstance(m.gate, G.BranchHead)
    plain, _ = I._load_hf_qwen3(str(base), "cpu")
    dq = sd["model.layers.0.self_attn.q_proj.delta"].to(torch.bfloat16)
    Hd = SHAPE.n_heads * SHAPE.head_dim
    assert torch.equal(m.weights.layers[0].w_qkv[:Hd], plain.layers[0].w_qkv[:Hd] + dq)
    assert torch.equal(m.weights.layers[1].w_qkv, plain.layers[1].w_qkv)
    with pytest.raises(ValueError, match="gate_scale"):
        I.load_model(str(run / "gate_final.pt"), gate_layer=1, device="cpu")   # head built for gate layer 0
    obj["metadata"] = {"gate_layer": 0}
    torch.save(obj, str(run / "gate_step5.pt"))
    with pytest.raises(ValueError, match="base_model"):
        I.load_model(str(run / "gate_step5.pt"), device="cpu")


def test_branch_head_save_load_roundtrip(tmp_path):
    from tokengate_amd import inference as I
    w = dec.random_decoder(SHAPE, seed=9, device="cpu")
    h = G.random_branch_head(w, 1, seed=2)
    h.bias_gain = 0.5
    p = str(tmp_path / "head.safetensors")
    I.save_head(h, p)
    h2 = I.load_head(p, "cpu")
    assert isinstance(h2, G.BranchHead) and h2.bias_gain == 0.5 and h2.scaled_softmax
    for a in ("w_gu", "w_row", "gate_scale", "attn_scale"):
        assert torch.equal(getattr(h, a), getattr(h2, a))
    assert math.isclose(float(h.w_row.float().std()), SHAPE.d_ff ** -0.5, rel_tol=0.3)
