"""The inference surface on the CPU: state-span sentinels, chat-template span marking, the
transformers Qwen3 checkpoint loader (safetensors; fused q|k|v and gate|up layouts), the head's
save / load round trip, and load_model's argument errors."""
import numpy as np
import pytest
import torch

from tokengate_amd import inference as I


def test_split_state_span():
    ids = [5, 6, I.STATE_START_ID, 7, 8, 9, I.STATE_END_ID, 10]
    clean, s, e = I.split_state_span(ids)
    assert clean == [5, 6, 7, 8, 9, 10] and (s, e) == (2, 5) and clean[s:e] == [7, 8, 9]
    for bad in ([1, 2, 3], [I.STATE_END_ID, 1, I.STATE_START_ID], [I.STATE_START_ID, I.STATE_START_ID, I.STATE_END_ID]):
        with pytest.raises(ValueError):
            I.split_state_span(bad)


class _Tok:
    """Character-level stand-in tokenizer (ids = code points)."""
    eos_token_id = 0

    def encode(self, text, add_special_tokens=False):
        return [ord(c) for c in text]

    def apply_chat_template(self, msgs, add_generation_prompt=True, tokenize=True, enable_thinking=False):
        return [1] + self.encode("U:" + msgs[0]["content"]) + [2]

    def decode(self, ids, skip_special_tokens=True):
        return "".join(chr(i) for i in ids if i > 2)


def test_apply_chat_template_marks_the_state():
    tok = _Tok()
    ids = I.apply_chat_template(tok, "Q {state} A", state="doc")
    clean, s, e = I.split_state_span(ids)
    assert "".join(chr(c) for c in clean[s:e]) == "doc"
    assert clean == I.apply_chat_template(tok, "Q doc A")
    raw = I.apply_chat_template(tok, "x{state}y", use_chat_template=False, state="zz")
    c2, s2, e2 = I.split_state_span(raw)
    assert c2 == [ord("x"), ord("z"), ord("z"), ord("y")] and (s2, e2) == (1, 3)
    with pytest.raises(ValueError):
        I.apply_chat_template(tok, "no placeholder", state="doc")


def test_find_article_boundaries():
    assert I.find_article_boundaries([1, 2, 9, 9, 3], [1, 2, 3]) == (2, 1)
    assert I.compute_prunable_span([1, 2, 9, 9, 3], [1, 2, 3]) == (2, 4)
    assert I.find_article_boundaries([1, 2], [1, 2]) == (2, 0)


def test_load_transformers_qwen3_checkpoint(tmp_path):
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen3Config(hidden_size=256, intermediate_size=384, num_attention_heads=4,
                                   num_key_value_heads=2, head_dim=128, num_hidden_layers=2, vocab_size=101,
                                   rms_norm_eps=1e-6, tie_word_embeddings=True)
    torch.manual_seed(0)
    m = transformers.Qwen3ForCausalLM(cfg).to(torch.bfloat16)
    with torch.no_grad():
        for p in m.parameters():
            p.normal_(0, 0.05)
    m.save_pretrained(str(tmp_path), safe_serialization=True)
    w, _ = I._load_hf_qwen3(str(tmp_path), "cpu")
    s = w.shape
    assert (s.n_layers, s.d_model, s.n_heads, s.n_kv_heads, s.head_dim, s.d_ff, s.vocab) == (2, 256, 4, 2, 128, 384, 101)
    L = m.model.layers[1]
    assert torch.equal(w.layers[1].w_qkv, torch.cat([L.self_attn.q_proj.weight, L.self_attn.k_proj.weight,
                                                       L.self_attn.v_proj.weight]))
    assert torch.equal(w.layers[1].w_gu, torch.cat([L.mlp.gate_proj.weight, L.mlp.up_proj.weight]))
    assert torch.equal(w.layers[1].w_down, L.mlp.down_proj.weight)
    assert torch.equal(w.layers[1].q_norm, L.self_attn.q_norm.weight)
    assert torch.equal(w.embed, m.model.embed_tokens.weight) and w.lm_head is w.embed
    assert torch.equal(w.final_norm, m.model.norm.weight)
    inv = 1.0 / (s.rope_theta ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))
    assert torch.equal(w.inv_freq, inv)


def test_head_round_trip(tmp_path):
    from tokengate_amd import gate as G
    g = torch.Generator().manual_seed(1)
    h = G.ScoringHead(torch.randn(256, 2048, generator=g).to(torch.bfloat16), torch.randn(256, generator=g),
                      torch.randn(256, generator=g), 0.25, torch.randn(26, 16, generator=g), torch.randn(26, 16, generator=g))
    I.save_head(h, str(tmp_path / "head.safetensors"))
    h2 = I.load_head(str(tmp_path / "head.safetensors"), "cpu")
    for a in ("w1", "b1", "w2", "gate_scale", "attn_scale"):
        assert torch.equal(getattr(h, a), getattr(h2, a))
    assert h2.b2 == 0.25


def test_load_model_argument_errors():
    with pytest.raises(ValueError, match="fa2"):
        I.load_model("random", gate_attn="flex", device="cpu")
    with pytest.raises(ValueError, match="bfloat16"):
        I.load_model("random", dtype=torch.float32, device="cpu")
    with pytest.raises(FileNotFoundError):
        I.load_model("no/such/dir", device="cpu")
