"""Writes gate_chain.npz: input/output vectors of the reference's gate-bias and Phase-2 transform
chain, produced by the reference's own functions (run in the build container only, where the
reference checkout exists; GPU runs and the tests read only the .npz).

Functions exercised (reference paths relative to its checkout):
  * E2EGate.forward / aggregate            tokengate/e2e_gate/gate_module/e2e_gate_module.py:348-399
    (Qwen3RMSNorm(1, eps=1e-6) over the sequence axis, times softplus(gate_scale); mean over heads)
  * build_gate_bias_vectorized             tokengate/e2e_gate/gate_module/gate_forward.py:968-1036
    (per_layer_gate branch, stored in the model dtype bf16)
  * _ssmax_ratio                           gate_forward.py:574-585
  * Qwen3FlexAttention._phase2_q_bias      tokengate/e2e_gate/attn/qwen3_flex_attention.py:433-473
    (scaled-softmax branch and the per-head temperature branch, bf16 query states)

The selection (top-K) is not taken from the reference here: its tie order is torch.topk's.  The
kept set is chosen by the caller (highest aggregate, lower position first among ties) and passed
in, so the vectors pin arithmetic only.

    python tests/golden/make_gate_chain_vectors.py      # rewrites tests/golden/gate_chain.npz
"""
import math
import os
import sys
import types

import numpy as np
import torch

REF = "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gate_chain.npz")


def main():
    sys.path.insert(0, REF)
    from tokengate.e2e_gate.gate_module.e2e_gate_module import E2EGate
    from tokengate.e2e_gate.gate_module.gate_forward import build_gate_bias_vectorized, _ssmax_ratio
    from tokengate.e2e_gate.attn.qwen3_flex_attention import Qwen3FlexAttention

    torch.manual_seed(0)
    g = torch.Generator().manual_seed(11)
    vec = {}
    # two articles: one of plain bf16-valued scores, one with many exact ties (few distinct values)
    cases = [dict(L=300, s=17, e=261, K=40, L2=3, H=4, D=8, ties=False),
             dict(L=200, s=5, e=180, K=60, L2=2, H=4, D=8, ties=True)]
    for ci, c in enumerate(cases):
        L, s, e, K, L2, H, D = c["L"], c["s"], c["e"], c["K"], c["L2"], c["H"], c["D"]
        n_art = e - s
        raw = torch.randn(n_art, 1, generator=g) * 2.5
        if c["ties"]:
            raw = torch.round(raw * 2) / 2
        raw = raw.to(torch.bfloat16).float()           # the branch's bf16 score cast to fp32
        gate = E2EGate(d_model=16, n_heads=H, n_layers_bias=L2)
        with torch.no_grad():
            gate.gate_scale.copy_(math.log(math.expm1(1.7)) + 0.4 * torch.randn(L2, H, generator=g))
            gate.attn_scale.copy_(math.log(math.expm1(1.0)) + 0.3 * torch.randn(L2, H, generator=g))
            b = gate(raw)                               # (n_art, L2, H) fp32
            agg = gate.aggregate(b)                     # (n_art,) fp32
        # kept set: K highest aggregates, lower position first among equal values
        order = np.lexsort((np.arange(n_art), -agg.double().numpy()))
        topk_local = torch.from_numpy(np.sort(order[:K]).astype(np.int64))
        keep = torch.cat([torch.arange(s), s + topk_local, torch.arange(e, L)])
        gb = build_gate_bias_vectorized(b, topk_local, s, e, keep, L, torch.bfloat16)   # (n_kept, L2, H)
        r = _ssmax_ratio(keep)                          # (1, n_kept) fp32
        n_kept = keep.numel()
        q = torch.randn(1, H, n_kept, D, generator=g).to(torch.bfloat16)
        at_eff = torch.nn.functional.softplus(gate.attn_scale.detach())    # attn_scale_eff (L2, H)
        q_ss, b_ss, q_ph, b_ph = [], [], [], []
        for l in range(L2):
            me = types.SimpleNamespace(gate_bias=gb[None, :, l, :], attn_scale=at_eff[l], ssmax_ratio=r,
                                       _gate_per_head=True)
            qo, bo, _ = Qwen3FlexAttention._phase2_q_bias(me, q)
            q_ss.append(qo)
            b_ss.append(bo)
            me.ssmax_ratio = None                       # the per-head temperature branch
            qo, bo, _ = Qwen3FlexAttention._phase2_q_bias(me, q)
            q_ph.append(qo)
            b_ph.append(bo)
        p = f"c{ci}_"
        vec.update({
            p + "geom": np.array([L, s, e, K, L2, H, D], np.int64),
            p + "raw": raw[:, 0].numpy(),
            p + "gate_scale": gate.gate_scale.detach().numpy(),
            p + "attn_scale": gate.attn_scale.detach().numpy(),
            p + "b": b.numpy(),
            p + "agg": agg.numpy(),
            p + "keep": keep.numpy(),
            p + "gb": gb.float().numpy(),
            p + "ratio": r[0].numpy(),
            p + "q": q.float().numpy(),
            p + "q_ssmax": torch.stack(q_ss).float().numpy(),
            p + "bias_ssmax": torch.stack(b_ss).float().numpy(),
            p + "q_perhead": torch.stack(q_ph).float().numpy(),
            p + "bias_perhead": torch.stack(b_ph).float().numpy(),
        })
    np.savez_compressed(OUT, **vec)
    print(f"wrote {OUT}: {len(vec)} arrays")


if __name__ == "__main__":
    main()
