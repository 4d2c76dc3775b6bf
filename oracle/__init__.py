"""CPU oracle of the TokenGate prefill hot path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import anything from
here, and only as the reference that results are compared against (or the timed CPU baseline),
never as the product path.  The
product (tokengate_amd) never imports this package and fails loudly when its HIP library is
missing.

Modules
  attention — key-bias causal GQA attention, forward (out, LSE) and backward (dQ, dK, dV, dBias),
              evaluated in float64 numpy from the bf16-rounded inputs.
  gate      — top-K selection with the lower-index tie rule, keep indices, pack (hidden, KV,
              positions, bias, cu_seqlens), the synthetic scoring head, the ssmax ratio.

Pinning (what checks each function, see tests/test_oracle_*.py):
  attention fwd/LSE  — torch SDPA (is_causal / additive float mask) and torch.logsumexp on the
                       same inputs; bias-shift invariance; -1e9 key removal; GQA vs repeat.
  attention bwd      — torch autograd through SDPA with a float mask (dQ, dK, dV, dmask ->
                       dBias); central finite differences on tiny inputs.
  top-K / keep       — brute-force enumeration on tiny inputs; torch.topk on tie-free inputs;
                       invariants (ascending, unique, prefix/suffix kept, count).
  pack               — per-row brute-force gather; padded-vs-varlen equivalence.
  scoring head       — torch.nn.functional linear/silu on the same weights.
  ssmax ratio        — closed form at hand-computed points.
Tie order of torch.topk is implementation-defined; the lower-index rule is this library's stated
rule and is pinned by brute force, not by the reference (parity of ties with the reference's
torch.topk is unpinned).
"""
