"""MI355X-native (gfx950) TokenGate prefill hot path: key-bias attention and the gate path.

Subpackages:
  fa2bias  — the kernels/fa2bias boundary (flash_attn_key_bias, flash_attn_key_bias_varlen,
             available, ext, require_varlen) over the HIP kernels in csrc/.
"""
