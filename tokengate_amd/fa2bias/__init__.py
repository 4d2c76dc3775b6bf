"""Drop-in for the reference's kernels/fa2bias package: the key-bias FlashAttention boundary."""
