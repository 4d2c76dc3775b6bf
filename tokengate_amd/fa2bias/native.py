"""The object ext() returns: FA2-compatible positional entry points over the C ABI.

The reference binds flash-attn 2.8.3's pybind module (`flash_attn_keybias_cuda`), whose
`fwd / bwd / varlen_fwd / varlen_bwd` take torch tensors positionally
(kernels/fa2bias/keybias.py:43, 56-57, 93-94, 107-109).  This class keeps those positional
signatures and their validation (the patched mha_fwd / mha_bwd checks, keybias.patch:18, 39-63,
94), allocates outputs with torch on the caller's device, and launches the gfx950 kernels through
ctypes on torch's current stream.  Tensors are never copied to make them fit: a layout the
kernels cannot read raises RuntimeError, as the reference's TORCH_CHECKs do.
"""
import ctypes

import torch

from tokengate_amd import _lib


def _check(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _check_qkv(q, k, v):
    _check(q.dtype in (torch.float16, torch.bfloat16), "FlashAttention only support fp16 and bf16 data type")
    _check(k.dtype == q.dtype, "query and key must have the same dtype")
    _check(v.dtype == q.dtype, "query and value must have the same dtype")
    _check(q.is_cuda and k.is_cuda and v.is_cuda, "Input tensor must be on CUDA device")
    _check(q.stride(-1) == 1 and k.stride(-1) == 1 and v.stride(-1) == 1,
           "Input tensor must have contiguous last dimension")
    _check(q.dtype == torch.bfloat16 and q.shape[-1] == 128,
           "this library supports bf16 with head_dim 128 only")


def _check_unsupported(p_dropout, window_size_left, window_size_right, softcap, return_softmax):
    # The reference build compiles these features out (kernels/fa2bias/build.py:137-138).
    _check(p_dropout == 0.0, "this library does not support dropout")
    _check(window_size_left < 0 and window_size_right < 0, "this library does not support local attention")
    _check(softcap == 0.0, "this library does not support softcap")
    _check(not return_softmax, "this library does not return the softmax")


def _check_bias(bias, batch, heads, seqlen_k, what="key bias"):
    _check(bias.dtype == torch.float32, f"{what} must have dtype fp32")
    _check(bias.is_cuda, f"{what} must be on CUDA device")
    _check(bias.stride(-1) == 1, f"{what} must have contiguous last dimension")
    _check(tuple(bias.shape) == (batch, heads, seqlen_k),
           f"{what} must have shape (batch_size, num_heads, seqlen_k)")


class KeyBiasExt:
    """fwd / varlen_fwd (and bwd / varlen_bwd) with flash-attn 2.8.3's positional signatures."""

    def fwd(self, q, k, v, out_, alibi_slopes_, p_dropout, softmax_scale, is_causal,
            window_size_left, window_size_right, softcap, return_softmax, gen_):
        _check_qkv(q, k, v)
        _check_unsupported(p_dropout, window_size_left, window_size_right, softcap, return_softmax)
        _check(q.dim() == 4 and k.dim() == 4 and v.dim() == 4, "q, k, v must be (batch, seqlen, heads, head_dim)")
        B, Sq, H, D = q.shape
        Sk, Hkv = k.shape[1], k.shape[2]
        _check(tuple(k.shape) == (B, Sk, Hkv, D) and tuple(v.shape) == (B, Sk, Hkv, D), "k and v shape mismatch")
        _check(H % Hkv == 0, "Number of heads in key/value must divide number of heads in query")
        bias = alibi_slopes_
        if bias is not None:
            _check_bias(bias, B, H, Sk)
        if out_ is not None:
            out = out_
            _check(out.dtype == q.dtype and tuple(out.shape) == tuple(q.shape) and out.stride(-1) == 1,
                   "out must match q in dtype and shape, with contiguous last dimension")
        else:
            out = torch.empty_like(q)
        lse = torch.empty((B, H, Sq), dtype=torch.float32, device=q.device)
        if B and Sq:
            ws, ws_ptr, ws_bytes = _lib.fwd_workspace("tg_keybias_fwd_workspace_size", q.device, B, Sq, Sk, H, Hkv,
                                                      int(bool(is_causal)))
            _lib.call("tg_keybias_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(),
                      bias.data_ptr() if bias is not None else None, out.data_ptr(), lse.data_ptr(),
                      B, Sq, Sk, H, Hkv, D,
                      q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1), k.stride(2),
                      v.stride(0), v.stride(1), v.stride(2), out.stride(0), out.stride(1), out.stride(2),
                      bias.stride(0) if bias is not None else 0, bias.stride(1) if bias is not None else 0,
                      float(softmax_scale), int(bool(is_causal)), ws_ptr, ws_bytes, _stream(q))
        return [out, lse, torch.empty(0, device=q.device), torch.empty(0, device=q.device)]

    def varlen_fwd(self, q, k, v, out_, cu_seqlens_q, cu_seqlens_k, seqused_k, leftpad_k, block_table_,
                   alibi_slopes_, max_seqlen_q, max_seqlen_k, p_dropout, softmax_scale, zero_tensors,
                   is_causal, window_size_left, window_size_right, softcap, return_softmax, gen_):
        _check_qkv(q, k, v)
        _check_unsupported(p_dropout, window_size_left, window_size_right, softcap, return_softmax)
        _check(seqused_k is None and leftpad_k is None and block_table_ is None,
               "seqused_k, leftpad_k and block_table are not supported")
        _check(cu_seqlens_q.data_ptr() == cu_seqlens_k.data_ptr() and max_seqlen_q == max_seqlen_k,
               "this library runs self-attention over one cu_seqlens (q and k must share it)")
        _check(cu_seqlens_q.dtype == torch.int32 and cu_seqlens_q.is_cuda and cu_seqlens_q.is_contiguous(),
               "cu_seqlens_q must have dtype int32, live on the device and be contiguous")
        _check(q.dim() == 3 and k.dim() == 3 and v.dim() == 3, "varlen q, k, v must be (total, heads, head_dim)")
        total, H, D = q.shape
        Hkv = k.shape[1]
        _check(k.shape[0] == total and tuple(v.shape) == tuple(k.shape), "k and v shape mismatch")
        _check(H % Hkv == 0, "Number of heads in key/value must divide number of heads in query")
        nseq = cu_seqlens_q.numel() - 1
        bias = alibi_slopes_
        if bias is not None:
            _check_bias(bias, nseq, H, max_seqlen_k, "key bias (num_seqs, num_heads, max_seqlen_k)")
        out = out_ if out_ is not None else torch.empty_like(q)
        if zero_tensors:
            out.zero_()
        lse = torch.empty((H, total), dtype=torch.float32, device=q.device)
        if nseq > 0 and total > 0 and max_seqlen_q > 0:
            ws, ws_ptr, ws_bytes = _lib.fwd_workspace("tg_keybias_varlen_fwd_workspace_size", q.device, nseq,
                                                      int(max_seqlen_q), H, Hkv, int(bool(is_causal)))
            _lib.call("tg_keybias_varlen_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(),
                      bias.data_ptr() if bias is not None else None, out.data_ptr(), lse.data_ptr(),
                      cu_seqlens_q.data_ptr(), nseq, int(max_seqlen_q), total, H, Hkv, D,
                      q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
                      out.stride(0), out.stride(1),
                      bias.stride(0) if bias is not None else 0, bias.stride(1) if bias is not None else 0,
                      float(softmax_scale), int(bool(is_causal)), ws_ptr, ws_bytes, _stream(q))
        return [out, lse, torch.empty(0, device=q.device), torch.empty(0, device=q.device)]

    def bwd(self, dout, q, k, v, out, softmax_lse, dq_, dk_, dv_, alibi_slopes_, p_dropout, softmax_scale,
            is_causal, window_size_left, window_size_right, softcap, deterministic, gen_, rng_state):
        _check_qkv(q, k, v)
        _check_unsupported(p_dropout, window_size_left, window_size_right, softcap, False)
        _check(dout.dtype == q.dtype and out.dtype == q.dtype, "dout and out must have the dtype of q")
        _check(dout.stride(-1) == 1 and out.stride(-1) == 1, "dout and out must have contiguous last dimension")
        B, Sq, H, D = q.shape
        Sk, Hkv = k.shape[1], k.shape[2]
        _check(tuple(dout.shape) == tuple(q.shape) and tuple(out.shape) == tuple(q.shape), "dout/out shape mismatch")
        _check(tuple(softmax_lse.shape) == (B, H, Sq) and softmax_lse.dtype == torch.float32
               and softmax_lse.is_contiguous(), "softmax_lse must be contiguous fp32 (batch, heads, seqlen_q)")
        bias = alibi_slopes_
        if bias is not None:
            _check_bias(bias, B, H, Sk)
        dq = dq_ if dq_ is not None else torch.empty_like(q)
        dk = dk_ if dk_ is not None else torch.empty_like(k)
        dv = dv_ if dv_ is not None else torch.empty_like(v)
        for t, ref in ((dq, q), (dk, k), (dv, v)):
            _check(t.shape == ref.shape and t.dtype == ref.dtype and t.stride(-1) == 1, "gradient buffer mismatch")
        softmax_d = torch.empty((B, H, Sq), dtype=torch.float32, device=q.device)
        dbias = torch.empty((B, H, Sk), dtype=torch.float32, device=q.device) if bias is not None else None
        strides = []
        for t in (q, k, v, out, dout, dq, dk, dv):
            strides += [t.stride(0), t.stride(1), t.stride(2)]
        strides += [bias.stride(0), bias.stride(1)] if bias is not None else [0, 0]
        strides += [dbias.stride(0), dbias.stride(1)] if dbias is not None else [0, 0]
        arr = (ctypes.c_int64 * len(strides))(*strides)
        if B and Sq and Sk:
            _lib.call("tg_keybias_bwd", dout.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                      softmax_lse.data_ptr(), bias.data_ptr() if bias is not None else None,
                      dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                      dbias.data_ptr() if dbias is not None else None, softmax_d.data_ptr(),
                      B, Sq, Sk, H, Hkv, D, ctypes.cast(arr, ctypes.c_void_p), float(softmax_scale),
                      int(bool(is_causal)), _stream(q))
        elif B and Sq:
            dq.zero_()
            softmax_d.zero_()
        return [dq, dk, dv, softmax_d, dbias]

    def varlen_bwd(self, dout, q, k, v, out, softmax_lse, dq_, dk_, dv_, cu_seqlens_q, cu_seqlens_k,
                   alibi_slopes_, max_seqlen_q, max_seqlen_k, p_dropout, softmax_scale, zero_tensors, is_causal,
                   window_size_left, window_size_right, softcap, deterministic, gen_, rng_state):
        _check_qkv(q, k, v)
        _check_unsupported(p_dropout, window_size_left, window_size_right, softcap, False)
        _check(cu_seqlens_q.data_ptr() == cu_seqlens_k.data_ptr() and max_seqlen_q == max_seqlen_k,
               "this library runs self-attention over one cu_seqlens (q and k must share it)")
        _check(cu_seqlens_q.dtype == torch.int32 and cu_seqlens_q.is_cuda and cu_seqlens_q.is_contiguous(),
               "cu_seqlens_q must have dtype int32, live on the device and be contiguous")
        _check(dout.stride(-1) == 1 and out.stride(-1) == 1, "dout and out must have contiguous last dimension")
        total, H, D = q.shape
        Hkv = k.shape[1]
        nseq = cu_seqlens_q.numel() - 1
        _check(tuple(softmax_lse.shape) == (H, total) and softmax_lse.dtype == torch.float32
               and softmax_lse.is_contiguous(), "softmax_lse must be contiguous fp32 (heads, total)")
        bias = alibi_slopes_
        if bias is not None:
            _check_bias(bias, nseq, H, max_seqlen_k, "key bias (num_seqs, num_heads, max_seqlen_k)")
        dq = dq_ if dq_ is not None else torch.empty_like(q)
        dk = dk_ if dk_ is not None else torch.empty_like(k)
        dv = dv_ if dv_ is not None else torch.empty_like(v)
        if zero_tensors:
            dq.zero_(); dk.zero_(); dv.zero_()
        softmax_d = torch.empty((H, total), dtype=torch.float32, device=q.device)
        dbias = torch.zeros((nseq, H, max_seqlen_k), dtype=torch.float32, device=q.device) if bias is not None else None
        strides = []
        for t in (q, k, v, out, dout, dq, dk, dv):
            strides += [t.stride(0), t.stride(1)]
        strides += [bias.stride(0), bias.stride(1)] if bias is not None else [0, 0]
        strides += [dbias.stride(0), dbias.stride(1)] if dbias is not None else [0, 0]
        arr = (ctypes.c_int64 * len(strides))(*strides)
        if nseq > 0 and total > 0 and max_seqlen_q > 0:
            _lib.call("tg_keybias_varlen_bwd", dout.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                      out.data_ptr(), softmax_lse.data_ptr(), bias.data_ptr() if bias is not None else None,
                      dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                      dbias.data_ptr() if dbias is not None else None, softmax_d.data_ptr(),
                      cu_seqlens_q.data_ptr(), nseq, int(max_seqlen_q), total, H, Hkv, D,
                      ctypes.cast(arr, ctypes.c_void_p), float(softmax_scale), int(bool(is_causal)), _stream(q))
        return [dq, dk, dv, softmax_d, dbias]
