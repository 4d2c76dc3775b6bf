"""ctypes binding of the C ABI declared in include/tokengate_hip.h.

The library is loaded from the fa2bias SITE directory (FA2BIAS_SITE overrides).  Every call
raises RuntimeError with the library's own message when the entry point returns nonzero.
Nothing here falls back to another implementation: a missing library is an error.
"""
import ctypes as C
import os
import threading

from tokengate_amd.fa2bias.site_path import LIB_NAME, SITE

_lock = threading.Lock()
_lib = None

vp, i32, i64, f32 = C.c_void_p, C.c_int32, C.c_int64, C.c_float

# name -> argtypes, in header order.  Keep in step with include/tokengate_hip.h.
SIGNATURES = {
    "tg_abi_version": [],
    "tg_last_error": [],
    "tg_keybias_fwd": [vp, vp, vp, vp, vp, vp,
                       i32, i32, i32, i32, i32, i32,
                       i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64,
                       i64, i64, f32, i32, vp, i64, vp],
    "tg_keybias_fwd_workspace_size": [i32, i32, i32, i32, i32, i32],
    "tg_keybias_fwd_noalloc": [vp, vp, vp, vp, vp, vp,
                               i32, i32, i32, i32, i32, i32,
                               i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64,
                               i64, i64, f32, i32, vp],
    "tg_keybias_varlen_fwd": [vp, vp, vp, vp, vp, vp, vp,
                              i32, i32, i32, i32, i32, i32,
                              i64, i64, i64, i64, i64, i64, i64, i64,
                              i64, i64, f32, i32, vp, i64, vp],
    "tg_keybias_varlen_fwd_workspace_size": [i32, i32, i32, i32, i32],
    "tg_keybias_varlen_kv_fwd": [vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                 i32, i32, i32, i32, i32, i32, i32,
                                 i64, i64, i64, i64, i64, i64, i64, i64,
                                 i64, i64, f32, i32, vp, i64, vp],
    "tg_keybias_varlen_kv_fwd_workspace_size": [i32, i32, i32, i32, i32, i32],
    "tg_keybias_bwd": [vp] * 12 + [i32] * 6 + [vp, f32, i32, vp],
    "tg_keybias_varlen_bwd": [vp] * 13 + [i32] * 6 + [vp, f32, i32, vp],
    "tg_gate_score_mlp": [vp, i64, i64, i32, i32, vp, vp, vp, f32, vp, vp],
    "tg_gate_score_mlp_ktiled": [vp, i64, i64, i32, i32, vp, vp, vp, f32, vp, vp],
    "tg_gate_topk_keep": [vp, vp, i32, i32, vp, vp, vp],
    "tg_gate_pack": [vp, i32, vp, vp, i32, i64, vp, vp, vp, f32, vp, vp],
    "tg_gate_select_pack": [vp, vp, vp, i32, i32, i32, vp, i32, i64, vp, vp, vp, f32, vp, i32, i32, vp],
    "tg_gate_select_pack_workspace_size": [i32, i32],
    "tg_gate_threshold_select": [vp, vp, i32, vp, i32, f32, f32, f32, vp, vp, vp, vp, vp],
    "tg_rmsnorm": [vp, i64, vp, i64, vp, i64, vp, vp, i64, i64, i32, f32, vp],
    "tg_qk_norm_rope": [vp, i64, vp, i64, i32, i32, i32, vp, vp, f32, vp, vp, vp, vp, i64, vp, i64, vp, i64, vp,
                        vp],
    "tg_silu_mul": [vp, i64, i64, i32, vp, i64, vp],
    "tg_gate_branch_readout": [vp, i64, i64, i32, vp, vp, vp],
    "tg_lm_head": [vp, i64, i32, vp, i64, i32, vp, i64, vp],
    "tg_linear_rows": [vp, i64, i32, vp, i64, i32, vp, i64, vp],
    "tg_linear_rows_norm": [vp, i64, vp, i64, vp, i64, vp, f32, i32, vp, i64, i32, vp, i64, i32, vp],
    "tg_linear_rows_swiglu": [vp, i64, i32, i32, vp, i64, vp, i64, vp],
    "tg_argmax_rows": [vp, i64, i32, i64, vp, vp],
}
RESTYPES = {"tg_last_error": C.c_char_p, "tg_keybias_fwd_workspace_size": C.c_int64,
            "tg_keybias_varlen_fwd_workspace_size": C.c_int64, "tg_keybias_varlen_kv_fwd_workspace_size": C.c_int64,
            "tg_gate_select_pack_workspace_size": C.c_int64}


def lib_path(site: str = None) -> str:
    return os.path.join(site or SITE, LIB_NAME)


def load(site: str = None):
    """Load (once) and return the ctypes library with argtypes set."""
    global _lib
    with _lock:
        if _lib is not None and site is None:
            return _lib
        path = lib_path(site)
        if not os.path.exists(path):
            raise RuntimeError(f"{LIB_NAME} is not built ({path}): build it with "
                               f"`python -m tokengate_amd.build`")
        lib = C.CDLL(path)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = RESTYPES.get(name, C.c_int)
        if site is None:
            _lib = lib
        return lib


def fwd_workspace(size_fn: str, device, *size_args):
    """Device workspace for the forward's key-range split (tg_keybias_fwd / tg_keybias_varlen_fwd),
    or None when the library plans no split for these sizes.  Returns (tensor, pointer, bytes)."""
    n = int(getattr(load(), size_fn)(*size_args))
    if n <= 0:
        return None, None, 0
    import torch
    ws = torch.empty(n, dtype=torch.uint8, device=device)
    return ws, ws.data_ptr(), n


SELECT_PACK_ERROR_OFFSET = 8   # byte offset of tg_gate_select_pack's wait-timeout flag (global word 2)


def call(name: str, *args) -> None:
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.tg_last_error().decode(errors="replace")
        raise RuntimeError(f"{name}: {msg}")
