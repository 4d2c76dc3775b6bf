"""The drop-in boundary on the CPU: availability, ABI stamp, exported symbols, argument errors and
fake kernels — the behaviours the reference's kernels/fa2bias/keybias.py has without a GPU."""
import ctypes
import json
import os
import re
import shutil
import subprocess
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_symbols():
    syms = []
    for name in os.listdir(os.path.join(ROOT, "include")):
        if name.endswith(".h"):
            text = open(os.path.join(ROOT, "include", name)).read()
            syms += re.findall(r"^\s*(?:int64_t|int|const\s+char\s*\*|void)\s*(tg_\w+)\s*\(", text, flags=re.M)
    return sorted(set(syms))


def test_library_exports_every_header_symbol():
    from tokengate_amd import _lib
    syms = _header_symbols()
    assert "tg_keybias_fwd" in syms and "tg_abi_version" in syms
    lib = ctypes.CDLL(_lib.lib_path())
    for s in syms:
        assert hasattr(lib, s), f"{s} declared in include/ but not exported"
    assert set(syms) == set(_lib.SIGNATURES), "ctypes signature table out of step with the header"


def test_abi_version_and_stamp():
    from tokengate_amd import _lib
    from tokengate_amd.fa2bias.site_path import ABI, BUILD_INFO, SITE
    assert _lib.load().tg_abi_version() == ABI
    assert json.load(open(os.path.join(SITE, BUILD_INFO)))["abi"] == ABI


def _run_py(code, env_extra):
    env = dict(os.environ, **env_extra)
    env["PYTHONPATH"] = ROOT
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, cwd=ROOT, timeout=300)
    return r


def test_available_false_and_ext_raises_without_build(tmp_path):
    code = ("from tokengate_amd.fa2bias import keybias as kb\n"
            "assert not kb.available()\n"
            "try:\n    kb.ext()\nexcept RuntimeError as e:\n    print('ERR', e)\n")
    r = _run_py(code, {"FA2BIAS_SITE": str(tmp_path)})
    assert r.returncode == 0, r.stderr
    assert "ERR" in r.stdout and "tokengate_amd.build" in r.stdout


def test_require_varlen_rejects_old_abi(tmp_path):
    from tokengate_amd import _lib
    shutil.copy(_lib.lib_path(), tmp_path / os.path.basename(_lib.lib_path()))
    (tmp_path / "BUILD_INFO.json").write_text(json.dumps({"abi": 1}))
    code = ("from tokengate_amd.fa2bias import keybias as kb\n"
            "assert kb.available()\n"
            "try:\n    kb.require_varlen()\nexcept RuntimeError as e:\n    print('ERR', e)\n")
    r = _run_py(code, {"FA2BIAS_SITE": str(tmp_path)})
    assert r.returncode == 0, r.stderr
    assert "ERR" in r.stdout and "ABI 1" in r.stdout
    (tmp_path / "BUILD_INFO.json").unlink()   # no stamp reads as ABI 1 too
    r = _run_py(code, {"FA2BIAS_SITE": str(tmp_path)})
    assert "ABI 1" in r.stdout


def test_require_varlen_accepts_current_build():
    from tokengate_amd.fa2bias import keybias
    keybias.require_varlen()


def test_c_abi_rejects_bad_head_dim_without_touching_the_gpu():
    from tokengate_amd import _lib
    lib = _lib.load()
    rc = lib.tg_keybias_fwd(16, 16, 16, None, 16, 16, 1, 8, 8, 2, 1, 64,
                            0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 1.0, 1, None, 0, None)
    assert rc != 0 and b"head_dim" in lib.tg_last_error()
    rc = lib.tg_keybias_fwd(16, 16, 16, None, 16, 16, 1, 8, 8, 3, 2, 128,
                            0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 1.0, 1, None, 0, None)
    assert rc != 0 and b"divide" in lib.tg_last_error()


def test_lm_head_rejects_bad_arguments_without_touching_the_gpu():
    from tokengate_amd import _lib
    lib = _lib.load()
    # (x, x_row_stride, n_rows, weight, vocab, dim, out, out_row_stride, stream); pointers are
    # never dereferenced: every check fails before a launch
    cases = [((16, 2048, 0, 16, 1000, 2048, 16, 1000, None), b"rows"),
             ((16, 2048, 9, 16, 1000, 2048, 16, 1000, None), b"rows"),
             ((16, 2048, 1, 16, 1000, 2000, 16, 1000, None), b"multiple of 512"),
             ((16, 1024, 1, 16, 1000, 2048, 16, 1000, None), b"strides"),
             ((None, 2048, 1, 16, 1000, 2048, 16, 1000, None), b"null"),
             ((8, 2048, 1, 16, 1000, 2048, 16, 1000, None), b"aligned")]
    for args, msg in cases:
        rc = lib.tg_lm_head(*args)
        assert rc != 0 and msg in lib.tg_last_error(), (args, lib.tg_last_error())
        rc = lib.tg_linear_rows(*args)
        assert rc != 0 and msg in lib.tg_last_error(), ("linear_rows", args, lib.tg_last_error())


def test_argmax_rows_rejects_bad_arguments_without_touching_the_gpu():
    from tokengate_amd import _lib
    lib = _lib.load()
    # (x, x_row_stride, n_rows, n_cols, out, stream)
    cases = [((None, 1000, 1, 1000, 16, None), b"null"), ((16, 1000, 1, 0, 16, None), b"n_cols"),
             ((16, 999, 1, 1000, 16, None), b"stride"), ((16, 1002, 1, 1000, 16, None), b"stride"),
             ((8, 1000, 1, 1000, 16, None), b"aligned")]
    for args, msg in cases:
        rc = lib.tg_argmax_rows(*args)
        assert rc != 0 and msg in lib.tg_last_error(), (args, lib.tg_last_error())


def test_select_pack_layout_and_keys_per_thread():
    """gate.plan's chunking for tg_gate_select_pack: 4 keys per thread (chunks of 2048 scores) for
    small batches (every span at most 32768 scores, at most 64 chunks in all), else the smallest of
    8 / 16 / 32 that keeps every span within 64 chunks; the C ABI rejects other values before any
    launch."""
    from tokengate_amd import _lib, gate
    lay = gate._select_layout
    assert lay([32448]) == (4, [0, 16])
    assert lay([32768] * 4) == (4, [0, 16, 32, 48, 64])
    assert lay([0, 100, 0]) == (4, [0, 0, 1, 1])
    assert lay([32769]) == (8, [0, 9])
    assert lay([32768] * 5) == (8, [0, 8, 16, 24, 32, 40])
    assert lay([64 * 4096]) == (8, [0, 64])
    assert lay([64 * 4096 + 1]) == (16, [0, 33])
    assert lay([64 * 16384, 5]) == (32, [0, 64, 65])
    assert lay([64 * 16384 + 1]) == (0, None)
    lib = _lib.load()
    for kpt in (2, 6, 64):
        rc = lib.tg_gate_select_pack(16, 16, 16, 1, 1, kpt, None, 0, 1, 16, None, None, 1e-6, 256, 1, 1, None)
        assert rc != 0 and b"keys_per_thread" in lib.tg_last_error()


def test_fwd_workspace_size_queries():
    """The split workspace is planned only for grids that leave the chip idle, and never for
    invalid sizes; the size queries make no GPU call."""
    from tokengate_amd import _lib
    lib = _lib.load()
    assert lib.tg_keybias_fwd_workspace_size(0, 4096, 4096, 16, 8, 1) == 0
    assert lib.tg_keybias_fwd_workspace_size(1, 4096, 4096, 16, 7, 1) == 0
    assert lib.tg_keybias_varlen_fwd_workspace_size(1, 0, 16, 8, 1) == 0
    # 32k causal fills the chip with 8-wave workgroups: no split
    assert lib.tg_keybias_fwd_workspace_size(1, 32768, 32768, 16, 8, 1) == 0
    # a 4k causal prompt fills the resident slots (no split); Phase 2 at K=2000 (2320 rows) and one
    # decode row over a long cache leave most of them empty and are split
    assert lib.tg_keybias_fwd_workspace_size(1, 4096, 4096, 16, 8, 1) == 0
    assert lib.tg_keybias_fwd_workspace_size(1, 2320, 2320, 16, 8, 1) > 0
    assert lib.tg_keybias_varlen_fwd_workspace_size(1, 2320, 16, 8, 1) > 0
    assert lib.tg_keybias_fwd_workspace_size(1, 1, 32768, 16, 8, 1) > 0
    # too few key tiles to split
    assert lib.tg_keybias_fwd_workspace_size(1, 1, 128, 16, 8, 1) == 0


def test_fwd_split_fits_the_resident_slots():
    """Every split plan keeps its chunks within the resident-workgroup slots, so its partials need
    at most CUs x 73,728 bytes (18 MiB at the 256 CUs assumed without a GPU): the bound behind the
    static scratch of tg_keybias_fwd_noalloc.  Grids of more than half the slots (a few thousand
    rows over a long cache) once planned 1.5x that."""
    from tokengate_amd import _lib
    lib = _lib.load()
    bound = 256 * 73728
    worst = 0
    for sq in (1, 3, 17, 500, 1000, 1500, 2000, 2320, 2500, 2800, 3000, 3072, 3500, 4000, 4096, 6000, 8192):
        for sk in (sq, 4096, 9000, 32768, 131072):
            if sk < sq:
                continue
            for b in (1, 2, 4):
                for causal in (0, 1):
                    n = lib.tg_keybias_fwd_workspace_size(b, sq, sk, 16, 8, causal)
                    worst = max(worst, n)
                    assert 0 <= n <= bound, (b, sq, sk, causal, n)
    for sq in (1, 700, 2320, 3000, 9000):
        n = lib.tg_keybias_varlen_fwd_workspace_size(3, sq, 16, 8, 1)
        assert 0 <= n <= bound, (sq, n)
    # the shapes that exceeded the scratch before the cap still split, inside the bound
    for args in ((1, 3072, 32768, 16, 8, 1), (1, 3072, 4096, 16, 8, 0), (1, 3000, 32768, 16, 8, 1)):
        assert 0 < lib.tg_keybias_fwd_workspace_size(*args) <= bound, args
    assert worst > 0


def test_python_checks_match_reference_messages():
    from tokengate_amd.fa2bias.keybias import ext
    q = torch.zeros(1, 8, 2, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 8, 1, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="CUDA device"):
        ext().fwd(q, k, k, None, None, 0.0, 0.1, True, -1, -1, 0.0, False, None)
    with pytest.raises(RuntimeError, match="fp16 and bf16"):
        ext().fwd(q.float(), k.float(), k.float(), None, None, 0.0, 0.1, True, -1, -1, 0.0, False, None)


def test_fake_kernels_give_reference_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode
    import tokengate_amd.fa2bias.keybias  # noqa: F401
    with FakeTensorMode():
        q = torch.empty(2, 100, 16, 128, dtype=torch.bfloat16)
        k = torch.empty(2, 100, 8, 128, dtype=torch.bfloat16)
        b = torch.empty(2, 16, 100)
        out, lse = torch.ops.recursive_kvs.fa2_keybias_fwd(q, k, k, b, 0.1, True)
        assert out.shape == q.shape and lse.shape == (2, 16, 100) and lse.dtype == torch.float32
        dq, dk, dv, db = torch.ops.recursive_kvs.fa2_keybias_bwd(q, q, k, k, q, lse, b, 0.1, True)
        assert dq.shape == q.shape and dk.shape == k.shape and db.shape == b.shape
        qv = torch.empty(300, 16, 128, dtype=torch.bfloat16)
        kv = torch.empty(300, 8, 128, dtype=torch.bfloat16)
        cu = torch.empty(4, dtype=torch.int32)
        ov, lv = torch.ops.recursive_kvs.fa2_keybias_varlen_fwd(qv, kv, kv, torch.empty(3, 16, 128), cu, 128, 0.1, True)
        assert ov.shape == qv.shape and lv.shape == (16, 300)
