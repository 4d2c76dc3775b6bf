"""Build the gfx950 C-ABI library (libtokengate_hip.so) into the fa2bias SITE directory.

Stands in for kernels/fa2bias/build.py (which downloads the flash-attn 2.8.3.post1 sdist, patches
it and compiles CUDA, build.py:40-148): here every kernel is this package's own HIP source under
csrc/, compiled with hipcc for gfx950 only, linked into one shared library, and stamped with the
ABI in BUILD_INFO.json next to it (build.py:152 writes the same stamp).

    python -m tokengate_amd.build            # compile into SITE (FA2BIAS_SITE overrides)
"""
import concurrent.futures as cf
import json
import os
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"

sys.path.insert(0, str(HERE / "fa2bias"))
from site_path import ABI, BUILD_INFO, LIB_NAME, SITE  # noqa: E402

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # Packed fp32 VALU ops are kept out of every kernel (hipcc would otherwise form them from
    # float2 code); the host pass warns that it does not know the feature, which is harmless.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def sources():
    return sorted(CSRC.glob("*.hip"))


def _compile(src: pathlib.Path, obj: pathlib.Path) -> None:
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr}")


def build(site: str = SITE, jobs: int = 8, verbose: bool = True) -> pathlib.Path:
    site = pathlib.Path(site)
    site.mkdir(parents=True, exist_ok=True)
    objdir = site / "_obj"
    objdir.mkdir(exist_ok=True)
    srcs = sources()
    objs = [objdir / (s.stem + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=min(jobs, len(srcs))) as ex:
        list(ex.map(lambda so: _compile(*so), zip(srcs, objs)))
    out = site / LIB_NAME
    tmp = site / (LIB_NAME + ".tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, out)
    shutil.rmtree(objdir, ignore_errors=True)
    (site / BUILD_INFO).write_text(json.dumps({"abi": ABI, "arch": ARCH, "lib": LIB_NAME}))
    if verbose:
        print(f"[build] {LIB_NAME} -> {site}", flush=True)
    return out


if __name__ == "__main__":
    build()
