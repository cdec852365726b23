"""Build libqmla.so in-tree with hipcc for gfx950 (MI355X).

    python qwen-mla-vllm_amd/build.py

Writes qwen-mla-vllm_amd/qmla/libqmla.so (atomically, via a temporary file and rename).
"""
from __future__ import annotations

import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "qmla" / "libqmla.so"
COMMON_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # no packed-fp32 VALU forms anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# (source, extra flags). MFMA accumulators stay in VGPRs: the online-softmax rescale touches them
# with VALU ops, and AGPR-resident accumulators make the compiler copy them back and forth.
SOURCES = [
    (CSRC / "qmla_decode.hip", ["-mllvm", "-amdgpu-mfma-vgpr-form"]),
    # these decode kernels' softmax never sees a NaN (masked scores are -inf, infinities stay honoured):
    # no canonicalizing v_max before every fmaxf of the tile maxima (measured no gain on qmla_decode)
    (CSRC / "qmla_cs.hip", ["-mllvm", "-amdgpu-mfma-vgpr-form", "-fno-honor-nans"]),
    (CSRC / "qmla_ws.hip", ["-mllvm", "-amdgpu-mfma-vgpr-form", "-fno-honor-nans"]),
    (CSRC / "qmla_ro.hip", ["-mllvm", "-amdgpu-mfma-vgpr-form", "-fno-honor-nans"]),
    (CSRC / "qmla_wsb.hip", ["-mllvm", "-amdgpu-mfma-vgpr-form", "-fno-honor-nans"]),
    (CSRC / "qmla_write.hip", []),
    (CSRC / "qmla_prep.hip", []),
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in (r.stderr or "").splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{errs}")
    if verbose and errs.strip():
        print(errs, file=sys.stderr)


def build(verbose: bool = False) -> pathlib.Path:
    """Compile every source to an object (in parallel), link libqmla.so, replace it atomically."""
    tag = f"tmp{os.getpid()}"
    objdir = PKG / "qmla" / f".obj_{tag}"
    objdir.mkdir(exist_ok=True)
    inc = [f"-I{REPO / 'include'}", f"-I{CSRC}"]
    tmp = OUT.with_suffix(f".so.{tag}")
    try:
        objs, procs = [], []
        for src, extra in SOURCES:
            obj = objdir / (src.stem + ".o")
            cmd = [hipcc(), *COMMON_FLAGS, *extra, *inc, "-c", str(src), "-o", str(obj)]
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
            objs.append(obj)
        failed = []
        for cmd, pr in procs:
            _, err = pr.communicate()
            err = "\n".join(l for l in (err or "").splitlines() if "packed-fp32-ops" not in l)
            if pr.returncode != 0:
                failed.append(f"{' '.join(cmd)}\n{err}")
            elif verbose and err.strip():
                print(err, file=sys.stderr)
        if failed:
            raise RuntimeError("hipcc failed:\n" + "\n".join(failed))
        _run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)], verbose)
        os.replace(tmp, OUT)
    finally:
        if tmp.exists():
            tmp.unlink()
        shutil.rmtree(objdir, ignore_errors=True)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
