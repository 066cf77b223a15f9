"""Build libnanokv_hip.so in-tree with hipcc for gfx950.

Usage: python -m nanokv_amd.build   (also called by __graft_entry__.build()).

Each .hip source is compiled to an object with its own floating-point
contraction policy, then all objects are linked into one shared library
next to this file.  Nothing here runs at import time.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
LIB_NAME = "libnanokv_hip.so"
ARCH = "gfx950"

# Sources and their extra flags.  The codec TU holds bit-exact restatements
# (quantiser, decode epilogue), so fp contraction is off there.
SOURCES = {
    "nkv_abi.hip": [],
    "nkv_codec.hip": ["-ffp-contract=off"],
    # MFMA accumulators in VGPRs: the fused kernel's softmax/rescale VALU work
    # runs on them every tile, and its read-only decoder fragments fill AGPRs
    "nkv_attend.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    # scores are never NaN (-inf masks are kept): fmaxf needs no NaN quieting
    "nkv_chunk.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1", "-fno-honor-nans"],
    "nkv_fast.hip": [],
    # the partition merges keep the reference's unfused fp32 products
    "nkv_merge.hip": ["-ffp-contract=off"],
    # RoPE rounds every fp64 product and sum separately, as the oracle does
    "nkv_rope.hip": ["-ffp-contract=off"],
    "nkv_camera.hip": ["-ffp-contract=off"],
}

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    # no packed-fp32 code generation (v_pk_*_f32) anywhere in this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the NanoKV HIP library cannot be built")
    return path


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that noise
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops' is not a recognized feature" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source and link the library; returns its path."""
    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)
    cc = hipcc()
    cmds = []
    objs = []
    for src, extra in SOURCES.items():
        obj = objdir / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([cc, *COMMON, *extra, "-c", str(CSRC / src), "-o", str(obj)])
    procs = []
    for cmd in cmds:
        if verbose:
            print(" ".join(cmd), file=sys.stderr)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                            stderr=subprocess.STDOUT, text=True)))
    errors = []
    for cmd, proc in procs:
        out, _ = proc.communicate()
        out = "\n".join(l for l in out.splitlines()
                        if "packed-fp32-ops' is not a recognized feature" not in l)
        if proc.returncode != 0:
            errors.append(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
        elif out.strip():
            print(out, file=sys.stderr)
    if errors:
        raise RuntimeError("\n".join(errors))
    lib = HERE / LIB_NAME
    tmp = HERE / (LIB_NAME + ".tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
