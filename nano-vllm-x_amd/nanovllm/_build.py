"""Build libnvx_spec.so (all HIP sources under csrc/) for gfx950 with hipcc.

Run ``python -m nanovllm._build`` (with nano-vllm-x_amd/ on sys.path) or call
``build()``.  The library is written in-tree to nanovllm/_lib/ so it travels with
the source tree.
"""
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR.parent / "csrc"
INCLUDE = PKG_DIR.parent.parent / "include"
LIB_DIR = PKG_DIR / "_lib"
LIB_PATH = LIB_DIR / "libnvx_spec.so"
SOURCES = ["capi.hip", "ngram.hip", "kvcache.hip", "sampler.hip", "attention.hip", "fused.hip", "draft.hip"]
ARCH = "gfx950"


def hipcc_path():
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build libnvx_spec.so")


def build(verbose=True):
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [
        hipcc_path(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
        # Packed fp32 VALU ops are kept out of every kernel.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-result", f"-I{INCLUDE}", f"-I{CSRC}",
        *[str(CSRC / s) for s in SOURCES], "-o", str(tmp),
    ]
    if verbose:
        print("[nanovllm build]", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines()
            if "packed-fp32-ops" not in ln]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[nanovllm build] wrote {LIB_PATH}", flush=True)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
