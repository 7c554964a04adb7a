"""Builds libssa_hip.so (the gfx950 kernels + C ABI) in-tree with hipcc.

    python -m ssa_amd.build            # -> ssa_amd/libssa_hip.so

The library is compiled for gfx950 only. Packed-fp32 instruction selection is disabled for all
device code (-packed-fp32-ops), so hipcc never emits v_pk_{add,mul,fma}_f32.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIB = PKG / "libssa_hip.so"
ARCH = "gfx950"

SOURCES = ["abi.hip", "summary.hip", "route.hip", "attn.hip", "decode.hip", "swap.hip", "ivf.hip"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libssa_hip.so)")


def compile_cmd(out: Path) -> list[str]:
    return [
        hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-shared", "-fPIC",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-function",
        f"-I{INCLUDE}", f"-I{CSRC}",
        *[str(CSRC / s) for s in SOURCES],
        "-o", str(out),
    ]


def build(verbose: bool = False) -> Path:
    """Compiles every source into LIB (atomically replaced). Raises on a compiler error."""
    tmp = LIB.with_name(LIB.name + f".tmp{os.getpid()}")
    cmd = compile_cmd(tmp)
    res = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                     if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        if tmp.exists():
            tmp.unlink()
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{msgs}")
    if verbose and msgs.strip():
        print(msgs, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
