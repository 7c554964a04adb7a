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

SOURCES = ["abi.hip", "summary.hip", "route.hip", "attn.hip", "decode.hip", "swap.hip", "ivf.hip",
           "tree.hip", "ccc.hip"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libssa_hip.so)")


FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wno-unused-function"]


def compile_cmd(src: Path, obj: Path) -> list[str]:
    return [hipcc(), f"--offload-arch={ARCH}", *FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src),
            "-o", str(obj)]


def _filtered(res) -> str:
    return "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                     if "packed-fp32-ops" not in l)


def build(verbose: bool = False) -> Path:
    """Compiles every source (in parallel, one object each) and links LIB (atomically replaced).
    Raises on a compiler or linker error."""
    from concurrent.futures import ThreadPoolExecutor
    objdir = ROOT / "_build" / f"obj{os.getpid()}"
    objdir.mkdir(parents=True, exist_ok=True)
    objs = [objdir / (Path(s).stem + ".o") for s in SOURCES]
    cmds = [compile_cmd(CSRC / s, o) for s, o in zip(SOURCES, objs)]
    with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1)) as pool:
        results = list(pool.map(lambda c: subprocess.run(c, capture_output=True, text=True), cmds))
    msgs = [_filtered(r) for r in results]
    for cmd, res, msg in zip(cmds, results, msgs):
        if res.returncode != 0:
            shutil.rmtree(objdir, ignore_errors=True)
            raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{msg}")
    tmp = LIB.with_name(LIB.name + f".tmp{os.getpid()}")
    # --no-undefined: a kernel whose host stub the compiler did not emit fails here, not at load
    link = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined",
            *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(link, capture_output=True, text=True)
    shutil.rmtree(objdir, ignore_errors=True)
    if res.returncode != 0:
        if tmp.exists():
            tmp.unlink()
        raise RuntimeError(f"link failed ({res.returncode}):\n{' '.join(link)}\n{_filtered(res)}")
    if verbose:
        for m in msgs + [_filtered(res)]:
            if m.strip():
                print(m, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
