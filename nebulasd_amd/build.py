"""Build the gfx950 C-ABI library ``nebulasd_amd/_lib/libnsd_attn.so`` in-tree.

``python -m nebulasd_amd.build`` (or ``__graft_entry__.build()``) runs one
``hipcc`` line over the HIP kernels and the host planner.  Every HIP source
is compiled with packed-fp32 instructions disabled
(``-Xclang -target-feature -Xclang -packed-fp32-ops``).
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
LIB_DIR = PKG / "_lib"
LIB_PATH = LIB_DIR / "libnsd_attn.so"
SOURCES = ["nsd_host.cpp", "nsd_prologue.hip", "nsd_attention.hip", "nsd_prefill.hip", "nsd_blocks.hip", "nsd_hostkv.hip",
           "nsd_layer.hip", "nsd_probe.hip", "nsd_decoder.hip", "nsd_gemm.hip"]
LIBS: list[str] = []  # the HIP runtime only
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the gfx950 kernels)")


COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", f"-I{ROOT / 'include'}", f"-I{CSRC}"]
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-Wno-unused-command-line-argument",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def compile_commands(obj_dir: Path) -> list[list[str]]:
    """One command per source: HIP sources through hipcc, host C++ through g++."""
    cmds = []
    for src in SOURCES:
        obj = obj_dir / (Path(src).stem + ".o")
        if src.endswith(".hip"):
            cmds.append([hipcc(), *HIP_FLAGS, *COMMON, "-c", str(CSRC / src), "-o", str(obj)])
        else:
            cmds.append(["g++", *COMMON, "-c", str(CSRC / src), "-o", str(obj)])
    return cmds


def link_command(obj_dir: Path, out: Path) -> list[str]:
    objs = [str(obj_dir / (Path(s).stem + ".o")) for s in SOURCES]
    return [hipcc(), f"--offload-arch={ARCH}", "--hip-link", "-shared", "-fPIC", *objs, *LIBS, "-o", str(out)]


def _run(cmds: list[list[str]], verbose: bool) -> None:
    procs = []
    for cmd in cmds:
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
    errors = []
    for cmd, proc in procs:
        out, err = proc.communicate()
        if proc.returncode != 0:
            errors.append(f"{' '.join(cmd)}\n{out}\n{err}")
        elif verbose and err.strip():
            print(err, file=sys.stderr)
    if errors:
        raise RuntimeError("build failed:\n" + "\n".join(errors))


def build(verbose: bool = False) -> Path:
    """Compile the library (always recompiles) and return its path."""
    LIB_DIR.mkdir(exist_ok=True)
    obj_dir = PKG / "_build"
    obj_dir.mkdir(exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run(compile_commands(obj_dir), verbose)
    _run([link_command(obj_dir, tmp)], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
