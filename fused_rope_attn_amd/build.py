"""Build ``libfra.so`` (the gfx950 kernels + C ABI) in-tree with hipcc.

Usage: ``python -m fused_rope_attn_amd.build`` (or ``build()`` from Python).
The library lands next to this file, where ``_lib.py`` loads it from, so it
travels with the source tree.  Building needs hipcc but no GPU.
"""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "csrc", "fra_kernels.hip")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(HERE, "libfra.so")
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; set HIPCC or install ROCm")


def command(out: str = LIB) -> list:
    return [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        # packed fp32 VALU ops stay off: the compiler must not form
        # v_pk_{add,mul,fma}_f32 from the scalar fp32 code.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", INCLUDE,
        "-o", out,
        SRC,
    ]


def build(verbose: bool = False) -> str:
    """Compile the library; returns its path.  Always recompiles."""
    tmp = LIB + ".tmp"
    cmd = command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
