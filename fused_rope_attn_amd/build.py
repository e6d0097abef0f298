"""Build ``libfra.so`` (the gfx950 kernels + C ABI) in-tree with hipcc.

Usage: ``python -m fused_rope_attn_amd.build`` (or ``build()`` from Python).
The library lands next to this file, where ``_lib.py`` loads it from, so it
travels with the source tree.  Building needs hipcc but no GPU.
"""
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
# Forward (fra_kernels.hip: kernels, dispatch and most of the C ABI) and
# backward (fra_bwd.hip) translation units, compiled in parallel.
SRCS = [os.path.join(CSRC, "fra_kernels.hip"), os.path.join(CSRC, "fra_bwd.hip")]
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(HERE, "libfra.so")
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; set HIPCC or install ROCm")


def compile_command(src: str, obj: str) -> list:
    return [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-c",
        # packed fp32 VALU ops stay off: the compiler must not form
        # v_pk_{add,mul,fma}_f32 from the scalar fp32 code.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", INCLUDE,
        "-I", CSRC,
        "-o", obj,
        src,
    ]


def link_command(objs: list, out: str) -> list:
    return [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", out] + objs


def _clean(stderr: str) -> str:
    return "\n".join(l for l in stderr.splitlines() if "packed-fp32-ops" not in l)


def build(verbose: bool = False) -> str:
    """Compile the library; returns its path.  Always recompiles."""
    with tempfile.TemporaryDirectory(prefix="fra_build_") as tmpd:
        objs = [os.path.join(tmpd, os.path.basename(s) + ".o") for s in SRCS]
        cmds = [compile_command(s, o) for s, o in zip(SRCS, objs)]
        if verbose:
            for c in cmds:
                print(" ".join(c), flush=True)
        procs = [subprocess.Popen(c, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True) for c in cmds]
        errs = []
        for c, pr in zip(cmds, procs):
            _, err = pr.communicate()
            if pr.returncode != 0:
                errs.append(f"hipcc failed ({pr.returncode}) on {c[-1]}:\n{_clean(err)}")
            elif verbose and _clean(err).strip():
                print(_clean(err), file=sys.stderr)
        if errs:
            raise RuntimeError("\n".join(errs))
        tmp = LIB + ".tmp"
        cmd = link_command(objs, tmp)
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc link failed ({res.returncode}):\n{_clean(res.stderr)}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
