"""Build ``libfra.so`` (the gfx950 kernels + C ABI) in-tree with hipcc.

Usage: ``python -m fused_rope_attn_amd.build`` (or ``build()`` from Python).
The library lands next to this file, where ``_lib.py`` loads it from, so it
travels with the source tree.  Building needs hipcc but no GPU.

Translation units, compiled in parallel:

* ``fra_fwd.hip`` and ``fra_bwd.hip`` -- argument checks, kernel choice and
  the C ABI (no kernels);
* ``fra_inst_fwd.hip`` and ``fra_inst_bwd.hip`` once per head_dim of
  ``FRA_HEAD_DIMS`` (``csrc/fra_fwd_types.h``), with ``-DFRA_HEAD_DIM=<D>``:
  that head_dim's forward and backward kernels.

``FRA_BUILD_DIMS=80,72`` (environment) builds only those head dims, for
quicker iteration on a kernel; the library then reports every other head_dim
as unsupported.  The default builds all.

The kernel units are compiled with the compiler's resource-usage remarks,
and the build fails if a kernel uses scratch memory (register spills) that
``SCRATCH_ALLOWED`` does not list: the instances the benchmark workloads run
must stay spill-free, and every known spill is listed with its size.
"""
import os
import re
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(HERE, "libfra.so")
ARCH = "gfx950"


# (mangled-name pattern, largest scratch bytes per lane allowed): instances
# that spill, all off the BASELINE workloads' paths -- head_dim 128 long
# kernels (fp32 full-width tables without the rotated-K workspace: up to 496
# B; with it 316 B; 16-bit or half-width tables: 8-20 B), head_dim 96 long
# kernels with fp32 full-width tables rotating K in the kernel (100-112 B),
# fp16 window kernels at head_dim 80 with two heads per workgroup (20-36 B),
# head_dim 96 window kernels with full-width tables (20-36 B) and the
# head_dim 96 backward long kernel (16 B).
SCRATCH_ALLOWED = [
    (r"long_kernelILi128E", 512),
    (r"long_kernelILi96E.*Li2ELb1ELb0E", 128),
    (r"window_kernelILi80ENS_3F16E", 64),
    (r"window_kernelILi96E.*ELb1ELi2E", 64),
    (r"bwd_long_kernelILi96E", 32),
]


def scratch_use(remarks: str) -> dict:
    """{kernel symbol: scratch bytes per lane} from -Rpass-analysis=kernel-resource-usage output."""
    out, cur = {}, None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur = m.group(1)
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and cur:
            out[cur] = int(m.group(1))
    return out


def check_scratch(use: dict) -> list:
    """Kernels whose scratch use SCRATCH_ALLOWED does not cover."""
    bad = []
    for name, nbytes in sorted(use.items()):
        if nbytes == 0:
            continue
        if not any(re.search(pat, name) and nbytes <= cap for pat, cap in SCRATCH_ALLOWED):
            bad.append(f"{name}: {nbytes} B/lane of scratch")
    return bad


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; set HIPCC or install ROCm")


def head_dims() -> list:
    """The head dims of FRA_HEAD_DIMS in csrc/fra_fwd_types.h (or FRA_BUILD_DIMS)."""
    env = os.environ.get("FRA_BUILD_DIMS", "").strip()
    if env:
        return [int(x) for x in env.split(",") if x.strip()]
    with open(os.path.join(CSRC, "fra_fwd_types.h")) as f:
        m = re.search(r"#define FRA_HEAD_DIMS\(X\)\s+(.*)", f.read())
    if not m:
        raise RuntimeError("FRA_HEAD_DIMS not found in fra_fwd_types.h")
    return [int(x) for x in re.findall(r"X\((\d+)\)", m.group(1))]


def compile_command(src: str, obj: str, defines=()) -> list:
    """hipcc line of one unit; ``defines`` are extra options (-D..., -mllvm ...)."""
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
        *defines,
        "-o", obj,
        src,
    ]


def link_command(objs: list, out: str) -> list:
    return [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", out] + objs


def _clean(stderr: str) -> str:
    return "\n".join(l for l in stderr.splitlines() if "packed-fp32-ops" not in l)


def units(tmpd: str) -> list:
    """(source, object, defines) of every translation unit."""
    dims = head_dims()
    common = []
    if os.environ.get("FRA_BUILD_DIMS", "").strip():
        common = ["-DFRA_HEAD_DIMS(X)=" + " ".join(f"X({d})" for d in dims)]
    out = [(os.path.join(CSRC, s), os.path.join(tmpd, s + ".o"), common) for s in ("fra_fwd.hip", "fra_bwd.hip")]
    usage = ["-Rpass-analysis=kernel-resource-usage"]
    for d in dims:
        out.append((os.path.join(CSRC, "fra_inst_fwd.hip"), os.path.join(tmpd, f"fra_inst_fwd_d{d}.o"),
                    common + [f"-DFRA_HEAD_DIM={d}"] + usage))
        out.append((os.path.join(CSRC, "fra_inst_bwd.hip"), os.path.join(tmpd, f"fra_inst_bwd_d{d}.o"),
                    common + [f"-DFRA_HEAD_DIM={d}"] + usage))
    return out


def build(verbose: bool = False) -> str:
    """Compile the library; returns its path.  Always recompiles."""
    jobs = max(1, min(16, os.cpu_count() or 1))
    with tempfile.TemporaryDirectory(prefix="fra_build_") as tmpd:
        todo = [(compile_command(s, o, dfs), o) for s, o, dfs in units(tmpd)]
        objs = [o for _, o in todo]
        if verbose:
            for c, _ in todo:
                print(" ".join(c), flush=True)
        errs, running, use = [], [], {}
        while todo or running:
            while todo and len(running) < jobs:
                c, _ = todo.pop(0)
                running.append((c, subprocess.Popen(c, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
            c, pr = running.pop(0)
            _, err = pr.communicate()
            use.update(scratch_use(err))
            err = "\n".join(l for l in err.splitlines() if "kernel-resource-usage" not in l and l.strip() != "|"
                            and not re.match(r"^\s*\d+ \|", l) and not re.match(r"^\s*\|\s*\^", l)
                            and not l.startswith("In file included from"))
            if pr.returncode != 0:
                errs.append(f"hipcc failed ({pr.returncode}) on {' '.join(c[-3:])}:\n{_clean(err)}")
            elif verbose and _clean(err).strip():
                print(_clean(err), file=sys.stderr)
        if errs:
            raise RuntimeError("\n".join(errs))
        bad = check_scratch(use)
        if bad:
            raise RuntimeError("kernels spill to scratch memory outside build.SCRATCH_ALLOWED:\n" + "\n".join(bad))
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
