"""Build libohip.so (the C-ABI HIP library) in-tree for gfx950.

    python -m oxionnx_amd.build

Every HIP source is compiled with hipcc for gfx950 only, with packed-fp32
instruction selection turned off and no floating-point contraction (the
epilogues reproduce the reference's unfused a*b + c).  Objects are compiled in
parallel into oxionnx_amd/_build/ and linked into oxionnx_amd/libohip.so.
"""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libohip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = [f"contract_{dt}_{part}.hip" for dt in ("i8", "f16", "f32", "bf16") for part in ("dense", "conv")] + [ "aux_kernels.hip", "nodes.hip", "ops.cpp", "dispatch.cpp"]

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
    f"-I{os.path.join(ROOT, 'include')}",
]


def _compile(src, incremental=False):
    obj = os.path.join(OUT_DIR, os.path.splitext(src)[0] + ".o")
    if incremental and os.path.exists(obj):
        kern = ["mfma_core.hpp", "launch.hpp", "internal.hpp", "halo_conv.hpp", "norm_stats.hpp"]
        local = {"ops.cpp": ["internal.hpp"], "dispatch.cpp": ["internal.hpp"],
                 "aux_kernels.hip": kern, "nodes.hip": ["internal.hpp", "norm_stats.hpp"]}.get(src, kern + ["contract.inc"])
        deps = [os.path.join(CSRC, f) for f in [src] + local]
        if src.endswith(".cpp"):
            deps.append(os.path.join(ROOT, "include", "ohip.h"))
        if all(os.path.getmtime(d) <= os.path.getmtime(obj) for d in deps):
            return obj
    lang = [] if src.endswith(".hip") else ["-x", "hip"]
    cmd = [HIPCC] + FLAGS + lang + ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose=True, incremental=False):
    """Compile every source (incremental=True skips objects newer than every
    source and header -- a development shortcut; the driver's build() always
    compiles everything)."""
    os.makedirs(OUT_DIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(lambda s: _compile(s, incremental), SOURCES))
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", LIB] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(incremental="--incremental" in sys.argv)
    sys.exit(0)
