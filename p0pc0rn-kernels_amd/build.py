"""Build recipe of the MI355X `gemm` path: libp0k.so (HIP, gfx950) and the Node N-API addon over it.

    python p0pc0rn-kernels_amd/build.py            # both
    python p0pc0rn-kernels_amd/build.py lib        # libp0k.so only

Everything is built in-tree (the built files travel with the repository snapshot to the GPU box) by calling hipcc / gcc
directly: the sources are few and compile in parallel in well under a minute.
"""
import os
import subprocess
import sys
import concurrent.futures as cf

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libp0k.so")
ADDON = os.path.join(PKG, "node", "p0k.node")
PROBE_SRC = os.path.join(PKG, "probe", "p0k_probe.hip")
PROBE_LIB = os.path.join(PKG, "probe", "libp0k_probe.so")   # the benchmark's measurement kernels (bench.py only)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["p0k_gemm_mfma.hip", "p0k_gemm_dma.hip", "p0k_gemv.hip", "p0k_rowstats.hip", "p0k_stats.hip", "p0k_attention.hip", "p0k_runtime.cpp", "p0k_check.cpp", "p0k_pack.cpp"]
HIP_FLAGS = [
    "-x", "hip", "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    # packed fp32 instructions stay off: ordinary float code only (v_pk_*_f32 are never emitted)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(ROOT, "include"),
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l and "is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError("build failed: " + " ".join(cmd) + "\n" + out)
    return out


def build_lib(verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    objs, cmds = [], []
    for s in SOURCES:
        o = os.path.join(OBJ, os.path.splitext(s)[0] + ".o")
        objs.append(o)
        cmds.append([HIPCC] + HIP_FLAGS + ["-c", os.path.join(CSRC, s), "-o", o])
    with cf.ThreadPoolExecutor(max_workers=min(8, len(cmds))) as ex:
        for out in ex.map(_run, cmds):
            if verbose and out.strip():
                print(out)
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", LIB] + objs)
    build_probe()
    return LIB


def build_probe():
    """libp0k_probe.so: the benchmark's HBM / matrix-core / LDS ceiling kernels and its launch gate, linked against
    libp0k.so (the probes enqueue on a context's stream); not part of the product library."""
    o = os.path.join(OBJ, "p0k_probe.o")
    _run([HIPCC] + HIP_FLAGS + ["-c", PROBE_SRC, "-o", o])
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", PROBE_LIB, o, "-L" + PKG, "-lp0k",
          "-Wl,-rpath,$ORIGIN/.."])
    return PROBE_LIB


def build_addon():
    """The N-API addon: plain C over node_api.h, linked against libp0k.so (found next to it through $ORIGIN/..)."""
    inc = "/usr/include/node"
    if not os.path.exists(os.path.join(inc, "node_api.h")):
        raise RuntimeError("node_api.h not found: the Node addon cannot be built")
    src = os.path.join(PKG, "node", "p0k_addon.c")
    _run(["gcc", "-O2", "-fPIC", "-shared", "-std=c11", "-Wall", "-I" + inc, "-I" + os.path.join(ROOT, "include"),
          src, "-o", ADDON, "-L" + PKG, "-lp0k", "-Wl,-rpath,$ORIGIN/..", "-Wl,--allow-shlib-undefined"])
    return ADDON


def build_all(verbose=False):
    build_lib(verbose)
    build_addon()


if __name__ == "__main__":
    what = sys.argv[1] if len(sys.argv) > 1 else "all"
    if what == "lib":
        print(build_lib(True))
    elif what == "addon":
        print(build_addon())
    else:
        build_all(True)
        print(LIB, ADDON)
