"""Builds libmxq.so (gfx950) in-tree from wuxianhuabu_amd/csrc.

    python -m wuxianhuabu_amd.build          # or: python wuxianhuabu_amd/build.py

Every HIP source is compiled with hipcc for gfx950 only, with packed fp32 ops
disabled (-packed-fp32-ops), then linked into wuxianhuabu_amd/libmxq.so. The
library travels with the source tree; nothing is installed.
"""
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libmxq.so")

SOURCES = ["mxq_layout.hip", "mxq_qmv.hip", *[f"mxq_qmv_b{b}.hip" for b in (2, 3, 4, 5, 6, 8)],
           "mxq_qmm.hip", "mxq_qmm_tiled.hip",
           *[f"mxq_qmm_tiled_b{b}.hip" for b in (2, 3, 4, 5, 6, 8)], "mxq_blockops.hip",
           "mxq_api.cpp", "mxq_safetensors.cpp"]
HEADERS = ["mxq_device.hpp", "mxq_internal.hpp", "mxq_ring.hpp", "mxq_tiled.hpp",
           "mxq_qmm_tiled_impl.hpp", "mxq_qmv_impl.hpp"]

ARCH = "gfx950"
COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas",
    "-I", os.path.join(ROOT, "include"),
]


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: libmxq cannot be built")
    return path


def build(verbose=False, extra_flags=()):
    """Compile all sources in parallel and link libmxq.so. Always rebuilds."""
    cc = hipcc()
    outdir = tempfile.mkdtemp(prefix="mxq_build_")
    try:
        procs = []
        objs = []
        for src in SOURCES:
            obj = os.path.join(outdir, src + ".o")
            cmd = [cc, *COMMON, *extra_flags]
            if src.endswith(".cpp"):
                cmd += ["-x", "hip"]
            cmd += ["-c", os.path.join(CSRC, src), "-o", obj]
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                                stderr=subprocess.STDOUT, text=True)))
            objs.append(obj)
        failed = []
        for src, p in procs:
            out, _ = p.communicate()
            # hipcc's host pass does not know the device-only feature name
            lines = [l for l in out.splitlines()
                     if "packed-fp32-ops' is not a recognized feature" not in l]
            if lines and (verbose or p.returncode != 0):
                print("\n".join(lines), file=sys.stderr)
            if p.returncode != 0:
                failed.append(src)
        if failed:
            raise RuntimeError("hipcc failed for: " + ", ".join(failed))
        tmp = LIB + ".tmp"
        cmd = [cc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        os.replace(tmp, LIB)
    finally:
        shutil.rmtree(outdir, ignore_errors=True)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
