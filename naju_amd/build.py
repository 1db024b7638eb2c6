"""Builds naju_amd/libnaju_scan.so from naju_amd/csrc/*.hip with hipcc for gfx950.

The library is built in-tree so that it travels with the repository snapshot.
Usage: python -m naju_amd.build
"""
import os
import subprocess
import sys

_PKG = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_PKG)
LIB_PATH = os.path.join(_PKG, "libnaju_scan.so")
SOURCES = [os.path.join(_PKG, "csrc", n)
           for n in ("naju_scan.hip", "naju_scan_mc.hip", "naju_mixer.hip", "naju_loss.hip", "naju_optim.hip")]

# Packed-FP32 VALU ops are disabled for all device code: only plain fp32
# arithmetic is emitted.
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(_ROOT, "include"),
]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    return "hipcc"


def _finish(cmd, proc, verbose):
    out, err = proc.communicate()
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    err = "\n".join(ln for ln in err.splitlines() if "packed-fp32-ops" not in ln)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose=False):
    """Compile every HIP source (in parallel, one object each) and link them
    into LIB_PATH. Always recompiles."""
    objs = [LIB_PATH + "." + os.path.basename(src) + ".o" for src in SOURCES]
    jobs = []
    for src, obj in zip(SOURCES, objs):
        cmd = [hipcc()] + HIPCC_FLAGS + ["-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        jobs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
    try:
        for cmd, proc in jobs:
            _finish(cmd, proc, verbose)
        tmp = LIB_PATH + ".tmp"
        cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC"] + objs + ["-o", tmp]
        if verbose:
            print(" ".join(cmd), flush=True)
        _finish(cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True), verbose)
        os.replace(tmp, LIB_PATH)
    finally:
        for cmd, proc in jobs:
            if proc.poll() is None:
                proc.kill()
                proc.wait()
        for obj in objs:
            if os.path.exists(obj):
                os.remove(obj)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
