"""Build libflagsparse_hip.so (gfx950) in-tree with hipcc.

Usage: python -m flagsparse_amd.csrc.build   (or call build()).

Each translation unit is compiled to an object file under
flagsparse_amd/csrc/_build/ in parallel, then linked into
flagsparse_amd/libflagsparse_hip.so.  The library links against the HIP
runtime by soname (libamdhip64.so.7); when torch is imported first its
bundled runtime satisfies that soname, so torch streams and our launches
share one runtime.
"""

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
REPO = os.path.dirname(PKG)
OUT = os.path.join(PKG, "libflagsparse_hip.so")
BUILD_DIR = os.path.join(HERE, "_build")

SOURCES = ["abi.cpp", "spmv.hip", "spmv_opt.hip", "spmm.hip", "spmm_group.hip", "transpose.hip", "sell.hip"]
# the measurement-only library (bench.py --gather-floor), with its own copy of
# the error reporting
DIAG_OUT = os.path.join(PKG, "libflagsparse_diag.so")
DIAG_SOURCES = ["abi.cpp", "diag.hip"]
ARCH = "gfx950"

COMMON_FLAGS = [
    "-O3",
    "-fPIC",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-I" + os.path.join(REPO, "include"),
    # Keep the compiler from forming packed-fp32 VALU ops (v_pk_*_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
]


def _hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build flagsparse_amd")


def _compile(src, extra):
    obj = os.path.join(BUILD_DIR, src + ".o")
    lang = ["-x", "hip"]
    cmd = [_hipcc(), *lang, *COMMON_FLAGS, *extra, "-c", os.path.join(HERE, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj, res.stderr


def _link(objs, out):
    tmp = out + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)


def build(verbose=False, extra_flags=None):
    """Compile every HIP source for gfx950 and link the shared libraries
    (the operator library and the measurement-only diagnostic library)."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    extra = list(extra_flags or [])
    srcs = list(dict.fromkeys(SOURCES + DIAG_SOURCES))
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        results = dict(zip(srcs, ex.map(lambda s: _compile(s, extra), srcs)))
    if verbose:
        for _, err in results.values():
            if err.strip():
                print(err, file=sys.stderr)
    _link([results[s][0] for s in SOURCES], OUT)
    _link([results[s][0] for s in DIAG_SOURCES], DIAG_OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
