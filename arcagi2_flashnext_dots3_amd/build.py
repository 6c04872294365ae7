"""Build the gfx950 C-ABI library (libspmla_gfx950.so) in-tree with hipcc.

Every .hip file under csrc/ is compiled to an object (in parallel) and linked into one shared library next to
this file; the Python loader (_lib.py) and the tests load that file. Objects go to _build/ (git-ignored).
All HIP code is compiled with packed fp32 instructions disabled (-packed-fp32-ops), see the feature flag below.
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
REPO = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libspmla_gfx950.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-Wno-unused-command-line-argument", "-I", CSRC, "-I", os.path.join(REPO, "include")]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    return err


def build(verbose=False):
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    bdir = os.path.join(REPO, "_build")
    os.makedirs(bdir, exist_ok=True)
    objs = [os.path.join(bdir, f[:-4] + ".o") for f in srcs]
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(_run, [HIPCC, *FLAGS, "-c", os.path.join(CSRC, s), "-o", o]) for s, o in zip(srcs, objs)]
        for s, f in zip(srcs, futs):
            msg = f.result()
            if verbose and msg:
                print(f"[build] {s}: {msg}", flush=True)
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
