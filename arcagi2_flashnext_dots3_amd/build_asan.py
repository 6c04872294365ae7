"""Host-side AddressSanitizer build of the C-ABI library, for CPU checks of its host code.

Every .hip file is compiled as in build.py, with AddressSanitizer on the host compilation only (each sanitizer
flag behind -Xarch_host: the device code is the ordinary gfx950 code), and linked into
_build/asan/libspmla_gfx950_asan.so. The library expects the ASan runtime to be loaded first, so a process that uses
it starts with LD_PRELOAD=<asan_runtime()> and SPMLA_LIB pointing at the library (tests/test_abi_asan.py runs the
C-ABI argument checks that way). Not used by the product path.
"""
import concurrent.futures
import glob
import os
import sys

from . import build as _b

ASAN_DIR = os.path.join(_b.REPO, "_build", "asan")
ASAN_LIB = os.path.join(ASAN_DIR, "libspmla_gfx950_asan.so")
HOST_ASAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]


def asan_runtime():
    """The clang ASan runtime that matches hipcc's host compiler, or None."""
    hits = sorted(glob.glob("/opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return hits[-1] if hits else None


def build_asan(verbose=False):
    srcs = sorted(f for f in os.listdir(_b.CSRC) if f.endswith(".hip"))
    os.makedirs(ASAN_DIR, exist_ok=True)
    objs = [os.path.join(ASAN_DIR, f[:-4] + ".o") for f in srcs]
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(_b._run, [_b.HIPCC, *_b.FLAGS, *HOST_ASAN, "-c", os.path.join(_b.CSRC, s), "-o", o])
                for s, o in zip(srcs, objs)]
        for s, f in zip(srcs, futs):
            msg = f.result()
            if verbose and msg:
                print(f"[build_asan] {s}: {msg}", flush=True)
    tmp = ASAN_LIB + ".tmp"
    _b._run([_b.HIPCC, "-shared", "-fPIC", f"--offload-arch={_b.ARCH}", "-Xarch_host", "-fsanitize=address",
             "-shared-libsan", "-o", tmp, *objs])
    os.replace(tmp, ASAN_LIB)
    return ASAN_LIB


if __name__ == "__main__":
    print(build_asan(verbose="-v" in sys.argv))
