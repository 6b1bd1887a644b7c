"""Build libmingru_hip.so (all HIP kernels + the C ABI) for gfx950 with hipcc.

The library is written next to this file so that it travels with the source
tree; it links the HIP runtime by SONAME only, so inside a process that has
imported torch it binds to the runtime torch already loaded.
"""
import glob
import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_NAME = "libmingru_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed-fp32 VALU ops are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def sources():
    return sorted(glob.glob(os.path.join(HERE, "csrc", "*.hip")))


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    return proc.returncode, out


def build(verbose: bool = False) -> str:
    """Compile every csrc/*.hip (one hipcc process per file, in parallel) and link them into one
    shared library; returns its path."""
    srcs = sources()
    inc = ["-I", os.path.join(ROOT, "include"), "-I", os.path.join(HERE, "csrc")]
    with tempfile.TemporaryDirectory(prefix="mg_build_") as objdir:
        objs = [os.path.join(objdir, os.path.basename(s) + ".o") for s in srcs]
        jobs = max(1, min(len(srcs), os.cpu_count() or 1, 16))
        with ThreadPoolExecutor(jobs) as pool:
            results = list(pool.map(lambda so: _run([hipcc(), *HIPCC_FLAGS, *inc, "-c", so[0], "-o", so[1]], verbose),
                                    zip(srcs, objs)))
        for src, (rc, out) in zip(srcs, results):
            if rc != 0:
                raise RuntimeError(f"hipcc failed on {os.path.basename(src)} ({rc}):\n{out}")
            if verbose and out.strip():
                print(out, flush=True)
        fd, tmp = tempfile.mkstemp(prefix=LIB_NAME + ".tmp", dir=HERE)
        os.close(fd)
        rc, out = _run([hipcc(), "--offload-arch=gfx950", "-fPIC", "-shared", *objs, "-o", tmp], verbose)
        if rc != 0:
            os.unlink(tmp)
            raise RuntimeError(f"hipcc link failed ({rc}):\n{out}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
