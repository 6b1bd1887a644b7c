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


# Kernels whose MFMAs are inline assembly on AGPR accumulators (the four-wave
# 16x16x32 loop): the compiler's hazard checks do not see into that assembly,
# whose instruction order keeps the hazards away only as written, so a spill the
# compiler inserts between those instructions can change results. Their
# register use is checked at every build.
NO_SPILL_KERNELS = ("gemm_persist_w4m_kernel", "gemm_kernelILi256ELi256ELi2ELi2E", "gemm_pair_kernel")


def _spilled_kernels(remarks):
    """(kernel, VGPR spills) of every guarded kernel that spills, from hipcc's
    -Rpass-analysis=kernel-resource-usage remarks."""
    bad, name = [], None
    for line in remarks.splitlines():
        if "Function Name: " in line:
            name = line.split("Function Name: ", 1)[1].split()[0]
        elif "VGPRs Spill: " in line and name and any(k in name for k in NO_SPILL_KERNELS):
            n = int(line.split("VGPRs Spill: ", 1)[1].split()[0])
            if n:
                bad.append((name, n))
    return bad


def build(verbose: bool = False) -> str:
    """Compile every csrc/*.hip (one hipcc process per file, in parallel) and link them into one
    shared library; returns its path."""
    srcs = sources()
    inc = ["-I", os.path.join(ROOT, "include"), "-I", os.path.join(HERE, "csrc")]
    with tempfile.TemporaryDirectory(prefix="mg_build_") as objdir:
        objs = [os.path.join(objdir, os.path.basename(s) + ".o") for s in srcs]
        jobs = max(1, min(len(srcs), os.cpu_count() or 1, 16))
        with ThreadPoolExecutor(jobs) as pool:
            def compile_one(so):
                extra = ["-Rpass-analysis=kernel-resource-usage"] if os.path.basename(so[0]) == "gemm.hip" else []
                return _run([hipcc(), *HIPCC_FLAGS, *extra, *inc, "-c", so[0], "-o", so[1]], verbose and not extra)

            results = list(pool.map(compile_one, zip(srcs, objs)))
        for src, (rc, out) in zip(srcs, results):
            if rc != 0:
                raise RuntimeError(f"hipcc failed on {os.path.basename(src)} ({rc}):\n{out}")
            if os.path.basename(src) == "gemm.hip":
                bad = _spilled_kernels(out)
                if bad:
                    raise RuntimeError("kernels with inline-assembly MFMAs spill registers (their results would not "
                                       "be trustworthy): " + ", ".join(f"{k} ({n})" for k, n in bad))
            elif verbose and out.strip():
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
