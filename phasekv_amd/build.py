"""Build the HIP library ``phasekv_amd/libphasekv_hip.so`` for gfx950 with hipcc.

    python -m phasekv_amd.build [--incremental]

Every ``csrc/*.hip`` translation unit is compiled to an object in parallel (the
MFMA decode kernel is split into one unit per variant for that), then linked.
The library is built in-tree so it travels with the source tree.
``--incremental`` reuses objects whose sources and headers are older than them.
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
OBJ_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libphasekv_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = "gfx950"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def compile_flags():
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        # packed fp32 VALU forms are kept out of the generated code
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-ffp-contract=fast-honor-pragmas",
        "-Wno-unused-result",
        "-I", os.path.join(REPO_DIR, "include"), "-I", CSRC,
    ]


def compile_command(src: str, obj: str):
    return [hipcc(), *compile_flags(), "-c", src, "-o", obj]


def link_command(objs, out_path: str):
    return [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", out_path]


def _stale(src: str, obj: str, headers) -> bool:
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(f) > t for f in [src, *headers])


def build(verbose: bool = True, incremental: bool = False, jobs: int = 0) -> str:
    """Compile every HIP source into the shared library; returns its path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    headers = glob.glob(os.path.join(CSRC, "*.h")) + glob.glob(os.path.join(REPO_DIR, "include", "*.h"))
    srcs = sources()
    objs = [os.path.join(OBJ_DIR, os.path.basename(s)[:-4] + ".o") for s in srcs]
    todo = [(s, o) for s, o in zip(srcs, objs) if not incremental or _stale(s, o, headers)]
    jobs = jobs or min(8, os.cpu_count() or 1)

    def run(pair):
        s, o = pair
        tmp = o + ".tmp"
        cmd = compile_command(s, tmp)
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode == 0:
            os.replace(tmp, o)
        return s, res

    failed = []
    # the largest units first, so the longest compiles start at once
    todo.sort(key=lambda p: -os.path.getsize(p[0]) - (10 ** 7 if "mfma_" in p[0] else 0))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        for s, res in pool.map(run, todo):
            if res.returncode != 0:
                failed.append(s)
                sys.stderr.write(res.stdout + res.stderr)
    if failed:
        raise RuntimeError(f"hipcc failed on {', '.join(os.path.basename(f) for f in failed)}")
    tmp = LIB_PATH + ".tmp"
    cmd = link_command(objs, tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc link failed with exit code {res.returncode}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    build(incremental="--incremental" in sys.argv[1:])
