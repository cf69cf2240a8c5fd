"""Build the gfx950 shared libraries in-tree with hipcc.

    python swift-ltx_amd/build.py            # rebuild every object
    python swift-ltx_amd/build.py --if-stale # only when a source is newer

csrc/*.hip -> lib/libswiftltx_q4.so, the drop-in library (include/swiftltx_q4.h).
csrc/bench/*.hip -> lib/libswiftltx_bench.so, measurement kernels that only
bench.py loads (the HBM read ceiling); not part of the C ABI.
Objects go to swift-ltx_amd/_build/, the libraries to swift-ltx_amd/lib/.
Every HIP file is compiled for gfx950 only, with packed-fp32 instruction
selection disabled (hipcc's host pass warns that it does not know the
feature; that warning is expected).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OBJ_DIR = os.path.join(PKG, "_build")
LIB_DIR = os.path.join(PKG, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libswiftltx_q4.so")
BENCH_LIB_PATH = os.path.join(LIB_DIR, "libswiftltx_bench.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

DEVICE_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(REPO, "include"),
]


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def bench_sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "bench", "*.hip")))


def headers() -> list[str]:
    return (sorted(glob.glob(os.path.join(CSRC, "*.hpp")))
            + sorted(glob.glob(os.path.join(REPO, "include", "*.h"))))


def is_stale() -> bool:
    if not os.path.exists(LIB_PATH) or not os.path.exists(BENCH_LIB_PATH):
        return True
    t = min(os.path.getmtime(LIB_PATH), os.path.getmtime(BENCH_LIB_PATH))
    return any(os.path.getmtime(f) > t
               for f in sources() + bench_sources() + headers() + [__file__])


def _compile(src: str) -> str:
    sub = "bench_" if os.path.basename(os.path.dirname(src)) == "bench" else ""
    obj = os.path.join(OBJ_DIR, sub + os.path.basename(src) + ".o")
    cmd = [HIPCC, *DEVICE_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def _link(objs: list[str], path: str) -> None:
    tmp = path + ".tmp%d" % os.getpid()
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, path)


def build(force: bool = True, jobs: int = 8) -> str:
    """Compile every csrc/*.hip (and csrc/bench/*.hip) for gfx950, link
    LIB_PATH and BENCH_LIB_PATH; returns LIB_PATH."""
    if not force and not is_stale():
        return LIB_PATH
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    main, bench = sources(), bench_sources()
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(_compile, main + bench))
    _link(objs[:len(main)], LIB_PATH)
    _link(objs[len(main):], BENCH_LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    stale_only = "--if-stale" in sys.argv
    print(build(force=not stale_only))
