"""Host-only build of libswiftltx_q4 with AddressSanitizer and
UndefinedBehaviorSanitizer, for the sanitized CPU test run
(tests/test_sanitized.py).

Every csrc/*.hip file is compiled as usual, with the sanitizers on its host
pass only (-Xarch_host): the safetensors reader, the C-ABI argument
validation, the workspace bookkeeping and the launch code are instrumented;
the device code is the regular build's (the CPU tests launch no kernel).
The library goes to _build_san/libswiftltx_q4_san.so, rebuilt when a source
is newer; a process that loads it must preload clang's ASan runtime
(asan_runtime()).

    python swift-ltx_amd/build_sanitized.py
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
OUT_DIR = os.path.join(PKG_DIR, "_build_san")
LIB_PATH = os.path.join(OUT_DIR, "libswiftltx_q4_san.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

# each sanitizer flag applies to the host pass only (-Xarch_host)
HOST_SAN = [
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=undefined",
    "-Xarch_host", "-fno-omit-frame-pointer",
]
FLAGS = ["--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         *HOST_SAN, "-I" + os.path.join(REPO, "include")]


def asan_runtime() -> str:
    """Path of clang's shared ASan runtime (which also carries UBSan's)."""
    clang = os.path.join(ROCM, "llvm", "bin", "clang")
    r = subprocess.run([clang, "-print-file-name=libclang_rt.asan-x86_64.so"],
                       capture_output=True, text=True, check=True)
    return r.stdout.strip()


def _compile(src: str) -> str:
    obj = os.path.join(OUT_DIR, os.path.basename(src) + ".o")
    r = subprocess.run([HIPCC, *FLAGS, "-c", src, "-o", obj], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def _sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def is_stale() -> bool:
    if not os.path.exists(LIB_PATH):
        return True
    deps = _sources() + [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hpp")]
    deps += [os.path.join(REPO, "include", f) for f in os.listdir(os.path.join(REPO, "include"))]
    t = os.path.getmtime(LIB_PATH)
    return any(os.path.getmtime(f) > t for f in deps + [__file__])


def build(jobs: int = 8, force: bool = False) -> str:
    if not force and not is_stale():
        return LIB_PATH
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = _sources()
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH + ".tmp%d" % os.getpid()
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC",
                        "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                        "-shared-libsan", "-o", tmp, *objs], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(force=True))
    sys.exit(0)
