"""The CPU tests of the safetensors reader (corpus included), the C-ABI
argument validation and the C oracle, rerun in a subprocess against builds
instrumented with AddressSanitizer and UndefinedBehaviorSanitizer: the
library's host code (swift-ltx_amd/build_sanitized.py; -Xarch_host, the
device code is unchanged) and the oracle's C (q4_oracle.build_c_sanitized),
with clang's ASan runtime preloaded into the Python process.  A positive
control first shows that the same setup reports a heap overread.
"""
import importlib.util
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SUITES = ["tests/test_safetensors.py", "tests/test_st_corpus.py", "tests/test_capi.py",
          "tests/test_oracle.py"]
REPORTS = ("ERROR: AddressSanitizer", "runtime error:", "ERROR: LeakSanitizer")


def _build_script():
    spec = importlib.util.spec_from_file_location(
        "sltx_build_sanitized", os.path.join(REPO, "swift-ltx_amd", "build_sanitized.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="module")
def san():
    b = _build_script()
    try:
        rt = b.asan_runtime()
    except (OSError, subprocess.CalledProcessError) as e:
        pytest.skip(f"no clang ASan runtime: {e}")
    if not os.path.isfile(rt):
        pytest.skip(f"no clang ASan runtime at {rt}")
    lib = b.build()   # rebuilt only when a source changed
    from oracle import q4_oracle
    odir = os.path.join(REPO, "oracle", "_build_san")
    q4_oracle.build_c_sanitized(odir)
    env = dict(os.environ, LD_PRELOAD=rt, SLTX_LIB_PATH=lib, SLTX_ORACLE_LIB_DIR=odir,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    return env


def test_sanitizer_reports_a_heap_overread(san, tmp_path):
    src = tmp_path / "overread.c"
    src.write_text("#include <stdlib.h>\n"
                   "int overread(int n) { int* a = malloc(n * sizeof(int)); int v;\n"
                   "  for (int i = 0; i < n; ++i) a[i] = i;\n"
                   "  v = a[n]; free(a); return v; }\n")
    so = tmp_path / "liboverread.so"
    clang = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin", "clang")
    subprocess.run([clang, "-O0", "-g", "-fPIC", "-shared", "-fsanitize=address,undefined",
                    "-shared-libsan", "-o", str(so), str(src)], check=True)
    r = subprocess.run([sys.executable, "-c",
                        f"import ctypes; ctypes.CDLL({str(so)!r}).overread(4)"],
                       env=san, capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "heap-buffer-overflow" in r.stderr, r.stderr[-2000:]


def test_cpu_suites_clean_under_sanitizers(san):
    r = subprocess.run([sys.executable, "-m", "pytest", *SUITES, "-m", "not gpu", "-q",
                        "-p", "no:cacheprovider"], cwd=REPO, env=san, capture_output=True,
                       text=True, timeout=900)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    for rep in REPORTS:
        assert rep not in out, out[-4000:]
    assert " passed" in out
