"""C ABI surface, checked on the CPU (no GPU calls).

* the library loads and exports every function include/*.h declares;
* argument validation runs before any HIP call and returns the documented
  status codes (the reference instead crashes or reads out of bounds, e.g.
  K % 32 != 0 at Kernels.swift:490).
Only validation paths that return before touching the device are exercised.
"""
import ctypes
import glob
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

ALIGNED = 0x10000  # fake, never dereferenced: validation fails before any access


def header_functions():
    names = set()
    for h in glob.glob(os.path.join(REPO, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(sltx_\w+)\s*\(", text))
    return names


def test_header_matches_binding_list(pkg):
    assert header_functions() == set(pkg.EXPORTED)


def test_library_exports_every_header_symbol(pkg):
    L = pkg.lib()
    for name in header_functions():
        assert hasattr(L, name), name
    assert L.sltx_abi_version() == 1


def _mm(pkg, fn="sltx_matmul_q4", x=ALIGNED, w=ALIGNED, s=ALIGNED, b=ALIGNED, out=ALIGNED,
        M=1, K=3072, N=3072, g=64):
    return getattr(pkg.lib(), fn)(x, w, s, b, out, M, K, N, g, None)


@pytest.mark.parametrize("fn", ["sltx_matmul_q4", "sltx_matmul_q4_fast", "sltx_matmul_q4_fast_f32"])
@pytest.mark.parametrize("kw,code,frag", [
    (dict(K=100), -1, "multiple of 32"),
    (dict(K=0), -1, "positive"),
    (dict(M=-1), -1, "negative"),
    (dict(N=-5), -1, "negative"),
    (dict(g=12), -1, "multiple of 8"),
    (dict(K=96, g=64), -1, "not a multiple of group_size"),
    (dict(g=16, K=128), -2, "unsupported"),
    (dict(g=256, K=512), -2, "unsupported"),
    (dict(x=0), -1, "null"),
    (dict(w=0), -1, "null"),
    (dict(out=0), -1, "null"),
    (dict(x=ALIGNED + 2), -1, "x must be 16-byte aligned"),
    (dict(w=ALIGNED + 4), -1, "weight must be 16-byte aligned"),
    (dict(s=ALIGNED + 1), -1, "scales/biases"),
    (dict(out=ALIGNED + 1), -1, "misaligned out"),
])
def test_validation_errors(pkg, fn, kw, code, frag):
    rc = _mm(pkg, fn=fn, **kw)
    assert rc == code
    assert frag in pkg.last_error()
    assert fn in pkg.last_error()


def test_empty_shapes_are_noops(pkg):
    # M == 0 or N == 0: nothing to do, no device needed, null pointers allowed
    assert _mm(pkg, M=0, x=0, out=0) == 0
    assert _mm(pkg, N=0, w=0, s=0, b=0, out=0) == 0
    assert pkg.lib().sltx_silu_mul(0, 0, 0, 0, None) == 0


def test_silu_mul_validation(pkg):
    L = pkg.lib()
    assert L.sltx_silu_mul(ALIGNED, ALIGNED, ALIGNED, -1, None) == -1
    assert L.sltx_silu_mul(0, ALIGNED, ALIGNED, 8, None) == -1
    assert L.sltx_silu_mul(ALIGNED + 1, ALIGNED, ALIGNED, 8, None) == -1


def _w(pkg, K=3072, g=64, w=ALIGNED):
    return pkg.CQ4Weight(w, ALIGNED, ALIGNED, K, g)


def test_linear_validation(pkg):
    L = pkg.lib()
    assert L.sltx_linear(ALIGNED, None, ALIGNED, 1, 3072, 64, 0, None) == -1
    w = _w(pkg, K=2048)
    assert L.sltx_linear(ALIGNED, ctypes.byref(w), ALIGNED, 1, 3072, 64, 0, None) == -1
    assert "weight K" in pkg.last_error()
    w = _w(pkg, K=3072, g=48)  # valid for the reference (g % 8 == 0), not built here
    assert L.sltx_linear(ALIGNED, ctypes.byref(w), ALIGNED, 4, 3072, 64, 1, None) == -2


def test_silu_mul_fused_validation(pkg):
    L = pkg.lib()
    g, u = _w(pkg), _w(pkg, g=32)
    assert L.sltx_matmul_q4_silu_mul(ALIGNED, ctypes.byref(g), ctypes.byref(u), ALIGNED, 1, 3072,
                                     64, None) == -1
    assert "group_size differ" in pkg.last_error()
    u = _w(pkg, K=1024)
    assert L.sltx_matmul_q4_silu_mul(ALIGNED, ctypes.byref(g), ctypes.byref(u), ALIGNED, 1, 3072,
                                     64, None) == -1
    u = _w(pkg, w=ALIGNED + 8)
    assert L.sltx_matmul_q4_silu_mul(ALIGNED, ctypes.byref(g), ctypes.byref(u), ALIGNED, 2, 3072,
                                     64, None) == -1


@pytest.mark.parametrize("args,frag", [
    (dict(x_dtype=3), "x_dtype"),
    (dict(out_dtype=7), "out_dtype"),
    (dict(epilogue=1), "epilogue"),
    (dict(bias=ALIGNED + 2), "misaligned bias"),
    (dict(out=ALIGNED + 2, out_dtype=2), "misaligned out"),
])
def test_ex_validation(pkg, args, frag):
    a = dict(x=ALIGNED, x_dtype=0, bias=None, epilogue=0, out=ALIGNED, out_dtype=2, M=8, N=64)
    a.update(args)
    w = _w(pkg)
    rc = pkg.lib().sltx_matmul_q4_ex(a["x"], a["x_dtype"], ctypes.byref(w), a["bias"],
                                     a["epilogue"], a["out"], a["out_dtype"], a["M"], a["N"], None)
    assert rc == -1
    assert frag in pkg.last_error()


def test_python_wrapper_raises(pkg):
    torch = pytest.importorskip("torch")
    x = torch.zeros(1, 100, dtype=torch.float16)
    w = torch.zeros(8, 12, dtype=torch.int32)
    s = torch.zeros(8, 1, dtype=torch.float16)
    with pytest.raises(pkg.SltxError) as ei:
        pkg.matmul_q4(x, w, s, s, 1, 100, 8, 64, out=torch.zeros(1, 8, dtype=torch.float16),
                      stream=0)
    assert ei.value.code == pkg.SLTX_ERR_INVALID


def test_last_error_is_thread_local(pkg):
    import threading
    assert _mm(pkg, K=100) == -1
    seen = {}

    def other():
        seen["msg"] = pkg.last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == ""
    assert "multiple of 32" in pkg.last_error()


# ---- decode-layer fusion entry points: validation paths only ----

def _wq(pkg, K=3072, g=64, weight=ALIGNED):
    return pkg.CQ4Weight(weight, ALIGNED, ALIGNED, K, g)


def test_rms_norm_validation(pkg):
    L = pkg.lib()
    assert L.sltx_rms_norm(ALIGNED, ALIGNED, 1e-5, ALIGNED, 0, 3072, None) == 0
    assert L.sltx_rms_norm(ALIGNED, ALIGNED, 1e-5, ALIGNED, -1, 3072, None) == -1
    assert L.sltx_rms_norm(0, ALIGNED, 1e-5, ALIGNED, 1, 3072, None) == -1
    assert "null" in pkg.last_error()
    assert L.sltx_rms_norm(ALIGNED, ALIGNED + 2, 1e-5, ALIGNED, 1, 3072, None) == -1
    assert "misaligned" in pkg.last_error()
    # residual_out and norm_out overlapping
    assert L.sltx_residual_rms_norm(ALIGNED, ALIGNED, ALIGNED, 1e-5, ALIGNED, ALIGNED + 64, 1,
                                    3072, None) == -1
    assert "overlap" in pkg.last_error()
    A, B, R, NO = ALIGNED, 2 * ALIGNED, 3 * ALIGNED, 4 * ALIGNED
    # an output that overlaps an input without being equal to it races
    assert L.sltx_residual_rms_norm(A, B, ALIGNED, 1e-5, A + 16, NO, 2, 3072, None) == -1
    assert "residual_out overlaps an input" in pkg.last_error()
    assert L.sltx_residual_rms_norm(A, B, ALIGNED, 1e-5, R, B + 6144, 2, 3072, None) == -1
    assert "norm_out overlaps an input" in pkg.last_error()
    assert L.sltx_rms_norm(A, ALIGNED, 1e-5, A + 6144, 2, 3072, None) == -1
    assert "overlap" in pkg.last_error()


def test_rmsnorm_matmul_validation(pkg):
    L = pkg.lib()
    w = _wq(pkg)
    assert L.sltx_rmsnorm_matmul_q4(ALIGNED, 0, 1e-5, ctypes.byref(w), ALIGNED, 5120, None) == -1
    assert "norm_weight" in pkg.last_error()
    assert L.sltx_rmsnorm_matmul_q4(ALIGNED, ALIGNED + 4, 1e-5, ctypes.byref(w), ALIGNED, 5120,
                                    None) == -1
    assert "16-byte" in pkg.last_error()
    bad = _wq(pkg, K=100)
    assert L.sltx_rmsnorm_matmul_q4(ALIGNED, ALIGNED, 1e-5, ctypes.byref(bad), ALIGNED, 5120,
                                    None) == -1
    assert "multiple of 32" in pkg.last_error()
    assert L.sltx_rmsnorm_matmul_q4(ALIGNED, ALIGNED, 1e-5, ctypes.byref(w), ALIGNED, 0, None) == 0


def test_residual_rmsnorm_silu_validation(pkg):
    L = pkg.lib()
    g, u = _wq(pkg), _wq(pkg)
    fn = L.sltx_residual_rmsnorm_matmul_q4_silu_mul
    # residual_out overlapping a
    assert fn(ALIGNED, 0x20000, ALIGNED, 1e-5, ALIGNED + 16, ctypes.byref(g), ctypes.byref(u),
              0x30000, 8192, None) == -1
    assert "overlaps" in pkg.last_error()
    u2 = _wq(pkg, K=2048)
    assert fn(ALIGNED, 0x20000, ALIGNED, 1e-5, 0x40000, ctypes.byref(g), ctypes.byref(u2),
              0x30000, 8192, None) == -1
    assert "K differ" in pkg.last_error()
    assert fn(ALIGNED, 0x20000, ALIGNED, 1e-5, 0x40000 + 8, ctypes.byref(g), ctypes.byref(u),
              0x30000, 8192, None) == -1
    assert "16-byte" in pkg.last_error()


def test_matmul_residual_validation(pkg):
    L = pkg.lib()
    w = _wq(pkg, K=8192)
    fn = L.sltx_matmul_q4_residual
    assert fn(ALIGNED, ctypes.byref(w), 0, 0x40000, 1, 3072, None) == -1
    assert "null residual" in pkg.last_error()
    # out overlapping residual without being equal
    assert fn(ALIGNED, ctypes.byref(w), 0x40000, 0x40000 + 2, 1, 3072, None) == -1
    assert "overlap" in pkg.last_error()
    # out overlapping x
    assert fn(ALIGNED, ctypes.byref(w), 0x40000, ALIGNED + 32, 1, 3072, None) == -1
    assert "overlaps x" in pkg.last_error()
    assert fn(ALIGNED, ctypes.byref(w), 0x40000, 0x40000, 0, 3072, None) == 0


def test_argmax_and_sample_validation(pkg):
    L = pkg.lib()
    A, O = ALIGNED, 0x40000
    assert L.sltx_argmax(A, 0, 0, O, None) == -1 and "positive" in pkg.last_error()
    assert L.sltx_argmax(A, 1, 10, O, None) == -1 and "SLTX_F16" in pkg.last_error()   # bf16
    assert L.sltx_argmax(None, 0, 10, O, None) == -1 and "null" in pkg.last_error()
    assert L.sltx_argmax(A + 2, 2, 10, O, None) == -1 and "misaligned" in pkg.last_error()
    fn = L.sltx_sample_top_p

    def call(n=100, dt=0, t=0.7, p=0.9, r=1.1, seen=None, ns=0, u=0.5, logits=A, out=O):
        return fn(logits, dt, n, t, p, r, seen, ns, u, out, None)
    assert call(n=0) == -1 and "positive" in pkg.last_error()
    assert call(n=(1 << 24) + 1) == -1 and "2^24" in pkg.last_error()
    assert call(dt=1) == -1 and "SLTX_F16" in pkg.last_error()
    for bad in (dict(t=0.0), dict(t=-1.0), dict(p=0.0), dict(r=0.0), dict(t=float("nan"))):
        assert call(**bad) == -1 and "must be positive" in pkg.last_error(), bad
    for u in (-0.1, 1.0, float("nan")):
        assert call(u=u) == -1 and "[0, 1)" in pkg.last_error()
    assert call(ns=-1) == -1 and "n_seen" in pkg.last_error()
    assert call(ns=3, seen=None) == -1 and "null" in pkg.last_error()
    assert call(out=None) == -1 and "null" in pkg.last_error()
    assert call(out=O + 2) == -1 and "misaligned" in pkg.last_error()
    assert call(seen=A + 1, ns=2) == -1 and "misaligned" in pkg.last_error()


def test_sample_noalloc_validation(pkg):
    """sltx_sample_top_p_noalloc rejects what sltx_sample_top_p rejects, and
    vocabularies past its fixed scratch (262144 logits), before any HIP call."""
    L = pkg.lib()
    A, O = ALIGNED, 0x40000
    fn = L.sltx_sample_top_p_noalloc

    def call(n=100, dt=0, t=0.7, p=0.9, r=1.1, seen=None, ns=0, u=0.5, logits=A, out=O):
        return fn(logits, dt, n, t, p, r, seen, ns, u, out, None)
    assert call(n=262145) == -1 and "262144" in pkg.last_error()
    assert call(n=(1 << 24)) == -1 and "262144" in pkg.last_error()
    assert call(n=0) == -1 and "positive" in pkg.last_error()
    assert call(dt=1) == -1 and "SLTX_F16" in pkg.last_error()
    assert call(t=0.0) == -1 and "must be positive" in pkg.last_error()
    assert call(u=1.0) == -1 and "[0, 1)" in pkg.last_error()
    assert call(ns=3, seen=None) == -1 and "null" in pkg.last_error()
    assert call(out=O + 2) == -1 and "misaligned" in pkg.last_error()


def test_sample_state_validation(pkg):
    """sltx_sample_top_p_state rejects what sltx_sample_top_p rejects, plus a
    missing or malformed state, before any device work."""
    L = pkg.lib()
    A, O = ALIGNED, 0x40000
    fn = L.sltx_sample_top_p_state

    def state(**kw):
        f = dict(history=A, history_len=A + 0x100, history_capacity=16, draws=A + 0x200,
                 next_draw=A + 0x300, draw_count=8)
        f.update(kw)
        return pkg.CSampleState(**f)

    def call(st, n=100, dt=0, t=0.7, p=0.9, r=1.1, logits=A, out=O):
        return fn(logits, dt, n, t, p, r, ctypes.byref(st) if st is not None else None, out, None)
    good = state()
    assert call(good, n=0) == -1 and "positive" in pkg.last_error()
    assert call(good, dt=1) == -1 and "SLTX_F16" in pkg.last_error()
    assert call(good, t=0.0) == -1 and "must be positive" in pkg.last_error()
    assert call(good, out=None) == -1 and "null" in pkg.last_error()
    assert call(None) == -1 and "null state" in pkg.last_error()
    assert call(state(history_capacity=-1)) == -1 and "history_capacity" in pkg.last_error()
    assert call(state(draw_count=0)) == -1 and "draw_count" in pkg.last_error()
    for k in ("history_len", "draws", "next_draw"):
        assert call(state(**{k: None})) == -1 and "null pointer in state" in pkg.last_error(), k
    assert call(state(history=None)) == -1 and "null pointer in state" in pkg.last_error()
    # an empty history needs no buffer
    for k in ("history", "history_len", "draws", "next_draw"):
        off = {"history": A + 2, "history_len": A + 0x102, "draws": A + 0x201,
               "next_draw": A + 0x303}[k]
        assert call(state(**{k: off})) == -1 and "misaligned" in pkg.last_error(), k
    assert "sltx_sample_top_p_state" in pkg.EXPORTED


def test_matmul_out_must_not_overlap_x(pkg):
    """Every GEMV block re-reads x while others store, so an output that
    overlaps the activation input is rejected before any device work."""
    L = pkg.lib()
    A = ALIGNED
    assert _mm(pkg, x=A, out=A + 64) == -1 and "out overlaps x" in pkg.last_error()
    assert _mm(pkg, fn="sltx_matmul_q4_fast_f32", M=4, x=A, out=A - 16) == -1
    assert "out overlaps x" in pkg.last_error()
    w = _w(pkg)
    assert L.sltx_matmul_q4_ex(A, 1, ctypes.byref(w), None, 0, A + 32, 2, 8, 64, None) == -1
    assert "out overlaps x" in pkg.last_error()
    g, u = _w(pkg), _w(pkg)
    assert L.sltx_matmul_q4_silu_mul(A, ctypes.byref(g), ctypes.byref(u), A, 2, 3072, 64,
                                     None) == -1
    assert "out overlaps x" in pkg.last_error()
    assert L.sltx_matmul_q4_geglu(A, ctypes.byref(g), ctypes.byref(u), A + 2, 1, 3072, 64,
                                  None) == -1
    assert "out overlaps x" in pkg.last_error()
    assert L.sltx_rmsnorm_matmul_q4(A, 0x30000, 1e-5, ctypes.byref(w), A + 16, 64, None) == -1
    assert "out overlaps x" in pkg.last_error()
    fn = L.sltx_residual_rmsnorm_matmul_q4_silu_mul
    assert fn(A, 0x20000, 0x30000, 1e-5, 0x40000, ctypes.byref(g), ctypes.byref(u), 0x20000,
              64, None) == -1
    assert "out overlaps" in pkg.last_error()


def test_matmul_residual_rms_norm_validation(pkg):
    """sltx_matmul_q4_residual_rms_norm rejects unsupported widths, misaligned
    rows and overlapping outputs before any device work."""
    L = pkg.lib()
    fn = L.sltx_matmul_q4_residual_rms_norm
    A, R, O, N_, X = 0x100000, 0x200000, 0x300000, 0x400000, 0x500000
    w = _w(pkg)

    def call(x=X, wp=ctypes.byref(w), res=R, nw=N_, M=4, N=3072, ro=O, no=0x600000):
        return fn(x, wp, res, nw, 1e-5, M, N, 0, ro, no, None)

    assert call(M=0) == 0 and call(N=0) == 0           # no-ops
    assert call(wp=None) == -1 and "null weight" in pkg.last_error()
    assert call(res=0) == -1 and "null" in pkg.last_error()
    assert call(N=3076) == -2 and "multiple of 8" in pkg.last_error()
    assert call(N=16392) == -2
    assert call(res=R + 2) == -1 and "16-byte aligned" in pkg.last_error()
    assert call(nw=N_ + 4) == -1 and "16-byte aligned" in pkg.last_error()
    assert call(ro=R + 16) == -1 and "overlap without being equal" in pkg.last_error()
    assert call(no=O + 16) == -1 and "norm_out overlaps" in pkg.last_error()
    assert call(no=R) == -1 and "norm_out overlaps" in pkg.last_error()
    assert call(ro=X + 64) == -1 and "overlaps x" in pkg.last_error()
    assert call(no=X) == -1 and "overlaps x" in pkg.last_error()
    wg = _w(pkg, g=48)
    assert call(wp=ctypes.byref(wg)) == -2
