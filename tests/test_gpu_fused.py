"""GPU parity of the decode-layer fusion entry points through the C ABI.

Reference operators: rmsNorm (Ops.swift:8-27; rms_norm, Kernels.swift:40-86),
residualRmsNorm (Ops.swift:256-279; residual_rms_norm, Kernels.swift:238-290),
elemAdd (Ops.swift:72-84; add, Kernels.swift:121-128) and their use around the
projections in the Llama decode layer (LlamaModel.swift:288-331).

Tolerances:
  * the fp16 residual stream (half(a + b)) is bit-exact;
  * normalized vectors agree with the oracle to 1 fp16 ulp (the GPU's fp32 sum
    of squares and rsqrt differ from the oracle's fp64 ones below fp32 rounding,
    which can move a value across an fp16 rounding boundary);
  * fused matmuls meet the GEMV / GEMM bounds of tests/helpers.py against the
    fp64 oracle applied to the oracle's normalized vector;
  * the residual epilogue is within 1 fp16 ulp of the projection plus 1 ulp of
    the result plus the matmul bound (the projection is rounded to fp16 before
    the add, as in the reference).
"""
import numpy as np
import pytest

from helpers import (GATE, TOL_GEMM_F16, TOL_GEMV, assert_parity, gpu_inputs, host, q4w,
                     to_dev)
from oracle import q4_oracle as o

pytestmark = pytest.mark.gpu

EPS = 1e-5


def _norm_weight(K, seed):
    rng = np.random.default_rng(seed)
    return (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)


def _assert_ulp(y, ref, max_ulp=1, max_frac=0.01, what=""):
    y = np.asarray(y, dtype=np.float16).astype(np.float64)
    ref = np.asarray(ref, dtype=np.float16)
    ulp = np.spacing(np.abs(ref)).astype(np.float64)
    d = np.abs(y - ref.astype(np.float64))
    assert np.all(d <= max_ulp * ulp), f"{what}: {np.max(d / ulp):.1f} ulp"
    frac = np.mean(d > 0)
    assert frac <= max_frac, f"{what}: {frac:.3%} of values differ"


@pytest.mark.parametrize("rows,dim", [(1, 3072), (7, 3072), (750, 3072), (3, 100), (2, 8192),
                                      (3, 16384), (2, 20000)])
def test_rms_norm(pkg, dev, rows, dim):
    import torch
    rng = np.random.default_rng(rows * 7 + dim)
    x = (rng.standard_normal((rows, dim)) * 3).astype(np.float16)
    w = _norm_weight(dim, dim)
    out = pkg.rms_norm(to_dev(x, dev), to_dev(w, dev), EPS, rows, dim)
    torch.cuda.synchronize()
    _assert_ulp(out.cpu().numpy(), o.rms_norm_ref(x, w, EPS), what=f"rms_norm {rows}x{dim}")


def test_rms_norm_misaligned_rows_take_the_scalar_kernel(pkg, dev):
    """Rows 2 bytes off a 16-byte boundary cannot use the 16-byte kernel: the
    scalar kernel gives the same result as an aligned copy."""
    import torch
    rng = np.random.default_rng(3)
    rows, dim = 9, 3072
    x = (rng.standard_normal((rows, dim)) * 3).astype(np.float16)
    w = _norm_weight(dim, 7)
    buf = torch.zeros(rows * dim + 1, dtype=torch.float16, device=dev)
    buf[1:].copy_(to_dev(x, dev).reshape(-1))
    xm = buf[1:].view(rows, dim)
    assert xm.data_ptr() % 16 != 0
    got = pkg.rms_norm(xm, to_dev(w, dev), EPS, rows, dim)
    torch.cuda.synchronize()
    _assert_ulp(got.cpu().numpy(), o.rms_norm_ref(x, w, EPS), what="misaligned rms_norm")


@pytest.mark.parametrize("rows,dim", [(1, 3072), (750, 3072), (5, 96), (4, 16384)])
def test_residual_rms_norm(pkg, dev, rows, dim):
    import torch
    rng = np.random.default_rng(rows + dim)
    a = (rng.standard_normal((rows, dim)) * 4).astype(np.float16)
    b = (rng.standard_normal((rows, dim)) * 2).astype(np.float16)
    w = _norm_weight(dim, dim + 1)
    res, nrm = pkg.residual_rms_norm(to_dev(a, dev), to_dev(b, dev), to_dev(w, dev), EPS, rows, dim)
    torch.cuda.synchronize()
    rres, rnrm = o.residual_rms_norm_ref(a, b, w, EPS)
    assert np.array_equal(res.cpu().numpy(), rres)
    _assert_ulp(nrm.cpu().numpy(), rnrm, what=f"residual_rms_norm {rows}x{dim}")


@pytest.mark.parametrize("rows,dim", [(3, 100), (2, 3072), (1, 20000)])
@pytest.mark.parametrize("alias", ["a", "b"])
def test_residual_rms_norm_in_place(pkg, dev, rows, dim, alias):
    """residual_out may be a or b itself (h = h + o in place).  dim % 8 != 0
    and dim > 16384 take the scalar kernel, whose second pass reads the stored
    residual back (recomputing it from a and b would add b twice); dim = 3072
    takes the 16-byte kernel.  norm_out may also replace an input."""
    import torch
    rng = np.random.default_rng(rows * 31 + dim)
    a = (rng.standard_normal((rows, dim)) * 4).astype(np.float16)
    b = (rng.standard_normal((rows, dim)) * 2).astype(np.float16)
    w = _norm_weight(dim, dim + 3)
    rres, rnrm = o.residual_rms_norm_ref(a, b, w, EPS)
    ta, tb = to_dev(a, dev), to_dev(b, dev)
    tgt = ta if alias == "a" else tb
    res, nrm = pkg.residual_rms_norm(ta, tb, to_dev(w, dev), EPS, rows, dim, residual_out=tgt)
    torch.cuda.synchronize()
    assert res.data_ptr() == tgt.data_ptr()
    assert np.array_equal(res.cpu().numpy(), rres)
    _assert_ulp(nrm.cpu().numpy(), rnrm, what=f"in-place residual_out={alias} {rows}x{dim}")
    # norm_out in place of an input (residual_out separate)
    ta, tb = to_dev(a, dev), to_dev(b, dev)
    tgt = ta if alias == "a" else tb
    res2, nrm2 = pkg.residual_rms_norm(ta, tb, to_dev(w, dev), EPS, rows, dim, norm_out=tgt)
    torch.cuda.synchronize()
    assert np.array_equal(res2.cpu().numpy(), rres)
    assert torch.equal(nrm2, nrm)


@pytest.mark.parametrize("rows,dim", [(3, 100), (2, 3072)])
def test_rms_norm_in_place(pkg, dev, rows, dim):
    import torch
    rng = np.random.default_rng(rows + 5 * dim)
    x = (rng.standard_normal((rows, dim)) * 3).astype(np.float16)
    w = _norm_weight(dim, 11)
    tx = to_dev(x, dev)
    out = pkg.rms_norm(tx, to_dev(w, dev), EPS, rows, dim, out=tx)
    torch.cuda.synchronize()
    _assert_ulp(out.cpu().numpy(), o.rms_norm_ref(x, w, EPS), what=f"in-place rms_norm {rows}x{dim}")


# (N, K, g): GEMV specialisations (K=3072 -> 32 lanes x 3, 2048 -> 64 x 1,
# 8192 -> 64 x 4, 4096 -> 64 x 2), the generic kernel (K=96), all group sizes.
RMS_SHAPES = [(5120, 3072, 64), (1000, 2048, 128), (257, 8192, 64), (64, 96, 32),
              (33, 4096, 32), (70, 28672, 64)]


@pytest.mark.parametrize("N,K,g", RMS_SHAPES)
def test_rmsnorm_matmul(pkg, dev, N, K, g):
    import torch
    x, [(w, s, b)] = o.make_inputs(1, N, K, g, seed=N + K)
    x = (x.astype(np.float32) * 5).astype(np.float16)   # the norm removes the scale
    nw = _norm_weight(K, K)
    xn = o.rms_norm_ref(x, nw, EPS)
    ref = o.matmul_q4_f64(xn, w, s, b, g)
    y = pkg.rmsnorm_matmul_q4(to_dev(x, dev), to_dev(nw, dev), EPS, q4w(pkg, w, s, b, K, g, dev), N)
    torch.cuda.synchronize()
    assert_parity(y.cpu().numpy(), ref, TOL_GEMV, f"rmsnorm_matmul N={N} K={K} g={g}")
    # same result as the unfused pair rms_norm -> matmul_q4 on the GPU
    xn_gpu = pkg.rms_norm(to_dev(x, dev), to_dev(nw, dev), EPS, 1, K)
    y2 = pkg.matmul_q4(xn_gpu, to_dev(w, dev), to_dev(s, dev), to_dev(b, dev), 1, K, N, g)
    torch.cuda.synchronize()
    assert_parity(y.cpu().numpy(), y2.cpu().numpy().astype(np.float64), TOL_GEMV, "fused vs unfused")


def test_rmsnorm_lm_head_full_size(pkg, dev):
    """Final norm + vocabulary head (LlamaModel.swift:219-220): N = 128256,
    two row-iterations per wave; 512 sampled rows against the oracle."""
    import torch
    N, K, g = 128256, 3072, 64
    x, [(w, s, b)] = gpu_inputs(1, N, K, g, seed=11, dev=dev)
    nw = _norm_weight(K, 12)
    y = pkg.rmsnorm_matmul_q4(x, to_dev(nw, dev), EPS, pkg.Q4Weight(w, s, b, K, g), N)
    torch.cuda.synchronize()
    rows = np.random.default_rng(1).choice(N, 512, replace=False)
    xn = o.rms_norm_ref(host(x), nw, EPS)
    ref = o.matmul_q4_f64(xn, host(w[rows]), host(s[rows]), host(b[rows]), g)
    assert_parity(y.cpu().numpy()[:, rows], ref, TOL_GEMV, "rmsnorm lm_head")


SWIGLU_SHAPES = [(8192, 3072, 64), (300, 2048, 128), (100, 96, 32), (64, 8192, 64),
                 (30, 20000, 32)]


@pytest.mark.parametrize("N,K,g", SWIGLU_SHAPES)
def test_residual_rmsnorm_swiglu(pkg, dev, N, K, g):
    import torch
    a, [(wg, sg, bg), (wu, su, bu)] = o.make_inputs(1, N, K, g, seed=N * 3 + K, n_weights=2)
    rng = np.random.default_rng(N)
    a = (a.astype(np.float32) * 4).astype(np.float16)
    bvec = (rng.standard_normal((1, K)) * 2).astype(np.float16)
    nw = _norm_weight(K, K + 5)
    rres, rn = o.residual_rms_norm_ref(a, bvec, nw, EPS)
    ref = o.silu_mul_f64(o.matmul_q4_f64(rn, wg, sg, bg, g), o.matmul_q4_f64(rn, wu, su, bu, g))
    res, y = pkg.residual_rmsnorm_matmul_q4_silu_mul(
        to_dev(a, dev), to_dev(bvec, dev), to_dev(nw, dev), EPS, q4w(pkg, wg, sg, bg, K, g, dev),
        q4w(pkg, wu, su, bu, K, g, dev), N)
    torch.cuda.synchronize()
    assert np.array_equal(res.cpu().numpy(), rres)
    assert_parity(y.cpu().numpy(), ref, TOL_GEMV, f"residual rmsnorm swiglu N={N} K={K} g={g}")


def _assert_residual(out, res, y64, tol, what):
    ref = o.residual_add_ref(res, y64).astype(np.float64)
    y64 = np.asarray(y64, dtype=np.float64)
    # the projection's own fp16 rounding (1 ulp of y) and the sum's (1 ulp of
    # the result), plus the matmul bound on y itself
    allow = (np.spacing(np.abs(y64).astype(np.float16)).astype(np.float64)
             + np.spacing(np.abs(ref.astype(np.float16))).astype(np.float64)
             + tol["rtol"] * np.abs(y64) + tol["atol_rms"] * np.sqrt(np.mean(y64 ** 2)))
    d = np.abs(np.asarray(out, dtype=np.float64) - ref)
    assert np.all(d <= allow), f"{what}: worst {np.max(d / allow):.2f}x the allowance"
    err = o.max_rel_err(out, ref)
    assert err <= GATE, f"{what}: max_rel_err {err:.2e}"


# (M, N, K, g): GEMV; GEMM with split-K (prefill down); small GEMM; generic GEMM path
RES_SHAPES = [(1, 3072, 8192, 64), (750, 3072, 8192, 64), (33, 192, 256, 64), (5, 100, 96, 32)]


@pytest.mark.parametrize("M,N,K,g", RES_SHAPES)
@pytest.mark.parametrize("in_place", [False, True])
def test_matmul_residual(pkg, dev, M, N, K, g, in_place):
    import torch
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=M + N + K)
    rng = np.random.default_rng(M * N)
    res = (rng.standard_normal((M, N)) * 6).astype(np.float16)
    y64 = o.matmul_q4_f64(x, w, s, b, g)
    res_d = to_dev(res, dev)
    out = res_d if in_place else None
    got = pkg.matmul_q4_residual(to_dev(x, dev), q4w(pkg, w, s, b, K, g, dev), res_d, M, N, out=out)
    torch.cuda.synchronize()
    tol = TOL_GEMV if M == 1 else TOL_GEMM_F16
    _assert_residual(got.cpu().numpy(), res, y64, tol, f"residual M={M} N={N} K={K} in_place={in_place}")


def test_decode_layer_fused_matches_unfused(pkg, dev):
    """One Llama-3.2-3B decode layer's matmul path, fused (4 launches) vs the
    reference's operator sequence built from this library's unfused ops
    (LlamaModel.swift:288-331; attention replaced by a fixed vector)."""
    import torch
    K, F, QKV = 3072, 8192, 5120
    gen = torch.Generator(device=dev)
    gen.manual_seed(21)
    x, [(wqkv, sqkv, bqkv)] = gpu_inputs(1, QKV, K, 64, seed=22, dev=dev)
    _, [(wo, so, bo)] = gpu_inputs(1, K, K, 64, seed=23, dev=dev)
    _, [(wg, sg, bg), (wu, su, bu)] = gpu_inputs(1, F, K, 64, seed=24, dev=dev, n_weights=2)
    _, [(wd, sd, bd)] = gpu_inputs(1, K, F, 64, seed=25, dev=dev)
    Q = lambda w, s, b, k: pkg.Q4Weight(w, s, b, k, 64)
    n1 = torch.from_numpy(_norm_weight(K, 1)).to(dev)
    n2 = torch.from_numpy(_norm_weight(K, 2)).to(dev)
    attn = torch.randn(1, K, generator=gen, device=dev).half()
    # fused
    qkv = pkg.rmsnorm_matmul_q4(x, n1, EPS, Q(wqkv, sqkv, bqkv, K), QKV)
    o_proj = pkg.linear(attn, Q(wo, so, bo, K), 1, K, K)
    res, act = pkg.residual_rmsnorm_matmul_q4_silu_mul(x, o_proj, n2, EPS, Q(wg, sg, bg, K),
                                                       Q(wu, su, bu, K), F)
    out = pkg.matmul_q4_residual(act, Q(wd, sd, bd, F), res, 1, K)
    # unfused, operator by operator
    xn = pkg.rms_norm(x, n1, EPS, 1, K)
    qkv2 = pkg.linear(xn, Q(wqkv, sqkv, bqkv, K), 1, K, QKV)
    res2, xn2 = pkg.residual_rms_norm(x, o_proj, n2, EPS, 1, K)
    act2 = pkg.matmul_q4_silu_mul(xn2, Q(wg, sg, bg, K), Q(wu, su, bu, K), 1, K, F)
    down2 = pkg.linear(act2, Q(wd, sd, bd, F), 1, F, K)
    out2 = (res2.float() + down2.float()).half()
    torch.cuda.synchronize()
    assert torch.equal(res, res2)
    _assert_two_paths(qkv, qkv2, TOL_GEMV, "qkv")
    _assert_two_paths(act, act2, TOL_GEMV, "gate/up")
    _assert_two_paths(out, out2, TOL_GEMV, "layer out")


def _assert_two_paths(a, b, tol, what):
    """Two fp16 GPU results of the same exact value v: each is within the
    GEMV bound of v before its own fp16 rounding (half an ulp), so they may
    differ by twice the bound plus one fp16 ulp (kernels with different
    instruction schedules round their fp32 sums differently)."""
    a = a.cpu().numpy().astype(np.float64)
    b16 = b.cpu().numpy()
    b = b16.astype(np.float64)
    allow = (2 * (tol["rtol"] * np.abs(b) + tol["atol_rms"] * np.sqrt(np.mean(b ** 2)))
             + np.spacing(np.abs(b16)).astype(np.float64))
    d = np.abs(a - b)
    assert np.all(d <= allow), f"{what}: worst {np.max(d / allow):.2f}x the allowance"
    assert o.max_rel_err(a, b) <= GATE, what


# (M, N, K, g): GEMV; GEMM; GEMM with split-K (few output tiles); generic path
GEGLU_SHAPES = [(1, 2048, 512, 64), (33, 1024, 512, 64), (750, 512, 8192, 64), (7, 100, 96, 32)]


@pytest.mark.parametrize("M,N,K,g", GEGLU_SHAPES)
def test_geglu(pkg, dev, M, N, K, g):
    """T5 encoder FFN gate/up (T5Encoder.swift:191-199) against the fp64
    closed form with GELU-tanh (inner clamp +-10)."""
    import torch
    x, [(wg, sg, bg), (wu, su, bu)] = o.make_inputs(M, N, K, g, seed=M + N + K, n_weights=2)
    gv = o.matmul_q4_f64(x, wg, sg, bg, g)
    uv = o.matmul_q4_f64(x, wu, su, bu, g)
    ref = o.gelu_tanh_f64(gv) * uv
    y = pkg.matmul_q4_geglu(to_dev(x, dev), q4w(pkg, wg, sg, bg, K, g, dev),
                            q4w(pkg, wu, su, bu, K, g, dev), M, K, N)
    torch.cuda.synchronize()
    y = y.cpu().numpy().astype(np.float64)
    assert o.max_rel_err(y, ref) <= GATE
    # each product carries the matmul bound, propagated through gelu(g) * u
    tol = TOL_GEMV if M == 1 else TOL_GEMM_F16
    eg = tol["rtol"] * np.abs(gv) + tol["atol_rms"] * np.sqrt(np.mean(gv ** 2))
    eu = tol["rtol"] * np.abs(uv) + tol["atol_rms"] * np.sqrt(np.mean(uv ** 2))
    allow = (_gelu_slope(gv) * np.abs(uv) * eg + np.abs(o.gelu_tanh_f64(gv)) * eu
             + np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64))
    d = np.abs(y - ref)
    assert np.all(d <= allow), f"geglu M={M}: worst {np.max(d / allow):.2f}x the allowance"


def _gelu_slope(v):
    """|d gelu_tanh / dv| at v, plus a margin for the curvature over the
    (small) error interval."""
    c = 0.7978845608
    t = np.tanh(np.clip(c * (v + 0.044715 * v ** 3), -10, 10))
    d = 0.5 * (1 + t) + 0.5 * v * (1 - t * t) * c * (1 + 3 * 0.044715 * v * v)
    return np.abs(d) + 0.2


@pytest.mark.parametrize("vocab,K,g", [(1000, 3072, 64), (300, 96, 32), (50, 4096, 128)])
def test_embedding_q4(pkg, dev, vocab, K, g):
    """Bit-exact against the oracle (fp32 q*s + b, one fp16 rounding); ids out
    of range give zero rows."""
    import torch
    _, [(w, s, b)] = o.make_inputs(1, vocab, K, g, seed=vocab + K)
    rng = np.random.default_rng(vocab)
    ids = np.concatenate([rng.integers(0, vocab, 37), [0, vocab - 1, -1, vocab, 5]]).astype(np.int32)
    out = pkg.embedding_q4(q4w(pkg, w, s, b, K, g, dev), vocab, to_dev(ids, dev))
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), o.embedding_q4_ref(w, s, b, ids, g))


def test_embedding_q4_full_vocab(pkg, dev):
    """Llama-3.2-3B tied embedding size (128256 x 3072): sampled ids."""
    import torch
    vocab, K, g = 128256, 3072, 64
    _, [(w, s, b)] = gpu_inputs(1, vocab, K, g, seed=31, dev=dev)
    ids = np.random.default_rng(2).integers(0, vocab, 64).astype(np.int32)
    out = pkg.embedding_q4(pkg.Q4Weight(w, s, b, K, g), vocab, to_dev(ids, dev))
    torch.cuda.synchronize()
    idt = torch.from_numpy(ids.astype(np.int64)).to(dev)
    ref = o.embedding_q4_ref(host(w[idt]), host(s[idt]), host(b[idt]), np.arange(len(ids)), g)
    assert np.array_equal(out.cpu().numpy(), ref)


# (M, N, K, g): the prefill o (K = 3072) and down (K = 8192) shapes at M = 750,
# small and multi-row shapes, the generic GEMM (K % 128 != 0), M = 1.
RRN_SHAPES = [(750, 3072, 3072, 64), (750, 3072, 8192, 64), (33, 192, 256, 64),
              (1000, 2048, 512, 128), (5, 96, 96, 32), (1, 3072, 3072, 64)]


@pytest.mark.parametrize("M,N,K,g", RRN_SHAPES)
@pytest.mark.parametrize("sum_rounded", [False, True])
def test_matmul_residual_rms_norm(pkg, dev, M, N, K, g, sum_rounded):
    """linear + residual add + RMSNorm in one call (LlamaModel.swift:269-272 with
    the unrounded sum of squares, :278-279 then :233 with the rounded stream)
    against the oracle: the residual stream within the residual epilogue's
    bound; the normalized rows within 1 fp16 ulp of half(r * rms * w), with r
    the GPU's own residual stream and rms from the oracle's fp64 sum of squares
    (of float(residual) + float(half(y)) unrounded, or of the rounded sum).
    The oracle's half(y) differs from the GPU's projection in the last fp16 bit
    on a few elements (within the GEMM bound), which moves one row's sum of
    squares by ~1e-5 relative: up to 5% of a row's values may then sit on the
    other side of an fp16 rounding boundary (still within 1 ulp).  The bit-exact
    test below pins the fused call to the unfused GPU sequence."""
    import torch
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=M + N + K)
    rng = np.random.default_rng(M * N + 1)
    res = (rng.standard_normal((M, N)) * 6).astype(np.float16)
    nw = _norm_weight(N, N + 3)
    y64 = o.matmul_q4_f64(x, w, s, b, g)
    r_dev, n_dev = pkg.matmul_q4_residual_rms_norm(to_dev(x, dev), q4w(pkg, w, s, b, K, g, dev),
                                                    to_dev(res, dev), to_dev(nw, dev), EPS, M, N,
                                                    sum_rounded)
    torch.cuda.synchronize()
    got_r, got_n = r_dev.cpu().numpy(), n_dev.cpu().numpy()
    what = f"M={M} N={N} K={K} g={g} sum_rounded={sum_rounded}"
    _assert_residual(got_r, res, y64, TOL_GEMM_F16, what)
    v = res.astype(np.float32) + y64.astype(np.float16).astype(np.float32)
    q = v.astype(np.float16).astype(np.float64) if sum_rounded else v.astype(np.float64)
    rms = (1.0 / np.sqrt(np.sum(q * q, axis=-1, keepdims=True) / N + EPS)).astype(np.float32)
    ref_n = ((got_r.astype(np.float32) * rms) * nw).astype(np.float16)
    _assert_ulp(got_n, ref_n, max_frac=0.05, what=what)


@pytest.mark.parametrize("K", [3072, 8192])
@pytest.mark.parametrize("sum_rounded", [False, True])
def test_matmul_residual_rms_norm_equals_unfused(pkg, dev, K, sum_rounded):
    """At the prefill shapes (M = 750, N = 3072; split-K in both plans) the fused
    call equals, bit for bit, this library's unfused sequence: the GEMM, then
    sltx_residual_rms_norm (o_proj step) or the residual GEMM epilogue and
    sltx_rms_norm (down_proj step and the next input norm).  Also in place
    (residual_out == residual)."""
    import torch
    M, N, g = 750, 3072, 64
    x, [(w, s, b)] = gpu_inputs(M, N, K, g, seed=K + 7, dev=dev)
    W = pkg.Q4Weight(w, s, b, K, g)
    gen = torch.Generator(device=dev)
    gen.manual_seed(K)
    res = (torch.randn(M, N, generator=gen, device=dev) * 6).half()
    nw = torch.from_numpy(_norm_weight(N, 5)).to(dev)
    fr, fn = pkg.matmul_q4_residual_rms_norm(x, W, res, nw, EPS, M, N, sum_rounded)
    if sum_rounded:
        ur = pkg.matmul_q4_residual(x, W, res, M, N)
        un = pkg.rms_norm(ur, nw, EPS, M, N)
    else:
        y = pkg.matmul_q4_fast(x, w, s, b, M, K, N, g)
        ur, un = pkg.residual_rms_norm(res, y, nw, EPS, M, N)
    inplace = res.clone()
    ir, inn = pkg.matmul_q4_residual_rms_norm(x, W, inplace, nw, EPS, M, N, sum_rounded,
                                              residual_out=inplace)
    torch.cuda.synchronize()
    assert torch.equal(fr, ur) and torch.equal(fn, un)
    assert ir.data_ptr() == inplace.data_ptr()
    assert torch.equal(ir, ur) and torch.equal(inn, un)
