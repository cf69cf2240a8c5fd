"""Seeded random shapes through the dispatch routes of the 4-bit matmul.

Each case draws (M, N, K, group size) from its own fixed seed, so a failure
names a reproducible shape.  The draws cover what the hand-picked shape lists
do not: odd N (partial weight tiles and unaligned output rows), K that the
specialised GEMV kernels do not take (the generic kernel), every group size,
split and unsplit GEMM plans.  A second set aims model-scale shapes at each
M > 1 route (narrow, small-M, mid-M with and without K halves, wide-M with
its K splits, the two-row GEMV, the GEMM) with the epilogues and output
dtypes of each.

Reference semantics: matmulQ4 / matmulQ4Fast / matmulQ4FastF32
(Ops.swift:285-381), the SwiGLU pair (LlamaModel.swift:275-277, 327-329),
the GeGLU pair (T5Encoder.swift:191-199), the residual add
(LlamaModel.swift:330-331) and DiTLinear's bias + GELU-tanh
(DiTModel.swift:102-125),
checked against the fp64 oracle at the tolerances of tests/helpers.py.  The
f16 GEMM is also checked against the product with weights rounded to fp16 as
the kernel rounds them, which leaves only fp32 accumulation error.
"""
import numpy as np
import pytest

from helpers import (GATE, TOL_GEMM_BF16, TOL_GEMM_F16, TOL_GEMV, TOL_ROUNDED_W, assert_parity, q4w,
                     rounded_weights_f16, to_dev)
from oracle import q4_oracle as o

pytestmark = pytest.mark.gpu


def _shape(seed, m_max, n_max, k_max):
    rng = np.random.default_rng(seed)
    g = int(rng.choice([32, 64, 128]))
    K = g * int(rng.integers(1, k_max // g + 1))
    M = int(rng.integers(2, m_max + 1)) if m_max > 1 else 1
    N = int(rng.integers(1, n_max + 1))
    return M, N, K, g


@pytest.mark.parametrize("case", range(20))
def test_random_gemm_f16(pkg, dev, case):
    import torch
    M, N, K, g = _shape(9000 + case, 300, 600, 2048)
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=case)
    y = pkg.matmul_q4_fast_f32(to_dev(x, dev), to_dev(w, dev), to_dev(s, dev), to_dev(b, dev), M,
                               K, N, g)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    what = f"M={M} N={N} K={K} g={g}"
    assert_parity(y, o.matmul_q4_f64(x, w, s, b, g), TOL_GEMM_F16, what)
    ok, worst = o.elementwise_ok(y, x.astype(np.float64) @ rounded_weights_f16(w, s, b, g).T,
                                 **TOL_ROUNDED_W)
    assert ok, (what, worst)


@pytest.mark.parametrize("case", range(8))
def test_random_gemm_bf16(pkg, dev, case):
    import torch
    M, N, K, g = _shape(9100 + case, 300, 600, 2048)
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=case, x_dtype="bf16")
    y = pkg.matmul_q4_ex(to_dev(x, dev).view(torch.bfloat16), q4w(pkg, w, s, b, K, g, dev), M, N,
                         out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_parity(y.cpu().numpy(), o.matmul_q4_f64(o.x_values(x, "bf16"), w, s, b, g),
                  TOL_GEMM_BF16, f"bf16 M={M} N={N} K={K} g={g}")


@pytest.mark.parametrize("case", range(20))
def test_random_gemv(pkg, dev, case):
    """M = 1: matmul_q4 takes the GEMV (specialised (L, CPL) kernels or, for K
    they do not cover, the generic one)."""
    import torch
    _, N, K, g = _shape(9200 + case, 1, 3000, 8192)
    x, [(w, s, b)] = o.make_inputs(1, N, K, g, seed=case)
    y = pkg.matmul_q4(to_dev(x, dev), to_dev(w, dev), to_dev(s, dev), to_dev(b, dev), 1, K, N, g)
    torch.cuda.synchronize()
    assert_parity(y.cpu().numpy(), o.matmul_q4_f64(x, w, s, b, g), TOL_GEMV,
                  f"gemv N={N} K={K} g={g}")


@pytest.mark.parametrize("case", range(10))
def test_random_swiglu(pkg, dev, case):
    """silu(x.Wg^T) * (x.Wu^T): M = 1 (fused GEMV) for even cases, M > 1
    (GEMM with the paired epilogue) for odd ones."""
    import torch
    M, N, K, g = _shape(9300 + case, 1 if case % 2 == 0 else 200, 1500, 3072)
    x, [(wg, sg, bg), (wu, su, bu)] = o.make_inputs(M, N, K, g, seed=case, n_weights=2)
    ref = o.silu_mul_f64(o.matmul_q4_f64(x, wg, sg, bg, g), o.matmul_q4_f64(x, wu, su, bu, g))
    y = pkg.matmul_q4_silu_mul(to_dev(x, dev), q4w(pkg, wg, sg, bg, K, g, dev),
                               q4w(pkg, wu, su, bu, K, g, dev), M, K, N)
    torch.cuda.synchronize()
    tol = TOL_GEMV if M == 1 else TOL_GEMM_F16
    assert_parity(y.cpu().numpy(), ref, tol, f"swiglu M={M} N={N} K={K} g={g}")


def _route_case(seed):
    """A shape aimed at one M > 1 route by seed % 7 (M <= 4, 5..32, 33..128,
    129..256, 257..519, the two-row GEMV, the mid-M K halves), model-scale
    N and K (ragged N too), and one of seven epilogues."""
    r = np.random.default_rng(seed)
    fam = seed % 7
    M = [int(r.integers(2, 5)), int(r.integers(5, 33)), int(r.integers(33, 129)),
         int(r.integers(129, 257)), int(r.integers(257, 520)), 2, int(r.integers(9, 33))][fam]
    g = int(r.choice([32, 64, 128], p=[0.25, 0.5, 0.25]))
    if fam == 5:
        N, K = int(r.integers(1, 5121)), 32 * int(r.integers(1, 129))
    elif fam == 6:
        N, K = int(r.integers(1, 4097)), int(r.choice([4096, 8192, 10240]))
    elif r.random() < 0.6:
        N = int(r.choice([3072, 4096, 5120, 8192, 1024, 2048]))
        K = int(r.choice([1024, 2048, 3072, 4096, 8192, 10240]))
    else:
        N, K = int(r.integers(1, 6000)), 128 * int(r.integers(1, 65))
    if r.random() < 0.3:
        N = max(1, N + int(r.integers(-31, 32)))
    K = max(g, K - K % g)
    epi = str(r.choice(["none", "residual", "bias_gelu_f32", "bias_bf16", "silu", "gelu", "f16"]))
    if epi in ("silu", "gelu") and N * K > 8192 * 10240:
        N = 8192
    return M, N, K, g, epi


@pytest.mark.parametrize("case", range(42))
def test_random_routes(pkg, dev, case):
    """Every M > 1 route at model-scale shapes with its epilogues, checked on
    six rows against the oracle: fp32 out (and a repeat equal bit for bit),
    fp16 out (equal to the fp32 result rounded), residual add, bias +
    GELU-tanh to fp32, bias to bf16, and the SiLU / GELU gated pairs."""
    import torch
    seed = 20000 + case
    M, N, K, g, epi = _route_case(seed)
    pair = epi in ("silu", "gelu")
    what = f"M={M} N={N} K={K} g={g} {epi} ({pkg.gemm_route(M, N, K, group_size=g, gated=pair)})"
    x, sets = o.make_inputs(M, N, K, g, seed=seed, n_weights=2 if pair else 1)
    rows = np.unique(np.array([0, 1, M // 3, M // 2, M - 2, M - 1]))
    xs = x[rows].astype(np.float64)
    tx = to_dev(x, dev)
    if pair:
        gate, up = (q4w(pkg, *w, K, g, dev) for w in sets)
        fn = pkg.matmul_q4_geglu if epi == "gelu" else pkg.matmul_q4_silu_mul
        y = fn(tx, gate, up, M, K, N)
        torch.cuda.synchronize()
        gp, upv = (o.matmul_q4_f64(xs, *w, g) for w in sets)
        want = o.gelu_tanh_f64(gp) * upv if epi == "gelu" else o.silu_mul_f64(gp, upv)
        assert o.max_rel_err(y.cpu().numpy()[rows].astype(np.float64), want) <= GATE, what
        return
    w, s, b = sets[0]
    proj = o.matmul_q4_f64(xs, w, s, b, g)
    raw = [to_dev(a, dev) for a in (w, s, b)]
    rng = np.random.default_rng(seed + 1)
    if epi == "none":
        y = pkg.matmul_q4_fast_f32(tx, *raw, M, K, N, g)
        again = pkg.matmul_q4_fast_f32(tx, *raw, M, K, N, g)
        torch.cuda.synchronize()
        assert torch.equal(y, again), what
        assert_parity(y.cpu().numpy()[rows], proj, TOL_GEMM_F16, what)
    elif epi == "f16":
        y = pkg.matmul_q4_fast(tx, *raw, M, K, N, g)
        y32 = pkg.matmul_q4_fast_f32(tx, *raw, M, K, N, g)
        torch.cuda.synchronize()
        assert torch.equal(y32.half(), y), what
        assert_parity(y.cpu().numpy()[rows], proj, TOL_GEMM_F16, what)
    elif epi == "residual":
        res = rng.standard_normal((M, N)).astype(np.float16)
        y = pkg.matmul_q4_residual(tx, q4w(pkg, w, s, b, K, g, dev), to_dev(res, dev), M, N)
        torch.cuda.synchronize()
        want = res[rows].astype(np.float64) + proj.astype(np.float16).astype(np.float64)
        assert_parity(y.cpu().numpy()[rows], want, TOL_GEMM_F16, what)
    else:
        bias = rng.standard_normal(N).astype(np.float32)
        gelu = epi == "bias_gelu_f32"
        y = pkg.matmul_q4_ex(tx, q4w(pkg, w, s, b, K, g, dev), M, N,
                             out_dtype=torch.float32 if gelu else torch.bfloat16,
                             bias=to_dev(bias, dev),
                             epilogue=pkg.SLTX_EPI_GELU_TANH if gelu else pkg.SLTX_EPI_NONE)
        torch.cuda.synchronize()
        if gelu:
            assert_parity(y.cpu().numpy()[rows], o.gelu_tanh_f64(proj + bias), TOL_GEMM_F16, what)
        else:
            assert_parity(y.float().cpu().numpy()[rows], proj + bias, TOL_GEMM_BF16, what)
