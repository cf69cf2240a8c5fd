"""Seeded random shapes through the dispatch routes of the 4-bit matmul.

Each case draws (M, N, K, group size) from its own fixed seed, so a failure
names a reproducible shape.  The draws cover what the hand-picked shape lists
do not: odd N (partial weight tiles and unaligned output rows), K that the
specialised GEMV kernels do not take (the generic kernel), every group size,
split and unsplit GEMM plans.

Reference semantics: matmulQ4 / matmulQ4Fast / matmulQ4FastF32
(Ops.swift:285-381) and the SwiGLU pair (LlamaModel.swift:275-277, 327-329),
checked against the fp64 oracle at the tolerances of tests/helpers.py.  The
f16 GEMM is also checked against the product with weights rounded to fp16 as
the kernel rounds them, which leaves only fp32 accumulation error.
"""
import numpy as np
import pytest

from helpers import (TOL_GEMM_BF16, TOL_GEMM_F16, TOL_GEMV, TOL_ROUNDED_W, assert_parity, q4w,
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
