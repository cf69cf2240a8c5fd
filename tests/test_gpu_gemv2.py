"""GPU parity of the two-row GEMV (M == 2, one weight set of at most
5120 x 4096, fp16 x; q4_gemv.hip with two x rows): each weight word is
dequantized once and dotted with both rows' prepared x.

Reference semantics: matmul_q4 (Kernels.swift:444-620) serves any M through
the same per-row dot (matmulQ4, Ops.swift:285-305); matmulQ4Fast /
matmulQ4FastF32 (Ops.swift:312-381) give the same product; the single-set
epilogues are linear + elemAdd (LlamaModel.swift:330-331) and DiTLinear's
bias + GELU-tanh (DiTModel.swift:102-125).  Covered: every lanes-per-row
and chunks-per-lane kernel the route takes (K = 512 .. 4096), odd row counts,
every group size, fp16 / fp32 / bf16 outputs (fp32 and fp16 agree bit for
bit), the epilogues (residual also in place), and a bit-exact check of the
dequantization with a different one-hot row in each of the two x rows.
"""
import numpy as np
import pytest

from helpers import TOL_GEMM_BF16, TOL_GEMM_F16, TOL_GEMV, assert_parity, q4w, to_dev
from oracle import q4_oracle as o

pytestmark = pytest.mark.gpu

# (N, K, g)
SHAPES = [
    (3072, 3072, 64), (5120, 3072, 64), (4096, 4096, 64), (4096, 4096, 128), (1000, 2048, 32),
    (77, 1024, 128), (257, 512, 64), (33, 3072, 32), (5, 512, 32), (500, 1536, 32), (130, 3072, 128),
    (3, 2048, 64),
]


@pytest.mark.parametrize("N,K,g", SHAPES)
def test_gemv2_shapes(pkg, dev, N, K, g):
    import torch
    assert pkg.gemm_route(2, N, K, group_size=g) == "gemv"
    x, [(w, s, b)] = o.make_inputs(2, N, K, g, seed=N * 5 + K + g)
    args = [to_dev(a, dev) for a in (x, w, s, b)]
    y16 = pkg.matmul_q4(*args, 2, K, N, g)
    yf = pkg.matmul_q4_fast(*args, 2, K, N, g)
    y32 = pkg.matmul_q4_fast_f32(*args, 2, K, N, g)
    torch.cuda.synchronize()
    assert_parity(y16.cpu().numpy(), o.matmul_q4_f64(x, w, s, b, g), TOL_GEMV,
                  f"N={N} K={K} g={g}")
    assert torch.equal(yf, y16)
    assert torch.equal(y32.half(), y16)


@pytest.mark.parametrize("K,g", [(3072, 64), (512, 128), (4096, 32)])
def test_gemv2_dequant_bit_exact(pkg, dev, K, g):
    """Row 0 of x is one-hot at k, row 1 at another column: each output is
    one dequantized weight, fp16(s*q+b) exactly, and with s = 1, b = 0 the
    unpacked code."""
    import torch
    N = 64
    rng = np.random.default_rng(K + g)
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    w = o.pack_q4(q)
    _, [(_, s, b)] = o.make_inputs(1, N, K, g, seed=K + 3)
    ones, zeros = np.ones_like(s), np.zeros_like(b)
    tw, ts, tb = to_dev(w, dev), to_dev(s, dev), to_dev(b, dev)
    t1, t0 = to_dev(ones, dev), to_dev(zeros, dev)
    deq = o.dequant_f64(w, s, b, g).astype(np.float16)
    ks = sorted(set(list(range(10)) + [31, 32, g - 1, g, K // 2 + 5, K - 1]))
    for k in ks:
        k2 = (K - 1 - k) % K
        x = np.zeros((2, K), np.float16)
        x[0, k] = 1.0
        x[1, k2] = 1.0
        tx = to_dev(x, dev)
        yq = pkg.matmul_q4(tx, tw, t1, t0, 2, K, N, g)
        yd = pkg.matmul_q4(tx, tw, ts, tb, 2, K, N, g)
        torch.cuda.synchronize()
        yq, yd = yq.cpu().numpy(), yd.cpu().numpy()
        for row, kk in ((0, k), (1, k2)):
            assert np.array_equal(yq[row].astype(np.int64), q[:, kk].astype(np.int64)), (k, row)
            assert np.array_equal(yd[row].view(np.uint16), deq[:, kk].view(np.uint16)), (k, row)


@pytest.mark.parametrize("N,K", [(3072, 3072), (200, 4096)])
def test_gemv2_epilogues(pkg, dev, N, K):
    """Residual add (also in place), bias + GELU-tanh to fp32, bias to bf16."""
    import torch
    g, M = 64, 2
    assert pkg.gemm_route(M, N, K) == "gemv"
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=N + K)
    rng = np.random.default_rng(N)
    res = rng.standard_normal((M, N)).astype(np.float16)
    bias = rng.standard_normal(N).astype(np.float32)
    wt = q4w(pkg, w, s, b, K, g, dev)
    proj = o.matmul_q4_f64(x, w, s, b, g)
    y = pkg.matmul_q4_residual(to_dev(x, dev), wt, to_dev(res, dev), M, N)
    inplace = to_dev(res, dev)
    pkg.matmul_q4_residual(to_dev(x, dev), wt, inplace, M, N, out=inplace)
    yg = pkg.matmul_q4_ex(to_dev(x, dev), wt, M, N, out_dtype=torch.float32,
                          bias=to_dev(bias, dev), epilogue=pkg.SLTX_EPI_GELU_TANH)
    yb = pkg.matmul_q4_ex(to_dev(x, dev), wt, M, N, out_dtype=torch.bfloat16,
                          bias=to_dev(bias, dev))
    torch.cuda.synchronize()
    want = res.astype(np.float64) + proj.astype(np.float16).astype(np.float64)
    # the sum is rounded to fp16 once more: the fp16 output tolerance
    assert_parity(y.cpu().numpy(), want, TOL_GEMM_F16, f"residual N={N}")
    assert torch.equal(inplace, y)
    assert_parity(yg.cpu().numpy(), o.gelu_tanh_f64(proj + bias), TOL_GEMV, f"bias+gelu N={N}")
    assert_parity(yb.float().cpu().numpy(), proj + bias, TOL_GEMM_BF16, f"bias bf16 N={N}")


def test_gemv2_in_graph(pkg, dev):
    """The route allocates nothing: captured into a HIP graph, every replay
    equals the eager result."""
    import torch
    M, N, K, g = 2, 3072, 3072, 64
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=11)
    args = [to_dev(a, dev) for a in (x, w, s, b)]
    eager = pkg.matmul_q4(*args, M, K, N, g)
    out = torch.empty_like(eager)
    st = torch.cuda.Stream()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=st):
        pkg.matmul_q4(*args, M, K, N, g, out=out, stream=st)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
