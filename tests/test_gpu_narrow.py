"""GPU parity of the narrow-M route (q4_narrow.hip: one weight set, M <= 4,
K a multiple of 512 with K / 512 in {4, 6, 8, 10, 12, 16, 20}) through the C
ABI.

The route takes those launches unless the small-M route would run two row
tiles per block at two blocks per CU: N >= 8161 with K <= 3072 (the
vocabulary head; tests/test_gpu_skinny.py covers that case).  Same semantics
as the GEMM (matmulQ4Fast / matmulQ4FastF32, Ops.swift:312-381): weights
dequantized to fp16 as s*q+b in one fp16 FMA, fp32 accumulation.  Checked
against the fp64 oracle, against the fp16-rounded weights, and bit for bit
through unit vectors.
"""
import numpy as np
import pytest

from helpers import (TOL_GEMM_BF16, TOL_GEMM_F16, TOL_ROUNDED_W, assert_parity, q4w,
                     rounded_weights_f16, to_dev)
from oracle import q4_oracle as o

pytestmark = pytest.mark.gpu

# (M, N, K, g).  The K split S doubles (up to 4, while the runs divide) until
# ceil(N / 4) * S reaches 4096 waves: small N gives S = 4 (or 2 when K / 512
# is 6 or 10), N around 4000-10000 gives S = 2, and N >= 16384 gives S = 1.
# Every run count, N not a multiple of 4, every group size, M = 1..4, and at
# most 78 KB of X in LDS (M * K * 2 bytes; M = 3 at K = 10240).
SHAPES = [
    (1, 50, 2048, 64), (2, 33, 6144, 32), (3, 64, 4096, 128), (4, 97, 5120, 64),
    (2, 41, 6144, 64), (3, 30, 8192, 32), (3, 21, 10240, 64), (1, 5, 3072, 64),
    (2, 6000, 2048, 64), (4, 4000, 3072, 64), (3, 10001, 4096, 32), (4, 10002, 6144, 128),
    (1, 16400, 4096, 64), (2, 16401, 5120, 128),
]

@pytest.mark.parametrize("M,N,K,g", SHAPES)
def test_narrow_shapes(pkg, dev, M, N, K, g):
    import torch
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=M * 131 + N + K)
    args = [to_dev(a, dev) for a in (x, w, s, b)]
    y32 = pkg.matmul_q4_fast_f32(*args, M, K, N, g)
    y16 = pkg.matmul_q4_fast(*args, M, K, N, g)
    torch.cuda.synchronize()
    y = y32.cpu().numpy()
    assert_parity(y, o.matmul_q4_f64(x, w, s, b, g), TOL_GEMM_F16, f"M={M} N={N} K={K}")
    ok, worst = o.elementwise_ok(y, x.astype(np.float64) @ rounded_weights_f16(w, s, b, g).T,
                                 **TOL_ROUNDED_W)
    assert ok, worst
    assert torch.equal(y32.half(), y16)


@pytest.mark.parametrize("M,N,K,g", [(4, 48, 2048, 64), (4, 52, 4096, 128), (3, 40, 3072, 32),
                                     (4, 9000, 4096, 64)])
def test_narrow_dequant_bit_exact(pkg, dev, M, N, K, g):
    """x rows are unit vectors e_k (M per call, over every k): each output is
    one dequantized weight, exact in fp32, so every lane, piece, run, wave
    and nibble position of the route is checked bit for bit against
    fp16(s*q+b), and with s = 1, b = 0 against the unpacked codes."""
    import torch
    _, [(w, s, b)] = o.make_inputs(1, N, K, g, seed=K + g + M)
    want = rounded_weights_f16(w, s, b, g).T.astype(np.float32)     # [K, N]
    codes = o.unpack_q4(w).T.astype(np.float32)
    tw, ts, tb = to_dev(w, dev), to_dev(s, dev), to_dev(b, dev)
    ones, zeros = to_dev(np.ones_like(s), dev), to_dev(np.zeros_like(b), dev)
    step = K // M
    for c in range(step):
        ks = np.arange(M) * step + c          # spread over runs and pieces
        x = np.zeros((M, K), dtype=np.float16)
        x[np.arange(M), ks] = 1.0
        tx = to_dev(x, dev)
        y = pkg.matmul_q4_fast_f32(tx, tw, ts, tb, M, K, N, g)
        yq = pkg.matmul_q4_fast_f32(tx, tw, ones, zeros, M, K, N, g)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), want[ks]), c
        assert np.array_equal(yq.cpu().numpy(), codes[ks]), c


@pytest.mark.parametrize("M", [2, 3, 4])
def test_narrow_residual_bias_gelu_dtypes(pkg, dev, M):
    """The single-set epilogues on the narrow route: residual add
    (linear + elemAdd, LlamaModel.swift:330-331), bias + GELU-tanh
    (DiTLinear's q4 branch, DiTModel.swift:102-125), and fp32 / bf16
    outputs (the residual entry sends M = 1 to the GEMV)."""
    import torch
    N, K, g = 158, 6144, 64   # K > 4096: M = 2 stays off the two-row GEMV
    assert pkg.gemm_route(M, N, K, group_size=g) == "narrow"
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=700 + M)
    rng = np.random.default_rng(M)
    res = rng.standard_normal((M, N)).astype(np.float16)
    bias = rng.standard_normal(N).astype(np.float32)
    wt = q4w(pkg, w, s, b, K, g, dev)
    proj = o.matmul_q4_f64(x, w, s, b, g)
    tx = to_dev(x, dev)
    y = pkg.matmul_q4_residual(tx, wt, to_dev(res, dev), M, N)
    yg = pkg.matmul_q4_ex(tx, wt, M, N, out_dtype=torch.float32, bias=to_dev(bias, dev),
                          epilogue=pkg.SLTX_EPI_GELU_TANH)
    yb = pkg.matmul_q4_ex(tx, wt, M, N, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    want = (res.astype(np.float64) + proj.astype(np.float16).astype(np.float64))
    assert_parity(y.cpu().numpy(), want, TOL_GEMM_F16, f"residual M={M}")
    assert_parity(yg.cpu().numpy(), o.gelu_tanh_f64(proj + bias), TOL_GEMM_F16,
                  f"bias+gelu M={M}")
    assert_parity(yb.float().cpu().numpy(), proj, TOL_GEMM_BF16,
                  f"bf16 out M={M}")


def test_narrow_in_graph(pkg, dev):
    """The route allocates nothing: it captures into a HIP graph as is, and the
    replays match the eager result."""
    import torch
    M, N, K, g = 4, 512, 3072, 64
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=9)
    args = [to_dev(a, dev) for a in (x, w, s, b)]
    eager = pkg.matmul_q4_fast(*args, M, K, N, g)
    out = torch.empty_like(eager)
    st = torch.cuda.Stream()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=st):
        pkg.matmul_q4_fast(*args, M, K, N, g, out=out, stream=st)
    for _ in range(3):
        out.zero_()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
