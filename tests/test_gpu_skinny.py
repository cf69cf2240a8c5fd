"""GPU parity of the small-M route (q4_skinny.hip: M <= 32, K a multiple of
1024 or of 2048) through the C ABI.

The narrow route (q4_narrow.hip, tests/test_gpu_narrow.py) runs one weight
set at M <= 4 where it applies (K / 512 in {4, 6, 8, 10, 12, 16, 20},
M * K * 2 <= 78 KB), unless this route runs two row tiles per block at two
blocks per CU (N >= 8161, K <= 3072).  The shapes here keep this route's own
configurations covered: gated pairs, M > 4, that two-tile case at M <= 4,
K = 1024, or X too large for the narrow route's LDS.

Same semantics as the GEMM (matmulQ4Fast / matmulQ4FastF32, Ops.swift:312-381;
the SwiGLU and GeGLU pairs, LlamaModel.swift:275-277 and
T5Encoder.swift:191-199): the weights are dequantized to fp16 as s*q+b in one
fp16 FMA and multiplied with fp32 accumulation, so the outputs are checked
against the fp64 oracle (tolerances of tests/helpers.py), against the
fp16-rounded weights, and bit for bit through unit vectors.
"""
import numpy as np
import pytest

from helpers import (TOL_GEMM_F16, TOL_ROUNDED_W, assert_parity, q4w, rounded_weights_f16,
                     to_dev)
from oracle import q4_oracle as o

pytestmark = pytest.mark.gpu

# (M, N, K, g): every tile count and step count the route instantiates
# (8 waves x 1..6 steps for M <= 16, x 1..4 for M <= 32; 16 waves x 1..5),
# N not a multiple of 16, every group size.  (At K = 4096 above 16 rows and
# at K = 10240 above 8, a set of at most 4096 rows takes the mid-M route.)
SHAPES = [
    (3, 200, 1024, 64), (5, 64, 2048, 32), (16, 100, 3072, 64), (8, 48, 4096, 128),
    (5, 80, 5120, 64), (7, 33, 6144, 64), (17, 96, 1024, 32), (32, 112, 1024, 64),
    (24, 4150, 4096, 128), (22, 4160, 4096, 64), (6, 96, 8192, 64), (16, 4200, 10240, 64),
    (9, 24, 14336, 32), (1, 300, 1024, 64), (4, 64, 10240, 64),
    (2, 8200, 3072, 64), (4, 8300, 2048, 32), (6, 8190, 3072, 128),
]


@pytest.mark.parametrize("M,N,K,g", SHAPES)
def test_skinny_shapes(pkg, dev, M, N, K, g):
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


@pytest.mark.parametrize("K,g,M,N", [(1024, 64, 16, 48), (2048, 32, 16, 48), (4096, 128, 16, 48),
                                     (3072, 64, 16, 48), (8192, 64, 16, 48), (3072, 64, 4, 8200)])
def test_skinny_dequant_bit_exact(pkg, dev, K, g, M, N):
    """x rows are unit vectors e_k (M per call, over every k): each output is
    one dequantized weight, exact in fp32, so every lane, step, wave and
    nibble position of the route is checked bit for bit against fp16(s*q+b),
    and with s = 1, b = 0 against the unpacked codes.  M = 4, N = 8200 is the
    two-tile block at two blocks per CU with X in LDS."""
    import torch
    _, [(w, s, b)] = o.make_inputs(1, N, K, g, seed=K + g)
    want = rounded_weights_f16(w, s, b, g).T.astype(np.float32)     # [K, N]
    codes = o.unpack_q4(w).T.astype(np.float32)
    tw, ts, tb = to_dev(w, dev), to_dev(s, dev), to_dev(b, dev)
    ones, zeros = to_dev(np.ones_like(s), dev), to_dev(np.zeros_like(b), dev)
    for c in range(K // M):
        ks = np.arange(M) * (K // M) + c          # spread over waves and steps
        x = np.zeros((M, K), dtype=np.float16)
        x[np.arange(M), ks] = 1.0
        tx = to_dev(x, dev)
        y = pkg.matmul_q4_fast_f32(tx, tw, ts, tb, M, K, N, g)
        yq = pkg.matmul_q4_fast_f32(tx, tw, ones, zeros, M, K, N, g)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), want[ks]), c
        assert np.array_equal(yq.cpu().numpy(), codes[ks]), c


# Gated pairs (M, N, K, g).  Above 16 rows at K = 2048 / 3072 only group size
# 32 stays on this route (the mid-M route's LDS does not hold its slabs):
# those cases keep the 2- and 3-step instantiations of 32 activation rows.
PAIR_SHAPES = [(5, 8192, 3072, 64), (8, 200, 3072, 64), (24, 4096, 4096, 64),
               (20, 64, 4096, 64), (24, 96, 3072, 32), (32, 64, 3072, 32)]


@pytest.mark.parametrize("M,N,K,g", PAIR_SHAPES)
@pytest.mark.parametrize("gelu", [False, True])
def test_skinny_gated_pair(pkg, dev, M, N, K, g, gelu):
    import torch
    assert pkg.gemm_route(M, N, K, group_size=g, gated=True) == "small_m"
    x, [(wg, sg, bg), (wu, su, bu)] = o.make_inputs(M, N, K, g, seed=M + N + K + gelu,
                                                    n_weights=2)
    gate = o.matmul_q4_f64(x, wg, sg, bg, g)
    up = o.matmul_q4_f64(x, wu, su, bu, g)
    ref = (o.gelu_tanh_f64(gate) * up) if gelu else o.silu_mul_f64(gate, up)
    fn = pkg.matmul_q4_geglu if gelu else pkg.matmul_q4_silu_mul
    y = fn(to_dev(x, dev), q4w(pkg, wg, sg, bg, K, g, dev), q4w(pkg, wu, su, bu, K, g, dev),
           M, K, N)
    torch.cuda.synchronize()
    assert_parity(y.cpu().numpy(), ref, TOL_GEMM_F16, f"{'geglu' if gelu else 'swiglu'} M={M}")


@pytest.mark.parametrize("M", [6, 12, 23])
def test_skinny_residual_and_bias_gelu(pkg, dev, M):
    """The single-set epilogues on the small-M route: residual add
    (linear + elemAdd, LlamaModel.swift:330-331) and bias + GELU-tanh with an
    fp16 activation (DiTLinear's q4 branch, DiTModel.swift:102-125)."""
    import torch
    N, K, g = 160, 4096, 64
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=300 + M)
    rng = np.random.default_rng(M)
    res = rng.standard_normal((M, N)).astype(np.float16)
    bias = rng.standard_normal(N).astype(np.float32)
    wt = q4w(pkg, w, s, b, K, g, dev)
    proj = o.matmul_q4_f64(x, w, s, b, g)
    y = pkg.matmul_q4_residual(to_dev(x, dev), wt, to_dev(res, dev), M, N)
    yg = pkg.matmul_q4_ex(to_dev(x, dev), wt, M, N, out_dtype=torch.float32,
                          bias=to_dev(bias, dev), epilogue=pkg.SLTX_EPI_GELU_TANH)
    torch.cuda.synchronize()
    want = (res.astype(np.float64) + proj.astype(np.float16).astype(np.float64))
    assert_parity(y.cpu().numpy(), want, TOL_GEMM_F16, f"residual M={M}")
    assert_parity(yg.cpu().numpy(), o.gelu_tanh_f64(proj + bias), TOL_GEMM_F16,
                  f"bias+gelu M={M}")


def test_skinny_in_graph(pkg, dev):
    """The route allocates nothing: it captures into a HIP graph as is, and the
    replays match the eager result."""
    import torch
    M, N, K, g = 6, 512, 3072, 64
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=5)
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
