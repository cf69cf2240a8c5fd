"""GPU parity of the wide-M route (q4_wide.hip: 32 < M <= 256, fp16
activations) through the C ABI: single weight sets and gated pairs, one
block along M (33..128 rows, 2-4 MFMA row tiles) and two (129..256 rows),
unsplit and split over K across blocks (the last block of each output tile
adds the splits' fp32 partial sums; tests/test_gpu_wide_splits.py covers
that hand-over), every group size, the single-set epilogues.

Same semantics as the GEMM (matmulQ4Fast / matmulQ4FastF32, Ops.swift:312-381;
the SwiGLU and GeGLU pairs, LlamaModel.swift:275-277 and
T5Encoder.swift:191-199): the weights are dequantized to fp16 as s*q+b in one
fp16 FMA and multiplied with fp32 accumulation, so the outputs are checked
against the fp64 oracle (tolerances of tests/helpers.py), against the
fp16-rounded weights, and bit for bit through unit vectors.  Row and column
counts that do not fill the last tile, K ranges of one to 80 rounds of 128 k,
and grids from one block to 512 are covered.
"""
import numpy as np
import pytest

from helpers import (TOL_GEMM_BF16, TOL_GEMM_F16, TOL_ROUNDED_W, assert_parity, q4w,
                     rounded_weights_f16, to_dev)
from oracle import q4_oracle as o

pytestmark = pytest.mark.gpu

# (M, N, K, g): one weight set
SHAPES = [
    (33, 5120, 3072, 64), (64, 3072, 3072, 64), (100, 4096, 4096, 128), (128, 3072, 8192, 64),
    (200, 3072, 8192, 64), (256, 500, 2048, 32), (48, 64, 128, 64), (70, 130, 384, 32),
    (129, 1000, 1024, 64), (96, 8192, 3072, 64), (160, 96, 2048, 128), (41, 4100, 1024, 32),
    (200, 5120, 3072, 64), (256, 5101, 2048, 32), (129, 5200, 1024, 64),   # three M-blocks
]


@pytest.mark.parametrize("M,N,K,g", SHAPES)
def test_wide_shapes(pkg, dev, M, N, K, g):
    import torch
    assert pkg.gemm_route(M, N, K, group_size=g) == "wide"
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


@pytest.mark.parametrize("K,g,M,N", [(3072, 64, 128, 200), (1024, 128, 64, 130),
                                     (2048, 32, 96, 64), (8192, 64, 128, 3072)])
def test_wide_dequant_bit_exact(pkg, dev, K, g, M, N):
    """x rows are unit vectors e_k (M per call, over every k): each output is
    one dequantized weight, exact in fp32, so every lane, K-group wave, round,
    split and nibble position of the route is checked bit for bit against
    fp16(s*q+b), and with s = 1, b = 0 against the unpacked codes."""
    import torch
    assert pkg.gemm_route(M, N, K, group_size=g) == "wide"
    _, [(w, s, b)] = o.make_inputs(1, N, K, g, seed=K + g)
    want = rounded_weights_f16(w, s, b, g).T.astype(np.float32)     # [K, N]
    codes = o.unpack_q4(w).T.astype(np.float32)
    tw, ts, tb = to_dev(w, dev), to_dev(s, dev), to_dev(b, dev)
    ones, zeros = to_dev(np.ones_like(s), dev), to_dev(np.zeros_like(b), dev)
    for c in range(-(-K // M)):
        ks = (np.arange(M) * (K // M) + c) % K    # spread over waves, rounds and splits
        x = np.zeros((M, K), dtype=np.float16)
        x[np.arange(M), ks] = 1.0
        tx = to_dev(x, dev)
        y = pkg.matmul_q4_fast_f32(tx, tw, ts, tb, M, K, N, g)
        yq = pkg.matmul_q4_fast_f32(tx, tw, ones, zeros, M, K, N, g)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), want[ks]), c
        assert np.array_equal(yq.cpu().numpy(), codes[ks]), c


@pytest.mark.parametrize("M,N,K,g", [(128, 8192, 3072, 64), (33, 4096, 3072, 64),
                                     (256, 1000, 2048, 32), (64, 10240, 4096, 64),
                                     (96, 70, 1024, 128), (180, 300, 8192, 64)])
@pytest.mark.parametrize("gelu", [False, True])
def test_wide_gated_pair(pkg, dev, M, N, K, g, gelu):
    import torch
    assert pkg.gemm_route(M, N, K, group_size=g, gated=True) == "wide"
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


@pytest.mark.parametrize("M,N,K", [(40, 200, 2048), (128, 3072, 8192), (250, 136, 1024)])
def test_wide_residual_and_bias_gelu(pkg, dev, M, N, K):
    """The single-set epilogues on the wide-M route, unsplit and split:
    residual add (linear + elemAdd, LlamaModel.swift:330-331; also in place) and bias +
    GELU-tanh with an fp16 activation and fp32 / bf16 outputs (DiTLinear's q4
    branch, DiTModel.swift:102-125)."""
    import torch
    g = 64
    assert pkg.gemm_route(M, N, K) == "wide"
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=300 + M)
    rng = np.random.default_rng(M)
    res = rng.standard_normal((M, N)).astype(np.float16)
    bias = rng.standard_normal(N).astype(np.float32)
    wt = q4w(pkg, w, s, b, K, g, dev)
    proj = o.matmul_q4_f64(x, w, s, b, g)
    y = pkg.matmul_q4_residual(to_dev(x, dev), wt, to_dev(res, dev), M, N)
    inplace = to_dev(res, dev)   # out is the residual itself
    pkg.matmul_q4_residual(to_dev(x, dev), wt, inplace, M, N, out=inplace)
    yg = pkg.matmul_q4_ex(to_dev(x, dev), wt, M, N, out_dtype=torch.float32,
                          bias=to_dev(bias, dev), epilogue=pkg.SLTX_EPI_GELU_TANH)
    yb = pkg.matmul_q4_ex(to_dev(x, dev), wt, M, N, out_dtype=torch.bfloat16,
                          bias=to_dev(bias, dev))
    torch.cuda.synchronize()
    want = (res.astype(np.float64) + proj.astype(np.float16).astype(np.float64))
    assert_parity(y.cpu().numpy(), want, TOL_GEMM_F16, f"residual M={M}")
    assert torch.equal(inplace, y)
    assert_parity(yg.cpu().numpy(), o.gelu_tanh_f64(proj + bias), TOL_GEMM_F16,
                  f"bias+gelu M={M}")
    assert_parity(yb.float().cpu().numpy(), proj + bias, TOL_GEMM_BF16, f"bias bf16 M={M}")


@pytest.mark.parametrize("M,N,K", [(128, 8192, 3072), (128, 3072, 8192)])
def test_wide_in_graph(pkg, dev, M, N, K):
    """Captured into a HIP graph after one eager call on the stream (which
    sizes the split-K workspace, N = 3072 x K = 8192 splits K): every replay,
    with eager work between them, matches the eager result."""
    import torch
    g = 64
    assert pkg.gemm_route(M, N, K) == "wide"
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=5)
    args = [to_dev(a, dev) for a in (x, w, s, b)]
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        eager = pkg.matmul_q4_fast(*args, M, K, N, g, stream=st)
    st.synchronize()
    out = torch.empty_like(eager)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=st):
        pkg.matmul_q4_fast(*args, M, K, N, g, out=out, stream=st)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        other = pkg.matmul_q4_fast(*args, M, K, N, g)   # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(other, eager)
