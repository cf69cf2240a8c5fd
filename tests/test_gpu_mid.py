"""GPU parity of the mid-M route (q4_mid.hip: 16 < M <= 32, and 8 < M <= 16
for one weight set of 4096..16384 rows; fp16 activations) through the C ABI:
gated pairs at K = 2048 / 3072 (32 gate + 32 up rows per block, group sizes
64 and 128) and single weight sets at K = 2048, 3072, 4096, 8192, 10240 (32
rows per block; the weight groups of 1024 k in two LDS slots, refilled as
the groups are used).

Same semantics as the GEMM (matmulQ4Fast / matmulQ4FastF32, Ops.swift:312-381;
the SwiGLU and GeGLU pairs, LlamaModel.swift:275-277 and
T5Encoder.swift:191-199): the weights are dequantized to fp16 as s*q+b in one
fp16 FMA and multiplied with fp32 accumulation, so the outputs are checked
against the fp64 oracle (tolerances of tests/helpers.py), against the
fp16-rounded weights, and bit for bit through unit vectors.  The shapes cover
every built weight-group count, the X ring's wrap-around and
the spare copies past the end, a last block with fewer than 32 rows, grids
from one block to 256, and every group size.
"""
import numpy as np
import pytest

from helpers import (TOL_GEMM_BF16, TOL_GEMM_F16, TOL_ROUNDED_W, assert_parity, q4w, rounded_weights_f16,
                     to_dev)
from oracle import q4_oracle as o

pytestmark = pytest.mark.gpu

# (M, N, K, g)
SHAPES = [
    (17, 5120, 2048, 64), (32, 5150, 3072, 128), (24, 6000, 2048, 128), (20, 5184, 3072, 64),
    (31, 8160, 3072, 64), (29, 5130, 2048, 64), (32, 20, 3072, 32), (18, 100, 2048, 32),
    (25, 3072, 3072, 64), (32, 8192, 3072, 32), (12, 5120, 3072, 64), (9, 4100, 2048, 128),
    (16, 16384, 2048, 32), (28, 4096, 4096, 64), (32, 3072, 8192, 64), (17, 4096, 10240, 128),
    (26, 4096, 4096, 32), (24, 100, 8192, 128), (29, 90, 10240, 64), (31, 4096, 4096, 128),
    (17, 64, 2048, 32),
]


@pytest.mark.parametrize("M,N,K,g", SHAPES)
def test_mid_shapes(pkg, dev, M, N, K, g):
    import torch
    assert pkg.gemm_route(M, N, K, group_size=g) == "mid"
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


@pytest.mark.parametrize("K,g,M,N", [(3072, 64, 32, 5120), (2048, 128, 24, 5150), (3072, 32, 17, 70), (8192, 64, 20, 96)])
def test_mid_dequant_bit_exact(pkg, dev, K, g, M, N):
    """x rows are unit vectors e_k (M per call, over every k): each output is
    one dequantized weight, exact in fp32, so every lane, k-step, K-group,
    round and nibble position of the route is checked bit for bit against
    fp16(s*q+b), and with s = 1, b = 0 against the unpacked codes."""
    import torch
    assert pkg.gemm_route(M, N, K, group_size=g) == "mid"
    _, [(w, s, b)] = o.make_inputs(1, N, K, g, seed=K + g)
    want = rounded_weights_f16(w, s, b, g).T.astype(np.float32)     # [K, N]
    codes = o.unpack_q4(w).T.astype(np.float32)
    tw, ts, tb = to_dev(w, dev), to_dev(s, dev), to_dev(b, dev)
    ones, zeros = to_dev(np.ones_like(s), dev), to_dev(np.zeros_like(b), dev)
    for c in range(-(-K // M)):
        ks = (np.arange(M) * (K // M) + c) % K    # spread over K-groups and rounds
        x = np.zeros((M, K), dtype=np.float16)
        x[np.arange(M), ks] = 1.0
        tx = to_dev(x, dev)
        y = pkg.matmul_q4_fast_f32(tx, tw, ts, tb, M, K, N, g)
        yq = pkg.matmul_q4_fast_f32(tx, tw, ones, zeros, M, K, N, g)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), want[ks]), c
        assert np.array_equal(yq.cpu().numpy(), codes[ks]), c


@pytest.mark.parametrize("M,N,K,g", [(32, 8192, 3072, 64), (17, 200, 3072, 64),
                                     (24, 10240, 2048, 64), (31, 40, 2048, 128),
                                     (32, 10240, 4096, 64), (27, 300, 4096, 128),
                                     (32, 8192, 2048, 32), (19, 72, 2048, 32)])
@pytest.mark.parametrize("gelu", [False, True])
def test_mid_gated_pair(pkg, dev, M, N, K, g, gelu):
    import torch
    assert pkg.gemm_route(M, N, K, group_size=g, gated=True) == "mid"
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


@pytest.mark.parametrize("M", [17, 32])
def test_mid_residual_and_bias_gelu(pkg, dev, M):
    """The single-set epilogues on the mid-M route: residual add
    (linear + elemAdd, LlamaModel.swift:330-331) and bias + GELU-tanh with an
    fp16 activation and bf16 / fp32 outputs (DiTLinear's q4 branch,
    DiTModel.swift:102-125)."""
    import torch
    N, K, g = 200, 2048, 64
    assert pkg.gemm_route(M, N, K) == "mid"
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=300 + M)
    rng = np.random.default_rng(M)
    res = rng.standard_normal((M, N)).astype(np.float16)
    bias = rng.standard_normal(N).astype(np.float32)
    wt = q4w(pkg, w, s, b, K, g, dev)
    proj = o.matmul_q4_f64(x, w, s, b, g)
    y = pkg.matmul_q4_residual(to_dev(x, dev), wt, to_dev(res, dev), M, N)
    yg = pkg.matmul_q4_ex(to_dev(x, dev), wt, M, N, out_dtype=torch.float32,
                          bias=to_dev(bias, dev), epilogue=pkg.SLTX_EPI_GELU_TANH)
    yb = pkg.matmul_q4_ex(to_dev(x, dev), wt, M, N, out_dtype=torch.bfloat16,
                          bias=to_dev(bias, dev))
    torch.cuda.synchronize()
    want = (res.astype(np.float64) + proj.astype(np.float16).astype(np.float64))
    assert_parity(y.cpu().numpy(), want, TOL_GEMM_F16, f"residual M={M}")
    assert_parity(yg.cpu().numpy(), o.gelu_tanh_f64(proj + bias), TOL_GEMM_F16,
                  f"bias+gelu M={M}")
    assert_parity(yb.float().cpu().numpy(), proj + bias, TOL_GEMM_BF16, f"bias bf16 M={M}")


def test_mid_in_graph(pkg, dev):
    """The route allocates nothing: it captures into a HIP graph as is, and the
    replays match the eager result."""
    import torch
    M, N, K, g = 24, 5120, 3072, 64
    assert pkg.gemm_route(M, N, K) == "mid"
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


def test_mid_declines_misaligned_scales(pkg, dev):
    """The route copies scales and biases as 16-byte pieces; with them at a
    2-byte offset (the C ABI accepts 2-byte alignment) the launch takes the
    GEMM's generic path instead and gives the same products, against the
    oracle.  An x that is not 16-byte aligned is rejected by the C ABI."""
    import torch
    M, N, K, g = 24, 5120, 3072, 64
    assert pkg.gemm_route(M, N, K) == "mid"
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=77)
    tx, tw = to_dev(x, dev), to_dev(w, dev)
    ts, tb = to_dev(s, dev), to_dev(b, dev)
    views = []
    for t in (ts, tb):
        buf = torch.empty(t.numel() + 8, dtype=t.dtype, device=dev)
        v = buf[1:1 + t.numel()].view(t.shape)   # 2 bytes past a 16-byte boundary
        v.copy_(t)
        assert v.data_ptr() % 16 == 2
        views.append(v)
    y_al = pkg.matmul_q4_fast_f32(tx, tw, ts, tb, M, K, N, g)
    y_mis = pkg.matmul_q4_fast_f32(tx, tw, views[0], views[1], M, K, N, g)
    torch.cuda.synchronize()
    ref = o.matmul_q4_f64(x, w, s, b, g)
    assert_parity(y_al.cpu().numpy(), ref, TOL_GEMM_F16, "aligned")
    assert_parity(y_mis.cpu().numpy(), ref, TOL_GEMM_F16, "scales and biases at +2 bytes")
    xbuf = torch.empty(M * K + 8, dtype=torch.float16, device=dev)
    with pytest.raises(pkg.SltxError):
        pkg.matmul_q4_fast_f32(xbuf[1:1 + M * K].view(M, K), tw, ts, tb, M, K, N, g)
