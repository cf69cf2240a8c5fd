"""GPU parity of the GEMM's persistent launches (q4_gemm.hip, PERSIST): more
output tiles than one block per CU, on the fast path (group size 64,
K % 256 == 0).  One block per CU walks a fixed list of tiles, the copy ring
runs on across tile boundaries (the last three k-tiles of a tile copy the
next tile's first ones), and each finished tile is stored from registers
(D^T accumulators, lanes trading columns with v_permlane32_swap).

Same semantics as every M > 1 route (matmulQ4Fast / matmulQ4FastF32,
Ops.swift:312-381; SwiGLU, LlamaModel.swift:275-277; DiTLinear's bias +
GELU-tanh, DiTModel.swift:102-125): checked against the fp64 oracle on
sampled rows (tests/helpers.py tolerances; gated pairs elementwise against
the fp16-rounded weights), bit for bit through unit-vector
activations (each output one dequantized weight), and across HIP graph
replays.  The shapes give XCDs uneven tile lists (some blocks one tile more
than others), tiles past N and past M, and column counts that are not a
multiple of 8 (element stores).
"""
import numpy as np
import pytest

from helpers import (GATE, TOL_GEMM_BF16, TOL_GEMM_F16, assert_parity, gpu_inputs, host,
                     rounded_weights_f16, to_dev)
from oracle import q4_oracle as o

pytestmark = pytest.mark.gpu


def _tiles(M, N, pair, bm=192):
    """Output tiles at the 192-row tile (the 128-row tile has more): over
    256 means a persistent launch whichever the planner picks."""
    return -(-M // bm) * -(-N // (128 if pair else 256))


@pytest.mark.parametrize("M,N,K", [(1000, 16384, 256), (1000, 12300, 512), (1400, 9000, 768)])
def test_persistent_plain(pkg, dev, M, N, K):
    import torch
    g = 64
    assert _tiles(M, N, False) > 256
    x, [(w, s, b)] = gpu_inputs(M, N, K, g, seed=M + N, dev=dev)
    y = pkg.matmul_q4_fast(x, w, s, b, M, K, N, g)
    y2 = pkg.matmul_q4_fast_f32(x, w, s, b, M, K, N, g)
    torch.cuda.synchronize()
    assert torch.equal(y, y2.half())
    rows = np.array([0, 1, 191, 192, 383, M // 2, M - 2, M - 1])
    ref = o.matmul_q4_f64(host(x)[rows].astype(np.float64), host(w), host(s), host(b), g)
    assert_parity(y2.cpu().numpy()[rows], ref, TOL_GEMM_F16, f"M={M} N={N} K={K}")


@pytest.mark.parametrize("M,N,K,gelu", [(800, 8192, 512, False), (1100, 6000, 256, True)])
def test_persistent_gated_pair(pkg, dev, M, N, K, gelu):
    import torch
    g = 64
    assert _tiles(M, N, True) > 256
    x, [(wg, sg, bg), (wu, su, bu)] = gpu_inputs(M, N, K, g, seed=M + K, dev=dev, n_weights=2)
    fn = pkg.matmul_q4_geglu if gelu else pkg.matmul_q4_silu_mul
    y = fn(x, pkg.Q4Weight(wg, sg, bg, K, g), pkg.Q4Weight(wu, su, bu, K, g), M, K, N)
    torch.cuda.synchronize()
    rows = np.array([0, 63, 64, 191, 192, M // 3, M - 1])
    xs = host(x)[rows].astype(np.float64)
    glu = (lambda a, b: o.gelu_tanh_f64(a) * b) if gelu else o.silu_mul_f64
    # the parity bar against the fp64 oracle ...
    ref = glu(o.matmul_q4_f64(xs, host(wg), host(sg), host(bg), g),
              o.matmul_q4_f64(xs, host(wu), host(su), host(bu), g))
    got = y.cpu().numpy()[rows].astype(np.float64)
    assert o.max_rel_err(got, ref) <= GATE
    # ... and elementwise against the product on the fp16-rounded weights the
    # kernel multiplies by (the weight rounding, compounded in gate x up, is
    # what the oracle check's elementwise allowance would otherwise have to
    # absorb at this short K): fp32 sums, fp16 output rounding, exp2/rcp
    ref_w = glu(xs @ rounded_weights_f16(host(wg), host(sg), host(bg), g).T,
                xs @ rounded_weights_f16(host(wu), host(su), host(bu), g).T)
    ok, worst = o.elementwise_ok(got, ref_w, rtol=1e-3, atol_rms=1e-4)
    assert ok, f"pair M={M} N={N}: {worst:.2f}x the allowance"


@pytest.mark.parametrize("out", ["f32", "bf16"])
def test_persistent_bf16_bias_gelu(pkg, dev, out):
    """DiTLinear's shape of call (bf16 activations, fp32 bias, GELU-tanh) on a
    persistent launch, fp32 and bf16 outputs."""
    import torch
    M, N, K, g = 900, 16384, 512, 64
    assert _tiles(M, N, False) > 256
    x, [(w, s, b)] = gpu_inputs(M, N, K, g, seed=11, dev=dev, x_dtype="bf16")
    bias = np.random.default_rng(12).standard_normal(N).astype(np.float32)
    odt = torch.float32 if out == "f32" else torch.bfloat16
    y = pkg.matmul_q4_ex(x, pkg.Q4Weight(w, s, b, K, g), M, N, out_dtype=odt,
                         bias=to_dev(bias, dev), epilogue=pkg.SLTX_EPI_GELU_TANH)
    torch.cuda.synchronize()
    rows = np.array([0, 191, 192, 500, M - 1])
    pre = o.matmul_q4_f64(o.x_values(host(x)[rows], "bf16"), host(w), host(s), host(b), g) + bias
    assert_parity(y.float().cpu().numpy()[rows], o.gelu_tanh_f64(pre), TOL_GEMM_BF16,
                  f"bf16 bias+gelu {out}")


def test_persistent_residual(pkg, dev):
    """The residual epilogue (linear + elemAdd, LlamaModel.swift:330-331) on a
    persistent launch: half(residual + half(x . W^T))."""
    import torch
    M, N, K, g = 800, 16384, 256, 64
    assert _tiles(M, N, False) > 256
    x, [(w, s, b)] = gpu_inputs(M, N, K, g, seed=13, dev=dev)
    res = np.random.default_rng(14).standard_normal((M, N)).astype(np.float16)
    y = pkg.matmul_q4_residual(x, pkg.Q4Weight(w, s, b, K, g), to_dev(res, dev), M, N)
    torch.cuda.synchronize()
    rows = np.array([0, 200, 383, 384, 600, M - 1])
    proj = o.matmul_q4_f64(host(x)[rows].astype(np.float64), host(w), host(s), host(b), g)
    want = res[rows].astype(np.float64) + proj.astype(np.float16).astype(np.float64)
    assert_parity(y.cpu().numpy()[rows], want, TOL_GEMM_F16, "persistent residual")


def test_persistent_dequant_bit_exact(pkg, dev):
    """x rows are unit vectors e_k: every output is one dequantized weight,
    exact in fp32, so each tile of each block's list (and each k-tile of the
    ring's hand-over between tiles) is checked bit for bit against
    fp16(s*q+b)."""
    import torch
    M, N, K, g = 800, 16384, 512, 64
    assert _tiles(M, N, False) > 256
    _, [(w, s, b)] = gpu_inputs(1, N, K, g, seed=15, dev=dev)
    want = rounded_weights_f16(host(w), host(s), host(b), g).T.astype(np.float32)   # [K, N]
    ks = (np.arange(M) * 7) % K
    xh = np.zeros((M, K), dtype=np.float16)
    xh[np.arange(M), ks] = 1.0
    y = pkg.matmul_q4_fast_f32(to_dev(xh, dev), w, s, b, M, K, N, g)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), want[ks])


def test_persistent_in_graph(pkg, dev):
    """Captured into a HIP graph: every replay, with eager work between them,
    equals the eager result bit for bit."""
    import torch
    M, N, K, g = 1000, 16384, 256, 64
    x, [(w, s, b)] = gpu_inputs(M, N, K, g, seed=16, dev=dev)
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        eager = pkg.matmul_q4_fast(x, w, s, b, M, K, N, g, stream=st)
    st.synchronize()
    out = torch.empty_like(eager)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=st):
        pkg.matmul_q4_fast(x, w, s, b, M, K, N, g, out=out, stream=st)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        other = pkg.matmul_q4_fast(x, w, s, b, M, K, N, g)
        torch.cuda.synchronize()
        assert torch.equal(other, eager)
