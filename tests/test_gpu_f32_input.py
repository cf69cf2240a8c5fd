"""fp32 activations in sltx_matmul_q4_ex: DiTLinear.applyF32in's quantized
branch (DiTModel.swift:102-125) casts x to fp16 with cast_f32_to_f16,
half(clamp(x, -65504, 65504)) (Kernels.swift:816-822), then runs
matmulQ4FastF32 and adds the fp32 bias.  Here the cast happens inside the
GEMM as it stages x (outputs up to 512 wide), or once into a per-stream
buffer before the fp16 routes (wider outputs, where the GEMM's column blocks
would each repeat the cast).

Checked (1) bit for bit against the same call fed the oracle's cast of x as
fp16 where the cast runs once (and to fp32 rounding where it runs inside the
GEMM, whose plan may split K differently), at the LTX
DiT feed-forward shapes (benchmark config 5: M = 6144, hidden 2048, ffn 8192)
with inputs beyond +-65504 and infinities, and (2) against the fp64 oracle
of that cast followed by the dequant matmul, on rows with and without
clamped values, at config 5 and at small and ragged shapes (group sizes 32 /
64 / 128, K not a multiple of 128, split K, M = 1).
"""
import numpy as np
import pytest

from helpers import TOL_GEMM_F16, assert_parity, q4w, to_dev
from oracle import q4_oracle as o

pytestmark = pytest.mark.gpu


def _x_f32(M, K, seed, big_rows=()):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    for r in big_rows:   # values the cast must clamp, and infinities
        cols = rng.choice(K, 6, replace=False)
        x[r, cols] = [1.0e5, -7.0e4, 65519.0, 2.0e9, np.inf, -np.inf]
    return x


@pytest.mark.parametrize("N,K,gelu", [(8192, 2048, True), (2048, 8192, False)])
def test_f32_dit_ffn_config5(pkg, dev, N, K, gelu):
    import torch
    M, g = 6144, 64
    big = (0, 17, 3000, 6143)
    x = _x_f32(M, K, seed=N + K, big_rows=big)
    _, [(w, s, b)] = o.make_inputs(1, N, K, g, seed=K)
    bias = np.random.default_rng(1).standard_normal(N).astype(np.float32)
    wt = q4w(pkg, w, s, b, K, g, dev)
    epi = pkg.SLTX_EPI_GELU_TANH if gelu else pkg.SLTX_EPI_NONE
    tb = to_dev(bias, dev)
    y32 = pkg.matmul_q4_ex(to_dev(x, dev), wt, M, N, out_dtype=torch.float32, bias=tb, epilogue=epi)
    x16 = o.cast_f32_to_f16_ref(x)
    y16 = pkg.matmul_q4_ex(to_dev(x16, dev), wt, M, N, out_dtype=torch.float32, bias=tb,
                           epilogue=epi)
    torch.cuda.synchronize()
    got = y32.cpu().numpy()
    assert np.isfinite(got).all()
    # wide outputs: x is cast once, then the fp16 GEMM runs -- bit for bit
    assert np.array_equal(got, y16.cpu().numpy())
    # the oracle on the rows holding clamped values and on 252 others
    rows = np.array(sorted(set(big) | set(range(5, M, 25))))
    ref = o.matmul_q4_f64(x16[rows], w, s, b, g) + bias
    if gelu:
        ref = o.gelu_tanh_f64(ref)
    for sel, what in ((np.isin(rows, big), "clamped rows"), (~np.isin(rows, big), "other rows")):
        assert_parity(got[rows][sel], ref[sel], TOL_GEMM_F16, f"config 5 N={N} {what}")


def test_f32_in_gemm_cast_config5_rows(pkg, dev):
    """N <= 512: the cast runs inside the GEMM as it stages x (fp32 loads,
    clamp, cast, LDS), here at the config-5 row count and K; against the same
    GEMM fed the cast as fp16 (its plan may split K differently: fp32
    rounding of 2048-term sums, some of +-65504-sized terms) and the oracle."""
    import torch
    M, N, K, g = 6144, 256, 2048, 64
    assert pkg.gemm_route(M, N, K, group_size=g, x_dtype=torch.float32) == "gemm"
    big = (0, 17, 3000, 6143)
    x = _x_f32(M, K, seed=9, big_rows=big)
    _, [(w, s, b)] = o.make_inputs(1, N, K, g, seed=10)
    wt = q4w(pkg, w, s, b, K, g, dev)
    y32 = pkg.matmul_q4_ex(to_dev(x, dev), wt, M, N, out_dtype=torch.float32)
    x16 = o.cast_f32_to_f16_ref(x)
    y16 = pkg.matmul_q4_ex(to_dev(x16, dev), wt, M, N, out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = y32.cpu().numpy()
    ok, worst = o.elementwise_ok(got, y16.cpu().numpy().astype(np.float64), rtol=1e-4,
                                 atol_rms=1e-4)
    assert ok, worst
    rows = np.array(sorted(set(big) | set(range(5, M, 25))))
    ref = o.matmul_q4_f64(x16[rows], w, s, b, g)
    for sel, what in ((np.isin(rows, big), "clamped rows"), (~np.isin(rows, big), "other rows")):
        assert_parity(got[rows][sel], ref[sel], TOL_GEMM_F16, f"in-GEMM cast {what}")


def test_f32_in_graph_without_cast_buffer(pkg, dev):
    """Captured on a stream that never ran the call eagerly, a wide-output
    fp32 call cannot allocate its cast buffer: it runs the in-GEMM cast
    instead, and every replay matches the eager (cast-pass) result to fp32
    rounding and the oracle to the GEMM tolerance."""
    import torch
    M, N, K, g = 300, 1024, 2048, 64
    x = _x_f32(M, K, seed=11, big_rows=(3,))
    _, [(w, s, b)] = o.make_inputs(1, N, K, g, seed=12)
    wt = q4w(pkg, w, s, b, K, g, dev)
    tx = to_dev(x, dev)
    eager = pkg.matmul_q4_ex(tx, wt, M, N, out_dtype=torch.float32)
    torch.cuda.synchronize()
    st = torch.cuda.Stream()
    out = torch.empty(M, N, dtype=torch.float32, device=dev)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=st):
        pkg.matmul_q4_ex(tx, wt, M, N, out=out, stream=st)
    ref = o.matmul_q4_f64(o.cast_f32_to_f16_ref(x), w, s, b, g)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        ok, worst = o.elementwise_ok(got, eager.cpu().numpy().astype(np.float64), rtol=1e-4,
                                     atol_rms=1e-4)
        assert ok, worst
        other = np.arange(M) != 3
        assert_parity(got[other], ref[other], TOL_GEMM_F16, "graph replay, in-GEMM cast")
        assert_parity(got[3:4], ref[3:4], TOL_GEMM_F16, "graph replay, clamped row")


@pytest.mark.parametrize("M,N,K,g", [(1, 256, 2048, 64), (33, 200, 3072, 32), (300, 1000, 1024, 128),
                                     (7, 40, 160, 32), (130, 3072, 8192, 64)])
def test_f32_small_and_ragged(pkg, dev, M, N, K, g):
    import torch
    want = "gemm" if N <= 512 else pkg.gemm_route(M, N, K, group_size=g)
    assert pkg.gemm_route(M, N, K, group_size=g, x_dtype=torch.float32) == want
    x = _x_f32(M, K, seed=M + N, big_rows=(M - 1,))
    _, [(w, s, b)] = o.make_inputs(1, N, K, g, seed=N)
    wt = q4w(pkg, w, s, b, K, g, dev)
    y = pkg.matmul_q4_ex(to_dev(x, dev), wt, M, N, out_dtype=torch.float32)
    yh = pkg.matmul_q4_ex(to_dev(x, dev), wt, M, N, out_dtype=torch.float16)
    torch.cuda.synchronize()
    x16 = o.cast_f32_to_f16_ref(x)
    ref = o.matmul_q4_f64(x16, w, s, b, g)
    got = y.cpu().numpy()
    if M > 1:
        assert_parity(got[:-1], ref[:-1], TOL_GEMM_F16, f"M={M} N={N} K={K} g={g}")
    assert_parity(got[-1:], ref[-1:], TOL_GEMM_F16, f"M={M} clamped row")
    # the fp16 output is the fp32 one rounded once
    assert torch.equal(yh, y.half())


def test_f32_nan_takes_the_lower_bound(pkg, dev):
    """NaN in x is cast as Metal's clamp treats it (fmax returns the non-NaN
    operand): -65504, so the output stays finite and equals the product with
    -65504 in that position."""
    import torch
    M, N, K, g = 40, 64, 256, 64
    x = _x_f32(M, K, seed=3)
    x[5, 7] = np.nan
    x2 = x.copy()
    x2[5, 7] = -65504.0
    _, [(w, s, b)] = o.make_inputs(1, N, K, g, seed=4)
    wt = q4w(pkg, w, s, b, K, g, dev)
    y = pkg.matmul_q4_ex(to_dev(x, dev), wt, M, N, out_dtype=torch.float32)
    y2 = pkg.matmul_q4_ex(to_dev(x2, dev), wt, M, N, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    assert torch.equal(y, y2)
