"""GPU parity of the 4-bit MFMA GEMM (M > 1) through the C ABI.

Reference semantics: the quantized GEMM behind matmulQ4Fast / matmulQ4FastF32
(Ops.swift:312-381), the SwiGLU prefill path (LlamaModel.swift:275-277) and the
DiT linear + GELU-tanh (DiTModel.swift:102-125, :953).  The reference's GEMM
itself lives in an external package that is not available, so parity is
against the fp64 oracle (plus a rounded-weight reference that pins the
dequantisation rounding); tolerances are stated in tests/helpers.py.
"""
import numpy as np
import pytest

from helpers import (TOL_GEMM_BF16, TOL_GEMM_F16, TOL_ROUNDED_W, TOL_GEMV, assert_parity,
                     gpu_inputs, host, load_golden, q4w, rounded_weights_bf16,
                     rounded_weights_f16, to_dev)
from oracle import q4_oracle as o

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["gemm_m3_n96_k256_g64", "gemm_m37_n160_k384_g64"])
def test_golden_gemm(pkg, dev, name):
    import torch
    t, meta = load_golden(name)
    M, N, K, g = (int(meta[k]) for k in ("M", "N", "K", "group_size"))
    args = [to_dev(t[k], dev) for k in ("x", "proj.weight", "proj.scales", "proj.biases")]
    y16 = pkg.matmul_q4_fast(*args, M, K, N, g)
    y32 = pkg.matmul_q4_fast_f32(*args, M, K, N, g)
    ymq = pkg.matmul_q4(*args, M, K, N, g)  # matmulQ4 with M > 1 routes to the GEMM
    torch.cuda.synchronize()
    assert_parity(y16.cpu().numpy(), t["y_f64"], TOL_GEMM_F16, name)
    assert_parity(y32.cpu().numpy(), t["y_f64"], TOL_GEMM_F16, name + " f32")
    assert torch.equal(ymq, y16)
    assert torch.equal(y32.half(), y16)


def test_golden_swiglu_gemm(pkg, dev):
    import torch
    t, meta = load_golden("swiglu_m5_n80_k256_g64")
    M, N, K, g = (int(meta[k]) for k in ("M", "N", "K", "group_size"))
    gate = q4w(pkg, t["gate_proj.weight"], t["gate_proj.scales"], t["gate_proj.biases"], K, g, dev)
    up = q4w(pkg, t["up_proj.weight"], t["up_proj.scales"], t["up_proj.biases"], K, g, dev)
    y = pkg.matmul_q4_silu_mul(to_dev(t["x"], dev), gate, up, M, K, N)
    torch.cuda.synchronize()
    assert_parity(y.cpu().numpy(), t["y_f64"], TOL_GEMM_F16, "swiglu gemm")


def test_golden_dit_bf16_gelu(pkg, dev):
    import torch
    t, meta = load_golden("dit_m9_n64_k128_g64_bf16_gelu")
    M, N, K, g = (int(meta[k]) for k in ("M", "N", "K", "group_size"))
    x = to_dev(t["x"], dev).view(torch.bfloat16)
    w = q4w(pkg, t["proj.weight"], t["proj.scales"], t["proj.biases"], K, g, dev)
    bias = to_dev(t["bias"], dev)
    y = pkg.matmul_q4_ex(x, w, M, N, out_dtype=torch.float32, bias=bias,
                         epilogue=pkg.SLTX_EPI_GELU_TANH)
    torch.cuda.synchronize()
    pre = t["y_pre_f64"]
    rms = float(np.sqrt(np.mean(pre * pre)))
    err = np.abs(y.cpu().numpy() - t["y_f64"])
    assert np.max(err) <= 1.2e-2 * rms, np.max(err) / rms
    assert o.max_rel_err(y.cpu().numpy(), t["y_f64"]) <= 1e-2


# (M, N, K, g): partial M/N tiles, K tails (K % 64 == 32), every group size.
SHAPES = [
    (2, 64, 256, 64), (3, 100, 3072, 64), (64, 128, 512, 32), (127, 256, 1024, 128),
    (128, 128, 128, 64), (129, 130, 256, 64), (300, 1000, 768, 64), (17, 96, 96, 32),
    (40, 72, 160, 32), (256, 512, 2048, 64),
    # M = 1 through the GEMM (the _fast entry points never route to the GEMV)
    (1, 300, 3072, 64), (1, 64, 96, 32),
    # K = 32: one partial k-tile
    (5, 40, 32, 32), (70, 300, 32, 32),
]


@pytest.mark.parametrize("M,N,K,g", SHAPES)
def test_gemm_shapes(pkg, dev, M, N, K, g):
    import torch
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=M * 31 + N + K)
    y = pkg.matmul_q4_fast_f32(to_dev(x, dev), to_dev(w, dev), to_dev(s, dev), to_dev(b, dev), M,
                               K, N, g)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    assert_parity(y, o.matmul_q4_f64(x, w, s, b, g), TOL_GEMM_F16, f"M={M} N={N} K={K}")
    # weights rounded to fp16 exactly as the kernel does: fp32 accumulation only
    ref_r = x.astype(np.float64) @ rounded_weights_f16(w, s, b, g).T
    ok, worst = o.elementwise_ok(y, ref_r, **TOL_ROUNDED_W)
    assert ok, worst


@pytest.mark.parametrize("K,g", [(256, 64), (96, 32), (512, 128)])
def test_gemm_dequant_bit_exact_identity(pkg, dev, K, g):
    """A = I_K: row k of the output is column k of the dequantized weights, so
    the kernel's fp16 (or bf16) dequantisation is checked bit for bit."""
    import torch
    N = 192
    x, [(w, s, b)] = o.make_inputs(1, N, K, g, seed=K)
    eye16 = np.eye(K, dtype=np.float16)
    y = pkg.matmul_q4_fast_f32(to_dev(eye16, dev), to_dev(w, dev), to_dev(s, dev), to_dev(b, dev),
                               K, K, N, g)
    torch.cuda.synchronize()
    want = rounded_weights_f16(w, s, b, g).T.astype(np.float32)
    assert np.array_equal(y.cpu().numpy(), want)
    eyeb = to_dev(o.f32_to_bf16_bits(np.eye(K, dtype=np.float32)), dev).view(torch.bfloat16)
    yb = pkg.matmul_q4_ex(eyeb, q4w(pkg, w, s, b, K, g, dev), K, N, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert np.array_equal(yb.cpu().numpy(), rounded_weights_bf16(w, s, b, g).T.astype(np.float32))
    # and the unpacked codes themselves: s = 1, b = 0
    ones, zeros = np.ones_like(s), np.zeros_like(b)
    yq = pkg.matmul_q4_fast_f32(to_dev(eye16, dev), to_dev(w, dev), to_dev(ones, dev),
                                to_dev(zeros, dev), K, K, N, g)
    torch.cuda.synchronize()
    assert np.array_equal(yq.cpu().numpy().T.astype(np.int64), o.unpack_q4(w).astype(np.int64))


def test_gemm_rows_match_gemv(pkg, dev):
    """Row independence: each GEMM row equals the GEMV of that row of x."""
    import torch
    M, N, K, g = 9, 512, 3072, 64
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=77)
    tw, ts, tb = to_dev(w, dev), to_dev(s, dev), to_dev(b, dev)
    tx = to_dev(x, dev)
    yg = pkg.matmul_q4_fast_f32(tx, tw, ts, tb, M, K, N, g).cpu().numpy()
    for m in range(M):
        yv = pkg.matmul_q4(tx[m:m + 1].contiguous(), tw, ts, tb, 1, K, N, g)
        torch.cuda.synchronize()
        ok, worst = o.elementwise_ok(yv.cpu().numpy()[0], yg[m], **TOL_GEMM_F16)
        assert ok, (m, worst)


@pytest.mark.parametrize("M,N,K", [(2, 64, 192), (37, 200, 256), (130, 96, 3072)])
def test_swiglu_gemm_shapes(pkg, dev, M, N, K):
    import torch
    g = 64
    x, [(wg, sg, bg), (wu, su, bu)] = o.make_inputs(M, N, K, g, seed=M + N + K, n_weights=2)
    ref = o.silu_mul_f64(o.matmul_q4_f64(x, wg, sg, bg, g), o.matmul_q4_f64(x, wu, su, bu, g))
    y = pkg.matmul_q4_silu_mul(to_dev(x, dev), q4w(pkg, wg, sg, bg, K, g, dev),
                               q4w(pkg, wu, su, bu, K, g, dev), M, K, N)
    torch.cuda.synchronize()
    assert_parity(y.cpu().numpy(), ref, TOL_GEMM_F16, f"swiglu M={M}")


@pytest.mark.parametrize("out", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("xdt", ["f16", "bf16"])
@pytest.mark.parametrize("epi", [0, 2])
def test_gemm_ex_dtypes_bias_gelu(pkg, dev, out, xdt, epi):
    import torch
    M, N, K, g = 70, 136, 512, 64
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=5, x_dtype=xdt)
    bias = (np.random.default_rng(6).standard_normal(N) * 0.5).astype(np.float32)
    pre = o.matmul_q4_f64(o.x_values(x, xdt), w, s, b, g) + bias
    ref = o.gelu_tanh_f64(pre) if epi == 2 else pre
    tx = to_dev(x, dev)
    if xdt == "bf16":
        tx = tx.view(torch.bfloat16)
    odt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[out]
    y = pkg.matmul_q4_ex(tx, q4w(pkg, w, s, b, K, g, dev), M, N, out_dtype=odt,
                         bias=to_dev(bias, dev), epilogue=epi)
    torch.cuda.synchronize()
    y = y.float().cpu().numpy()
    rms = float(np.sqrt(np.mean(pre * pre)))
    tol_w = 1.2e-2 if xdt == "bf16" else 3e-3
    tol_o = {"f16": 1e-3, "bf16": 4e-3, "f32": 1e-5}[out]
    allow = tol_o * np.abs(ref) + tol_w * rms
    assert np.all(np.abs(y - ref) <= allow), float(np.max(np.abs(y - ref) / allow))
    assert o.max_rel_err(y, ref) <= 1e-2


# ---- benchmark configs at full size (sampled rows against the oracle) ----

def _sample_check(y, x, w, s, b, g, rows_m, tol, what, x_dtype="f16"):
    xs = host(x)[rows_m]
    ref = o.matmul_q4_f64(o.x_values(xs, x_dtype), host(w), host(s), host(b), g)
    return assert_parity(y.float().cpu().numpy()[rows_m], ref, tol, what)


def test_prefill_gate_up_swiglu_m750(pkg, dev):
    """Benchmark config 3: X [750, 3072] x gate/up [8192 x 3072], fused SiLU x up."""
    import torch
    M, N, K, g = 750, 8192, 3072, 64
    x, [(wg, sg, bg), (wu, su, bu)] = gpu_inputs(M, N, K, g, seed=3, dev=dev, n_weights=2)
    y = pkg.matmul_q4_silu_mul(x, pkg.Q4Weight(wg, sg, bg, K, g), pkg.Q4Weight(wu, su, bu, K, g),
                               M, K, N)
    torch.cuda.synchronize()
    rows = np.array([0, 1, 127, 128, 333, 640, 748, 749])
    xs = host(x)[rows].astype(np.float64)
    ref = o.silu_mul_f64(o.matmul_q4_f64(xs, host(wg), host(sg), host(bg), g),
                         o.matmul_q4_f64(xs, host(wu), host(su), host(bu), g))
    assert_parity(y.cpu().numpy()[rows], ref, TOL_GEMM_F16, "prefill gate/up")


def test_prefill_down_m750(pkg, dev):
    """Benchmark config 3: X [750, 8192] x down [3072 x 8192], fp16 out."""
    import torch
    M, N, K, g = 750, 3072, 8192, 64
    x, [(w, s, b)] = gpu_inputs(M, N, K, g, seed=4, dev=dev)
    y = pkg.matmul_q4_fast(x, w, s, b, M, K, N, g)
    y2 = pkg.matmul_q4_fast(x, w, s, b, M, K, N, g)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    _sample_check(y, x, w, s, b, g, np.array([0, 5, 128, 511, 749]), TOL_GEMM_F16, "prefill down")


def test_lm_head_m750(pkg, dev):
    """Benchmark config 4b: X [750, 3072] x lm_head [128256 x 3072]."""
    import torch
    M, N, K, g = 750, 128256, 3072, 64
    x, [(w, s, b)] = gpu_inputs(M, N, K, g, seed=5, dev=dev)
    y = pkg.matmul_q4_fast(x, w, s, b, M, K, N, g)
    torch.cuda.synchronize()
    rows_m = np.array([0, 300, 749])
    cols = np.sort(np.random.default_rng(8).choice(N, size=4096, replace=False))
    ref = o.matmul_q4_f64(host(x)[rows_m].astype(np.float64), host(w)[cols], host(s)[cols],
                          host(b)[cols], g)
    assert_parity(y.cpu().numpy()[rows_m][:, cols], ref, TOL_GEMM_F16, "lm_head 750")


def test_dit_ffn_m6144_bf16(pkg, dev):
    """Benchmark config 5: bf16 X [6144, 2048] x up [8192 x 2048] -> GELU-tanh ->
    down [2048 x 8192], fp32 out (DiTModel.swift:930-956 dataflow)."""
    import torch
    M, K1, N1, g = 6144, 2048, 8192, 64
    x, [(wu, su, bu)] = gpu_inputs(M, N1, K1, g, seed=6, dev=dev, x_dtype="bf16")
    _, [(wd, sd, bd)] = gpu_inputs(1, K1, N1, g, seed=7, dev=dev)
    h = pkg.matmul_q4_ex(x, pkg.Q4Weight(wu, su, bu, K1, g), M, N1, out_dtype=torch.bfloat16,
                         epilogue=pkg.SLTX_EPI_GELU_TANH)
    y = pkg.matmul_q4_ex(h, pkg.Q4Weight(wd, sd, bd, N1, g), M, K1, out_dtype=torch.float32)
    torch.cuda.synchronize()
    rows = np.array([0, 1, 4095, 6143])
    xr = o.x_values(host(x)[rows], "bf16")
    pre = o.matmul_q4_f64(xr, host(wu), host(su), host(bu), g)
    href = o.gelu_tanh_f64(pre)
    hk = o.x_values(host(h)[rows], "bf16")
    rms = float(np.sqrt(np.mean(pre * pre)))
    # bf16 weights (2^-9 per product) and the bf16 store of h (half ulp 2^-9)
    allow = 4e-3 * np.abs(href) + 1.2e-2 * rms
    assert np.all(np.abs(hk - href) <= allow), float(np.max(np.abs(hk - href) / allow))
    # second GEMM checked against the oracle on the kernel's own bf16 h
    ref = o.matmul_q4_f64(hk, host(wd), host(sd), host(bd), g)
    assert_parity(y.cpu().numpy()[rows], ref, TOL_GEMM_BF16, "dit down")


# ---- split-K: few output tiles, long K (the kernel splits K and reduces the
# fp32 partials in split order, then applies the epilogue) ----

@pytest.mark.parametrize("M,N,K,xdt,epi,out", [
    (40, 300, 4096, "f16", 2, "f16"),      # 2 tiles x 8 splits, bias + GELU
    (130, 200, 8192, "bf16", 0, "f32"),    # bf16 activations, fp32 out
    (7, 96, 2048, "f16", 0, "f16"),
])
def test_gemm_split_k(pkg, dev, M, N, K, xdt, epi, out):
    import torch
    g = 64
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=M + K, x_dtype=xdt)
    bias = (np.random.default_rng(3).standard_normal(N) * 0.5).astype(np.float32)
    pre = o.matmul_q4_f64(o.x_values(x, xdt), w, s, b, g) + bias
    ref = o.gelu_tanh_f64(pre) if epi == 2 else pre
    tx = to_dev(x, dev)
    if xdt == "bf16":
        tx = tx.view(torch.bfloat16)
    odt = {"f16": torch.float16, "f32": torch.float32}[out]
    qw = q4w(pkg, w, s, b, K, g, dev)
    y = pkg.matmul_q4_ex(tx, qw, M, N, out_dtype=odt, bias=to_dev(bias, dev), epilogue=epi)
    y2 = pkg.matmul_q4_ex(tx, qw, M, N, out_dtype=odt, bias=to_dev(bias, dev), epilogue=epi)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)  # the split reduction is ordered: deterministic
    y = y.float().cpu().numpy()
    rms = float(np.sqrt(np.mean(pre * pre)))
    tol_w = 1.2e-2 if xdt == "bf16" else 3e-3
    tol_o = {"f16": 1e-3, "f32": 1e-5}[out]
    allow = tol_o * np.abs(ref) + tol_w * rms
    assert np.all(np.abs(y - ref) <= allow), float(np.max(np.abs(y - ref) / allow))


@pytest.mark.parametrize("M,N,K", [(64, 256, 4096), (3, 128, 8192)])
def test_swiglu_gemm_split_k(pkg, dev, M, N, K):
    import torch
    g = 64
    x, [(wg, sg, bg), (wu, su, bu)] = o.make_inputs(M, N, K, g, seed=N + K, n_weights=2)
    ref = o.silu_mul_f64(o.matmul_q4_f64(x, wg, sg, bg, g), o.matmul_q4_f64(x, wu, su, bu, g))
    y = pkg.matmul_q4_silu_mul(to_dev(x, dev), q4w(pkg, wg, sg, bg, K, g, dev),
                               q4w(pkg, wu, su, bu, K, g, dev), M, K, N)
    torch.cuda.synchronize()
    assert_parity(y.cpu().numpy(), ref, TOL_GEMM_F16, f"swiglu split M={M}")


def test_split_k_under_graph_capture(pkg, dev):
    """A split-K GEMM captured in a graph (workspace allocated by an eager call
    first) replays to the eager result; a fresh stream captured cold runs
    unsplit and still matches."""
    import torch
    M, N, K, g = 16, 256, 4096, 64
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=12)
    tx, qw = to_dev(x, dev), q4w(pkg, w, s, b, K, g, dev)
    ref = pkg.matmul_q4_fast_f32(tx, qw.weight, qw.scales, qw.biases, M, K, N, g)
    torch.cuda.synchronize()
    for warm in (True, False):
        out = torch.empty(M, N, device=dev, dtype=torch.float32)
        st = torch.cuda.Stream()
        if warm:
            with torch.cuda.stream(st):
                pkg.matmul_q4_fast_f32(tx, qw.weight, qw.scales, qw.biases, M, K, N, g, out=out,
                                       stream=st)
            st.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=st):
            pkg.matmul_q4_fast_f32(tx, qw.weight, qw.scales, qw.biases, M, K, N, g, out=out)
        for _ in range(3):
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            ok, worst = o.elementwise_ok(out.cpu().numpy(), ref.cpu().numpy().astype(np.float64),
                                         rtol=1e-5, atol_rms=1e-5)
            assert ok, (warm, worst)


@pytest.mark.parametrize("kind", ["plain", "silu", "residual", "f32_bias_gelu"])
@pytest.mark.parametrize("M,N,K", [(33, 256, 512), (750, 3072, 8192)])
def test_unaligned_outputs_match_aligned(pkg, dev, kind, M, N, K):
    """Outputs (and the residual input) 2 bytes (fp16) or 4 bytes (fp32) off a
    16-byte boundary take the per-element store path of the staged epilogue
    (and of the split-K reduction at M=750, K=8192); the values must be
    bit-identical to the aligned run's."""
    import torch
    x, [(w, s, b), (w2, s2, b2)] = gpu_inputs(M, N, K, 64, seed=M + K, dev=dev, n_weights=2)
    W = pkg.Q4Weight(w, s, b, K, 64)
    W2 = pkg.Q4Weight(w2, s2, b2, K, 64)
    f32 = kind == "f32_bias_gelu"
    dt = torch.float32 if f32 else torch.float16
    res_a = (torch.randn(M, N, device=dev) * 4).half()
    res_buf = torch.empty(M * N + 1, device=dev, dtype=torch.float16)
    res_u = res_buf[1:].view(M, N)
    res_u.copy_(res_a)
    bias = torch.randn(N, device=dev)

    def run(out, res):
        if kind == "plain":
            return pkg.linear(x, W, M, K, N, fast=True, out=out)
        if kind == "silu":
            return pkg.matmul_q4_silu_mul(x, W, W2, M, K, N, out=out)
        if kind == "residual":
            return pkg.matmul_q4_residual(x, W, res, M, N, out=out)
        return pkg.matmul_q4_ex(x, W, M, N, out_dtype=torch.float32, bias=bias,
                                epilogue=pkg.SLTX_EPI_GELU_TANH, out=out)

    aligned = run(torch.empty(M, N, device=dev, dtype=dt), res_a)
    buf = torch.empty(M * N + 1, device=dev, dtype=dt)
    unaligned = run(buf[1:].view(M, N), res_u)
    torch.cuda.synchronize()
    assert unaligned.data_ptr() % 16 != 0
    assert torch.equal(aligned, unaligned), kind


@pytest.mark.parametrize("kind", ["f16", "silu", "bf16"])
def test_scales_biases_at_2_byte_offset(pkg, dev, kind):
    """Scales and biases 2 bytes off a 4-byte boundary (allowed: 2-byte
    alignment) cannot move as dword pairs, so the launcher routes them to the
    generic kernel; the values must match the aligned run and the oracle."""
    import torch
    M, N, K, g = 70, 320, 1024, 64
    x, sets = gpu_inputs(M, N, K, g, seed=17, dev=dev, n_weights=2,
                         x_dtype="bf16" if kind == "bf16" else "f16")

    def shifted(t):
        buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=dev)
        buf[1:].copy_(t.reshape(-1))
        v = buf[1:].view(t.shape)
        assert v.data_ptr() % 4 == 2
        return v

    Wa = [pkg.Q4Weight(w, s, b, K, g) for w, s, b in sets]
    Wu = [pkg.Q4Weight(w, shifted(s), shifted(b), K, g) for w, s, b in sets]

    def run(W):
        if kind == "silu":
            return pkg.matmul_q4_silu_mul(x, W[0], W[1], M, K, N)
        if kind == "bf16":
            return pkg.matmul_q4_ex(x, W[0], M, N, out_dtype=torch.float32)
        return pkg.linear(x, W[0], M, K, N, fast=True)

    ya, yu = run(Wa), run(Wu)
    torch.cuda.synchronize()
    hs = [(host(w), host(s), host(b)) for w, s, b in sets]
    xh = host(x)
    if kind == "bf16":
        ref = o.matmul_q4_f64(o.bf16_bits_to_f32(xh), *hs[0], g)
        tol = TOL_GEMM_BF16
    elif kind == "silu":
        ref = o.silu_mul_f64(o.matmul_q4_f64(xh, *hs[0], g), o.matmul_q4_f64(xh, *hs[1], g))
        tol = TOL_GEMM_F16
    else:
        ref = o.matmul_q4_f64(xh, *hs[0], g)
        tol = TOL_GEMM_F16
    assert_parity(yu.float().cpu().numpy(), ref, tol, f"2-byte-offset scales {kind}")
    assert_parity(ya.float().cpu().numpy(), ref, tol, f"aligned scales {kind}")
    ok, worst = o.elementwise_ok(yu.float().cpu().numpy(), ya.float().cpu().numpy().astype(np.float64),
                                 rtol=1e-3, atol_rms=1e-3)
    assert ok, worst


def test_release_workspace(pkg, dev):
    """A split-K GEMM allocates the stream's workspace; releasing it (after
    the queued work) and calling again allocates a new one with identical
    results.  Releasing a stream that has none is a no-op."""
    import torch
    M, N, K = 750, 3072, 8192
    x, [(w, s, b)] = gpu_inputs(M, N, K, 64, seed=5, dev=dev)
    st = torch.cuda.Stream()
    pkg.release_workspace(st)   # none yet
    with torch.cuda.stream(st):
        y1 = pkg.matmul_q4_fast(x, w, s, b, M, K, N, 64, stream=st)
    pkg.release_workspace(st)
    with torch.cuda.stream(st):
        y2 = pkg.matmul_q4_fast(x, w, s, b, M, K, N, 64, stream=st)
    st.synchronize()
    assert torch.equal(y1, y2)
    pkg.release_workspace(st)
    pkg.release_workspace(st)
