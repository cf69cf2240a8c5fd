"""GPU parity of the 4-bit GEMV (M == 1) through the C ABI.

Reference semantics: matmul_q4 (Kernels.swift:444-620) via matmulQ4
(Ops.swift:285-305); fused SwiGLU replaces linear(gate)/linear(up)/siluMul
(LlamaModel.swift:327-329).  Tolerances are stated in tests/helpers.py.
"""
import numpy as np
import pytest

from helpers import (GATE, TOL_GEMV, assert_parity, gpu_inputs, host, load_golden, q4w,
                     to_dev)
from oracle import q4_oracle as o

pytestmark = pytest.mark.gpu

GEMV_GOLDEN = ["gemv_n64_k128_g64", "gemv_n128_k3072_g64", "gemv_n96_k256_g32",
               "gemv_n64_k512_g128", "gemv_n50_k160_g32"]


@pytest.mark.parametrize("name", GEMV_GOLDEN)
def test_golden_gemv(pkg, dev, name):
    import torch
    t, meta = load_golden(name)
    N, K, g = int(meta["N"]), int(meta["K"]), int(meta["group_size"])
    y = pkg.matmul_q4(to_dev(t["x"], dev), to_dev(t["proj.weight"], dev),
                      to_dev(t["proj.scales"], dev), to_dev(t["proj.biases"], dev), 1, K, N, g)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    assert_parity(y, t["y_f64"], TOL_GEMV, name)
    # within 2 fp16 ulp of the emulation of the reference's own summation order
    emu = t["y_emu"].astype(np.float64)
    ulp = np.spacing(np.abs(emu).astype(np.float16)).astype(np.float64)
    # absolute slack: the fp32 accumulation error (~1e-5) dwarfs an fp16 ulp near 0
    assert np.all(np.abs(y.astype(np.float64) - emu) <= 2 * ulp + 2e-4)


# (N, K, g): every lanes-per-row / chunks-per-lane specialisation the
# dispatcher can pick, the generic fallback, odd row counts, all group sizes.
SHAPES = [
    (1, 3072, 64), (7, 3072, 64), (100, 512, 64), (257, 1024, 32), (1000, 2048, 128),
    (3072, 3072, 64), (1024, 3072, 64), (333, 4096, 64), (3072, 8192, 64), (96, 10240, 64),
    (64, 14336, 128), (40, 16384, 64), (200, 6144, 32), (130, 1536, 64), (70, 7168, 64),
    (33, 3584, 64), (9, 96, 32), (11, 160, 32), (5, 2080, 32), (17, 224, 32),
    # two row-iterations per wave with 8 chunks per lane (the smallest block cap)
    (8200, 16384, 64),
    # K = 32: one chunk per row
    (3, 32, 32), (500, 32, 32),
    # generic kernel over several 512-chunk segments of x (Llama-70B's down K = 28672)
    (40, 32000, 64), (7, 28672, 64),
]


@pytest.mark.parametrize("N,K,g", SHAPES)
def test_gemv_shapes(pkg, dev, N, K, g):
    import torch
    x, [(w, s, b)] = o.make_inputs(1, N, K, g, seed=N * 7 + K)
    y = pkg.matmul_q4(to_dev(x, dev), to_dev(w, dev), to_dev(s, dev), to_dev(b, dev), 1, K, N, g)
    torch.cuda.synchronize()
    assert_parity(y.cpu().numpy(), o.matmul_q4_f64(x, w, s, b, g), TOL_GEMV, f"N={N} K={K} g={g}")


@pytest.mark.parametrize("K,g", [(256, 64), (3072, 64), (160, 32), (512, 128)])
def test_gemv_nibbles_and_dequant_bit_exact(pkg, dev, K, g):
    """One-hot x picks column k: with s=1, b=0 the output is the unpacked code
    q[n,k] exactly; with the benchmark's scales/biases it is fp16(s*q+b) exactly."""
    import torch
    N = 64
    rng = np.random.default_rng(K)
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    w = o.pack_q4(q)
    _, [(_, s, b)] = o.make_inputs(1, N, K, g, seed=K + 1)
    ones, zeros = np.ones_like(s), np.zeros_like(b)
    tw = to_dev(w, dev)
    ks = sorted(set(list(range(16)) + [31, 32, 33, g - 1, g, K // 2 + 5, K - 8, K - 1]))
    deq = o.dequant_f64(w, s, b, g)
    for k in ks:
        x = np.zeros((1, K), np.float16)
        x[0, k] = 1.0
        tx = to_dev(x, dev)
        y1 = pkg.matmul_q4(tx, tw, to_dev(ones, dev), to_dev(zeros, dev), 1, K, N, g)
        y2 = pkg.matmul_q4(tx, tw, to_dev(s, dev), to_dev(b, dev), 1, K, N, g)
        torch.cuda.synchronize()
        assert np.array_equal(y1.cpu().numpy()[0].astype(np.int64), q[:, k].astype(np.int64)), k
        want = deq[:, k].astype(np.float16)
        assert np.array_equal(y2.cpu().numpy()[0].view(np.uint16), want.view(np.uint16)), k


def test_gemv_all_eight_codes_is_zero(pkg, dev):
    import torch
    N, K, g = 256, 3072, 64
    x, [(_, s, b)] = o.make_inputs(1, N, K, g, seed=3)
    w8 = o.pack_q4(np.full((N, K), 8, np.uint8))
    y = pkg.matmul_q4(to_dev(x, dev), to_dev(w8, dev), to_dev(s, dev), to_dev(b, dev), 1, K, N, g)
    torch.cuda.synchronize()
    assert np.all(np.abs(y.float().cpu().numpy()) <= 1e-3)


@pytest.mark.parametrize("name", ["swiglu_m1_n64_k192_g64"])
def test_golden_swiglu_gemv(pkg, dev, name):
    import torch
    t, meta = load_golden(name)
    N, K, g = int(meta["N"]), int(meta["K"]), int(meta["group_size"])
    gate = q4w(pkg, t["gate_proj.weight"], t["gate_proj.scales"], t["gate_proj.biases"], K, g, dev)
    up = q4w(pkg, t["up_proj.weight"], t["up_proj.scales"], t["up_proj.biases"], K, g, dev)
    y = pkg.matmul_q4_silu_mul(to_dev(t["x"], dev), gate, up, 1, K, N)
    torch.cuda.synchronize()
    assert_parity(y.cpu().numpy(), t["y_f64"], TOL_GEMV, name)
    # the reference's two-step path (fp16 gate/up, then silu_mul) differs only
    # by its intermediate roundings
    assert o.max_rel_err(y.cpu().numpy(), t["y_emu"].astype(np.float64)) < 5e-3


@pytest.mark.parametrize("N,K", [(64, 3072), (8192, 3072), (300, 8192), (50, 160), (8200, 10240),
                                 (20, 20000)])
def test_swiglu_gemv_shapes(pkg, dev, N, K):
    import torch
    g = 32 if K % 64 else 64
    x, [(wg, sg, bg), (wu, su, bu)] = o.make_inputs(1, N, K, g, seed=N + K, n_weights=2)
    ref = o.silu_mul_f64(o.matmul_q4_f64(x, wg, sg, bg, g), o.matmul_q4_f64(x, wu, su, bu, g))
    y = pkg.matmul_q4_silu_mul(to_dev(x, dev), q4w(pkg, wg, sg, bg, K, g, dev),
                               q4w(pkg, wu, su, bu, K, g, dev), 1, K, N)
    torch.cuda.synchronize()
    assert_parity(y.cpu().numpy(), ref, TOL_GEMV, f"swiglu N={N} K={K}")


# benchmark configs at full size: q/o, k/v, down, lm_head.  The oracle checks a
# sample of rows; size-independent properties cover the rest.
FULL = [("q_proj", 3072, 3072), ("k_proj", 1024, 3072), ("down_proj", 3072, 8192),
        ("lm_head", 128256, 3072)]


@pytest.mark.parametrize("name,N,K", FULL)
def test_gemv_full_size(pkg, dev, name, N, K):
    import torch
    g = 64
    x, [(w, s, b)] = gpu_inputs(1, N, K, g, seed=N + K, dev=dev)
    # keep x/16 out of fp16 subnormals so that scaling x by 2 is exact in every
    # intermediate (the kernel pre-scales half of x by 1/16)
    x = torch.where(x.abs() < 2.0 ** -8, torch.zeros_like(x), x)
    y = pkg.matmul_q4(x, w, s, b, 1, K, N, g)
    # exact x2 scaling: every intermediate scales by a power of two
    y2 = pkg.matmul_q4(x * 2, w, s, b, 1, K, N, g)
    # row permutation: rows are computed independently with identical arithmetic
    perm = torch.randperm(N, device=dev)
    yp = pkg.matmul_q4(x, w[perm].contiguous(), s[perm].contiguous(), b[perm].contiguous(), 1, K,
                       N, g)
    y_again = pkg.matmul_q4(x, w, s, b, 1, K, N, g)
    torch.cuda.synchronize()
    # fp16 subnormal outputs sit on an absolute grid, where rounding does not
    # commute with scaling; everywhere else the match is exact
    normal = y.abs() >= 2.0 ** -13
    assert torch.equal(y2[normal], (y * 2)[normal])
    assert torch.all((y2.float() - 2 * y.float()).abs() <= 2.0 ** -23)
    assert torch.equal(yp, y[:, perm])
    assert torch.equal(y_again, y)  # deterministic
    rows = np.random.default_rng(N).choice(N, size=min(N, 768), replace=False)
    rows.sort()
    ref = o.matmul_q4_f64(host(x), host(w)[rows], host(s)[rows], host(b)[rows], g)
    assert_parity(y.cpu().numpy()[:, rows], ref, TOL_GEMV, name)


def test_gemv_full_size_swiglu(pkg, dev):
    """gate/up [8192 x 3072] fused with SiLU x up (benchmark config 2)."""
    import torch
    N, K, g = 8192, 3072, 64
    x, [(wg, sg, bg), (wu, su, bu)] = gpu_inputs(1, N, K, g, seed=11, dev=dev, n_weights=2)
    gate, up = pkg.Q4Weight(wg, sg, bg, K, g), pkg.Q4Weight(wu, su, bu, K, g)
    y = pkg.matmul_q4_silu_mul(x, gate, up, 1, K, N)
    torch.cuda.synchronize()
    rows = np.random.default_rng(5).choice(N, size=1024, replace=False)
    xs = host(x)
    ref = o.silu_mul_f64(o.matmul_q4_f64(xs, host(wg)[rows], host(sg)[rows], host(bg)[rows], g),
                         o.matmul_q4_f64(xs, host(wu)[rows], host(su)[rows], host(bu)[rows], g))
    assert_parity(y.cpu().numpy()[:, rows], ref, TOL_GEMV, "gate/up swiglu")


def test_gemv_on_side_stream_and_linear_route(pkg, dev):
    import torch
    N, K, g = 512, 3072, 64
    x, [(w, s, b)] = o.make_inputs(1, N, K, g, seed=21)
    ref = o.matmul_q4_f64(x, w, s, b, g)
    qw = q4w(pkg, w, s, b, K, g, dev)
    tx = to_dev(x, dev)
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        y = pkg.linear(tx, qw, 1, K, N, fast=False, stream=st)
    st.synchronize()
    assert_parity(y.cpu().numpy(), ref, TOL_GEMV, "side stream")
    y_fast = pkg.linear(tx, qw, 1, K, N, fast=True)  # M == 1: still the GEMV
    torch.cuda.synchronize()
    assert torch.equal(y_fast, y)


def test_silu_mul_standalone(pkg, dev):
    import torch
    rng = np.random.default_rng(31)
    for n in (1, 7, 8, 4096 + 3, 750 * 8192):
        a = (rng.standard_normal(n) * 3).astype(np.float16)
        bb = rng.standard_normal(n).astype(np.float16)
        want = o.c_silu_mul(a, bb)
        ta, tb = to_dev(a, dev), to_dev(bb, dev)
        got = pkg.silu_mul(ta, tb)
        torch.cuda.synchronize()
        got = got.cpu().numpy()
        ulp = np.spacing(np.abs(want)).astype(np.float64)
        diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
        assert np.all(diff <= ulp), n
        assert np.mean(got.view(np.uint16) == want.view(np.uint16)) > 0.99
    # misaligned (offset) views take the scalar path
    a = to_dev((rng.standard_normal(1001)).astype(np.float16), dev)
    b = to_dev((rng.standard_normal(1001)).astype(np.float16), dev)
    got = pkg.silu_mul(a[1:], b[1:])
    torch.cuda.synchronize()
    want = o.c_silu_mul(a[1:].cpu().numpy(), b[1:].cpu().numpy())
    assert np.max(np.abs(got.cpu().numpy().astype(np.float64) - want.astype(np.float64))
                  / (np.spacing(np.abs(want)).astype(np.float64))) <= 1.0


@pytest.mark.parametrize("lds", [False, True])
def test_bench_hbm_read_reads_every_word(dev, lds):
    """bench.py's read ceiling (csrc/bench/hbm_read.hip, into registers, and
    through direct global -> LDS copies) touches every 32-bit word once: the
    XOR of its per-block words equals the XOR of the buffer, for sizes that
    are not multiples of the grid's step, with one or several steps per block
    (odd and even counts); a size that is not a multiple of 16 is rejected."""
    import torch
    import bench
    sink = torch.empty(bench.bench_lib().sltx_bench_hbm_read_blocks(), dtype=torch.int32,
                       device=dev)
    for nbytes in (16, 4096 * 16 + 48, 1024 * 4096 * 16 * 3 + 16384 * 3 + 16 * 5,
                   64 * 2 ** 20 + 16 * 7):
        src = torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), device=dev, dtype=torch.int64).to(torch.int32)
        bench.hbm_read(torch, src, sink, lds=lds)
        torch.cuda.synchronize()
        want = np.bitwise_xor.reduce(src.cpu().numpy().view(np.uint32))
        got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
        assert got == want, nbytes
    with pytest.raises(RuntimeError):
        bench.hbm_read(torch, torch.zeros(5, dtype=torch.int16, device=dev), sink, lds=lds)
