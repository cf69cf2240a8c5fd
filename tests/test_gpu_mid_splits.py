"""GPU parity of the mid-M route's K halves (q4_mid.hip, SPLIT): one weight
set whose 32-row blocks would fill at most half of the CUs (N <= 4096) runs
two blocks per output tile, each over half of K; each stores its half's fp32
sums to the per-stream workspace and counts its arrival on the tile's
counter, and the block that arrives second adds the two halves in split
order and applies the epilogue (q4_split.hpp).  It also resets the counter
for the next launch.

Same semantics as every M > 1 route (matmulQ4Fast / matmulQ4FastF32,
Ops.swift:312-381; the residual add of LlamaModel.swift:330-331; bias +
GELU-tanh of DiTModel.swift:102-125).  Covered: the three half-K builds
(K = 4096, 8192, 10240), group sizes 32, 64 and 128, ragged and tiny N, M
from 17 to 32, fp16 and fp32 outputs (which must agree bit for bit), the
epilogues, launches back to back on one stream with different tile counts
(the counters must return to zero after each), split launches inside a HIP
graph replayed between eager ones, and the unsplit fallback of a capture
that cannot allocate the workspace.  The sum is the same whichever block arrives last, so
every repeat must equal the first result bit for bit.
"""
import numpy as np
import pytest

from helpers import TOL_GEMM_F16, TOL_ROUNDED_W, assert_parity, q4w, rounded_weights_f16, to_dev
from oracle import q4_oracle as o

pytestmark = pytest.mark.gpu


def mid_splits(N, K, g):
    """The K splits the mid-M route plans for one weight set (its rule: two
    halves when 2 x the 32-row blocks fit the 256 CUs, the half holds 2, 4 or
    5 weight groups of 1024 k and whole 16-byte pieces of scales per row)."""
    nblocks, ng, groups = -(-N // 32), K // 1024, K // g
    if 2 * nblocks > 256 or ng % 2 or ng // 2 not in (2, 4, 5) or (groups // 2) % 8:
        return 1
    return 2


# (M, N, K, g)
CASES = [
    (32, 4096, 4096, 64),     # T5 q/k/v/o at M = 32
    (32, 4096, 10240, 64),    # T5 wo
    (24, 3072, 8192, 64),     # Llama down
    (17, 4096, 10240, 128),
    (29, 1000, 4096, 128),    # ragged last tile
    (20, 33, 8192, 32),       # two tiles, the second one column wide
    (31, 4096, 4096, 32),
]


def _inputs(dev, M, N, K, g, seed):
    x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=seed)
    return (x, w, s, b), [to_dev(a, dev) for a in (x, w, s, b)]


@pytest.mark.parametrize("M,N,K,g", CASES)
def test_mid_split_parity(pkg, dev, M, N, K, g):
    import torch
    assert mid_splits(N, K, g) == 2
    assert pkg.gemm_route(M, N, K, group_size=g) == "mid"
    (x, w, s, b), args = _inputs(dev, M, N, K, g, seed=M + N + K + g)
    y = pkg.matmul_q4_fast_f32(*args, M, K, N, g)
    again = [pkg.matmul_q4_fast_f32(*args, M, K, N, g) for _ in range(4)]
    y16 = pkg.matmul_q4_fast(*args, M, K, N, g)
    torch.cuda.synchronize()
    for r in again:
        assert torch.equal(r, y)
    assert torch.equal(y.half(), y16)
    got = y.cpu().numpy()
    assert_parity(got, o.matmul_q4_f64(x, w, s, b, g), TOL_GEMM_F16, f"M={M} N={N} K={K} g={g}")
    ok, worst = o.elementwise_ok(got, x.astype(np.float64) @ rounded_weights_f16(w, s, b, g).T,
                                 **TOL_ROUNDED_W)
    assert ok, worst


@pytest.mark.parametrize("M", [25, 32])
def test_mid_split_epilogues(pkg, dev, M):
    """Residual add (also in place) and bias + GELU-tanh run after the halves
    are added (on the block that adds them)."""
    import torch
    N, K, g = 4096, 4096, 64
    assert mid_splits(N, K, g) == 2 and pkg.gemm_route(M, N, K, group_size=g) == "mid"
    (x, w, s, b), _ = _inputs(dev, M, N, K, g, seed=900 + M)
    rng = np.random.default_rng(M)
    res = rng.standard_normal((M, N)).astype(np.float16)
    bias = rng.standard_normal(N).astype(np.float32)
    wt = q4w(pkg, w, s, b, K, g, dev)
    proj = o.matmul_q4_f64(x, w, s, b, g)
    y = pkg.matmul_q4_residual(to_dev(x, dev), wt, to_dev(res, dev), M, N)
    inplace = to_dev(res, dev)   # out is the residual itself: the adding block reads, then writes
    pkg.matmul_q4_residual(to_dev(x, dev), wt, inplace, M, N, out=inplace)
    yg = pkg.matmul_q4_ex(to_dev(x, dev), wt, M, N, out_dtype=torch.float32,
                          bias=to_dev(bias, dev), epilogue=pkg.SLTX_EPI_GELU_TANH)
    torch.cuda.synchronize()
    want = res.astype(np.float64) + proj.astype(np.float16).astype(np.float64)
    assert_parity(y.cpu().numpy(), want, TOL_GEMM_F16, f"residual M={M}")
    assert torch.equal(inplace, y)
    assert_parity(yg.cpu().numpy(), o.gelu_tanh_f64(proj + bias), TOL_GEMM_F16,
                  f"bias+gelu M={M}")


def test_mid_splits_back_to_back(pkg, dev):
    """Split launches of three shapes with different tile counts, interleaved
    on one stream with no synchronization between them (120 launches): each
    launch must leave every counter at zero for the next, and each must equal
    the first bit for bit."""
    import torch
    shapes = [CASES[0], CASES[2], CASES[5]]
    inputs = [_inputs(dev, *c, seed=11 + i)[1] for i, c in enumerate(shapes)]
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        first = [pkg.matmul_q4_fast(*a, M, K, N, g, stream=st)
                 for a, (M, N, K, g) in zip(inputs, shapes)]
        outs = [[pkg.matmul_q4_fast(*a, M, K, N, g, stream=st)
                 for a, (M, N, K, g) in zip(inputs, shapes)] for _ in range(40)]
    st.synchronize()
    for rnd in outs:
        for r, f in zip(rnd, first):
            assert torch.equal(r, f)


def test_mid_splits_in_graph(pkg, dev):
    """Split launches captured into a HIP graph (after eager calls on the
    stream, which size its workspace), replayed with eager split launches on
    the same stream between the replays: every replay equals the eager
    results bit for bit."""
    import torch
    shapes = [CASES[1], CASES[4]]
    inputs = [_inputs(dev, *c, seed=31 + i)[1] for i, c in enumerate(shapes)]
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        eager = [pkg.matmul_q4_fast(*a, M, K, N, g, stream=st)
                 for a, (M, N, K, g) in zip(inputs, shapes)]
    st.synchronize()
    outs = [torch.empty_like(e) for e in eager]
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=st):
        for _ in range(2):   # two launches of each in the graph
            for a, (M, N, K, g), out in zip(inputs, shapes, outs):
                pkg.matmul_q4_fast(*a, M, K, N, g, out=out, stream=st)
    for _ in range(3):
        for out in outs:
            out.zero_()
        torch.cuda.synchronize()
        # the replay and the eager launches share the stream's workspace, so
        # they run in order on that stream
        with torch.cuda.stream(st):
            gr.replay()
            between = [pkg.matmul_q4_fast(*a, M, K, N, g, stream=st)
                       for a, (M, N, K, g) in zip(inputs, shapes)]
        torch.cuda.synchronize()
        for out, b, e in zip(outs, between, eager):
            assert torch.equal(out, e)
            assert torch.equal(b, e)


def test_mid_split_unsplit_in_fresh_capture(pkg, dev):
    """A capture on a stream whose workspace does not exist yet cannot
    allocate it: the launch runs the whole K in one block per tile (the same
    product, its fp32 sums in another order), inside the oracle's tolerance."""
    import torch
    M, N, K, g = CASES[0]
    (x, w, s, b), args = _inputs(dev, M, N, K, g, seed=77)
    out = torch.empty(M, N, dtype=torch.float32, device=dev)
    st = torch.cuda.Stream()
    st.synchronize()
    pkg.release_workspace(st)   # torch reuses streams: drop any workspace it holds
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=st):
        pkg.matmul_q4_fast_f32(*args, M, K, N, g, out=out, stream=st)
    gr.replay()
    torch.cuda.synchronize()
    assert_parity(out.cpu().numpy(), o.matmul_q4_f64(x, w, s, b, g), TOL_GEMM_F16, "unsplit")
