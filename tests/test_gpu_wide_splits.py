"""GPU parity of the wide-M route's K splits (q4_wide.hip, SPLIT): each block
stores its split's fp32 sums to the per-stream workspace, counts its arrival
on its output tile's counter, and the last block of the tile adds the S
partial sums in split order (as the split-K reduce pass adds them) and
applies the epilogue; it also resets the counter for the next launch.

Same semantics as every M > 1 route (matmulQ4Fast / matmulQ4FastF32,
Ops.swift:312-381; the SwiGLU / GeGLU pairs, LlamaModel.swift:275-277,
T5Encoder.swift:191-199).  Covered: 2, 3, 4 and 8 splits, one and two blocks
along M, gated pairs, ragged and odd column counts (element loads and
stores), fp16 and fp32 outputs (which must agree bit for bit), launches
back to back on one stream with different tile counts (the counters must
return to zero after each), and split launches inside a HIP graph replayed
between eager ones.  The sum is the same whichever block arrives last, so
every repeat must equal the first result bit for bit.
"""
import numpy as np
import pytest

from helpers import GATE, TOL_GEMM_F16, assert_parity, to_dev
from oracle import q4_oracle as o

pytestmark = pytest.mark.gpu


def wide_splits(M, N, K, g, pair):
    """The K splits the wide route plans for this shape (its rule: split
    while the blocks would not fill the GPU or a split's K range holds more
    than 64 scale groups, in whole rounds of 128 k, up to 8 splits; three
    instead of two where two leave a quarter of the CUs idle and three fit)."""
    mblocks = -(-M // 128)
    nblocks = -(-N // (32 if pair else 64))
    if mblocks == 2 and 160 <= nblocks * 2 and nblocks * 3 <= 256:   # three M-blocks
        mblocks = 3
    blocks, rounds, s = nblocks * mblocks, K // 128, 1
    while s < 8 and rounds % (2 * s) == 0 and (K // s // g > 64 or
                                                (blocks * s < 160 and rounds // (2 * s) >= 4)):
        s *= 2
    if (s < 3 and blocks * s < 192 and blocks * 3 <= 256 and rounds % 3 == 0 and rounds // 3 >= 4
            and K // 3 // g <= 64):
        s = 3
    return s


# (M, N, K, g, epilogue, splits)
CASES = [
    (128, 5120, 3072, 64, None, 3),      # Llama q|k|v at M = 128
    (64, 5101, 3072, 32, None, 3),       # three splits, odd N
    (200, 2600, 3072, 64, None, 3),      # three splits, two blocks along M, ragged N
    (128, 3072, 3072, 64, None, 4),      # Llama o
    (128, 4096, 10240, 64, None, 4),     # T5 wo at M = 128
    (64, 1024, 8192, 64, None, 8),
    (200, 3072, 8192, 64, None, 2),      # two blocks along M
    (100, 1000, 4096, 32, None, 8),      # ragged last column block
    (64, 1001, 2048, 64, None, 4),       # odd N: element loads and stores
    (128, 2560, 3072, 64, "gelu", 3),    # gated pairs
    (96, 1024, 4096, 64, "silu", 8),
]
T5_WO, GELU_PAIR = CASES[4], CASES[9]


def _run(pkg, args, M, N, K, g, epi, out=None, stream=None, f32=False):
    x, ws = args
    if epi is None:
        fn = pkg.matmul_q4_fast_f32 if f32 else pkg.matmul_q4_fast
        return fn(x, *ws[0], M, K, N, g, out=out, stream=stream)
    gate, up = (pkg.Q4Weight(*w, K, g) for w in ws)
    fn = pkg.matmul_q4_geglu if epi == "gelu" else pkg.matmul_q4_silu_mul
    return fn(x, gate, up, M, K, N, out=out, stream=stream)


def _inputs(dev, M, N, K, g, epi, seed):
    x, sets = o.make_inputs(M, N, K, g, seed=seed, n_weights=1 if epi is None else 2)
    return (x, sets), (to_dev(x, dev), [tuple(to_dev(a, dev) for a in w) for w in sets])


@pytest.mark.parametrize("M,N,K,g,epi,splits", CASES)
def test_wide_split_parity(pkg, dev, M, N, K, g, epi, splits):
    import torch
    assert wide_splits(M, N, K, g, epi is not None) == splits
    assert pkg.gemm_route(M, N, K, group_size=g, gated=epi is not None) == "wide"
    (x, sets), args = _inputs(dev, M, N, K, g, epi, seed=M + N + K)
    y = _run(pkg, args, M, N, K, g, epi)
    again = [_run(pkg, args, M, N, K, g, epi) for _ in range(4)]
    torch.cuda.synchronize()
    for r in again:
        assert torch.equal(r, y)
    rows = np.unique(np.array([0, 1, 31, 32, M // 2, M - 1]))
    xs = x[rows].astype(np.float64)
    if epi is None:
        y32 = _run(pkg, args, M, N, K, g, epi, f32=True)
        torch.cuda.synchronize()
        assert torch.equal(y32.half(), y)
        want = o.matmul_q4_f64(xs, *sets[0], g)
        assert_parity(y32.cpu().numpy()[rows], want, TOL_GEMM_F16, f"M={M} N={N} K={K} S={splits}")
    else:
        gp = o.matmul_q4_f64(xs, *sets[0], g)
        up = o.matmul_q4_f64(xs, *sets[1], g)
        want = o.gelu_tanh_f64(gp) * up if epi == "gelu" else o.silu_mul_f64(gp, up)
        got = y.cpu().numpy()[rows].astype(np.float64)
        assert o.max_rel_err(got, want) <= GATE, f"{epi} M={M} N={N} K={K} S={splits}"


def test_wide_splits_back_to_back(pkg, dev):
    """Split launches of three shapes with different tile counts and split
    counts, interleaved on one stream with no synchronization between them
    (120 launches): each launch must leave every counter at zero for the
    next, and each must equal the first bit for bit."""
    import torch
    shapes = [CASES[0], T5_WO, CASES[5]]   # 3, 4 and 8 splits
    inputs = [_inputs(dev, *c[:5], seed=7 + i)[1] for i, c in enumerate(shapes)]
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        first = [_run(pkg, a, *c[:5], stream=st) for a, c in zip(inputs, shapes)]
        outs = [[_run(pkg, a, *c[:5], stream=st) for a, c in zip(inputs, shapes)] for _ in range(40)]
    st.synchronize()
    for rnd in outs:
        for r, f in zip(rnd, first):
            assert torch.equal(r, f)


def test_wide_splits_in_graph(pkg, dev):
    """Split launches captured into a HIP graph (after eager calls on the
    stream, which size its workspace), replayed with eager split launches on
    the same stream between the replays: every replay equals the eager
    results bit for bit."""
    import torch
    shapes = [T5_WO, GELU_PAIR]
    inputs = [_inputs(dev, *c[:5], seed=21 + i)[1] for i, c in enumerate(shapes)]
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        eager = [_run(pkg, a, *c[:5], stream=st) for a, c in zip(inputs, shapes)]
    st.synchronize()
    outs = [torch.empty_like(e) for e in eager]
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=st):
        for a, c, out in zip(inputs, shapes, outs):
            _run(pkg, a, *c[:5], out=out, stream=st)
        for a, c, out in zip(inputs, shapes, outs):   # a second launch of each in the graph
            _run(pkg, a, *c[:5], out=out, stream=st)
    for _ in range(3):
        for out in outs:
            out.zero_()
        torch.cuda.synchronize()
        # the replay and the eager launches share the stream's workspace, so
        # they run in order on that stream
        with torch.cuda.stream(st):
            gr.replay()
            between = [_run(pkg, a, *c[:5], stream=st) for a, c in zip(inputs, shapes)]
        torch.cuda.synchronize()
        for out, b, e in zip(outs, between, eager):
            assert torch.equal(out, e)
            assert torch.equal(b, e)
