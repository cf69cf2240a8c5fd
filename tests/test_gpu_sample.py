"""argmax and top-p sampling on the GPU (sltx_argmax, sltx_sample_top_p)
against the oracle (argmax_ref, sample_ref; Ops.swift:757-806, 2060-2098).

* argmax is index work: bit-exact, including ties (first index), NaNs (never
  win; NaN at index 0 gives 0), infinities and n = 1.
* sampling: the probabilities are the reference's fp32 steps, but the GPU
  forms its sums differently (a strided + tree softmax denominator; exact
  integer running masses).  The oracle's gpu_sums mode forms the same sums,
  so the GPU token must equal it wherever no other token lies within 5e-7
  (in probability) of the draw, and otherwise lie within that window (exp's
  last ulp may differ, which moves draws among dense tail tokens).  Against the reference's own sequential fp32 sums the token must lie
  within the rounding those sums carry on the same input, measured by the
  oracle: tol = 2 * max |fp32 running sum - exact| over the nucleus (the
  cutoff test and the r -= p walk each carry it) + the softmax denominator's
  relative error + 1e-6, near-equal probabilities (relative 1e-5) allowed to
  swap.
* cases: vocabulary 2 .. 128256 (Llama 3.2's), fp16 and fp32 logits, a peaked
  (LM-like) and a flat distribution (nucleus beyond the 8192 sorted in LDS),
  integer-valued logits (exact ties), top_p below and above the total mass,
  repeated / out-of-range seen ids, and replay from a captured HIP graph.
"""
import zlib

import numpy as np
import pytest

from oracle import q4_oracle as o

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


# ----------------------------------------------------------------- argmax --

def _argmax_cases():
    rng = np.random.default_rng(30)
    nan, inf = np.nan, np.inf
    cases = []
    for n in (1, 7, 1000, 4097, 128256):
        cases.append(rng.standard_normal(n))
        cases.append(rng.integers(-4, 4, n).astype(np.float64))        # ties
    v = rng.standard_normal(128256); v[0] = nan; cases.append(v)
    v = rng.standard_normal(128256); v[rng.integers(0, 128256, 50)] = nan; cases.append(v)
    v = rng.standard_normal(5000); v[4999] = 50.0; cases.append(v)        # last index
    v = rng.standard_normal(5000); v[0] = 50.0; cases.append(v)           # first index
    cases += [np.array([-inf, -inf, -inf]), np.array([-inf, nan, -inf]), np.array([1.0, inf, inf]),
              np.array([nan, nan]), np.array([0.0, -0.0, 0.0])]
    v = np.full(128256, -1.0); v[[9000, 70000, 120000]] = 3.0; cases.append(v)
    return cases


@pytest.mark.parametrize("dt", [np.float16, np.float32])
def test_argmax_exact(pkg, dev, dt):
    import torch
    for i, a in enumerate(_argmax_cases()):
        x = a.astype(dt)
        out = pkg.argmax(_t(x, dev))
        torch.cuda.synchronize()
        assert out.dtype == torch.int32 and out.numel() == 1
        assert int(out.item()) == o.argmax_ref(x), (i, x.size)


# --------------------------------------------------------------- sampling --

def acceptable(logits, T, top_p, pen, seen, u, gpu_sums=False, tol=None, tie=1e-5):
    """(oracle token, tokens within rounding of the draw)."""
    tok, info = o.sample_ref(logits, T, top_p, pen, seen, u, detail=True, gpu_sums=gpu_sums)
    ps = info["probs"].astype(np.float64)
    order = info["order"]
    c = np.cumsum(ps)
    lo = np.concatenate([[0.0], c[:-1]])
    n = ps.size
    if tol is None:
        k = min(n, 2 * info["cutoff"] + 1)
        tol = 2 * float(info["cum_err"][:k].max()) + info["sum_rel_err"] + 1e-6
    # cutoffs the rounding admits: a contiguous run of positions
    ks = [info["cutoff"]] + (np.nonzero(np.abs(c - top_p) <= tol)[0] + 1).tolist()
    if c[-1] < top_p + tol:
        ks.append(n)
    kmin, kmax = min(ks), max(ks)
    r_lo, r_hi = u * c[kmin - 1], u * c[kmax - 1]
    ranges = []   # [first, last] positions the draw may land on
    hit = np.nonzero((lo[:kmax] - tol <= r_hi) & (c[:kmax] + tol >= r_lo))[0]
    if hit.size:
        ranges.append((int(hit[0]), int(hit[-1])))
    if r_lo <= tol or r_hi >= c[kmin - 1] - tol:   # the walk's fall-back to the first token
        ranges.append((0, 0))
    neg = -ps   # ascending
    toks = set()
    for a, b in ranges:   # widen to near-equal probabilities (they may swap places)
        a2 = int(np.searchsorted(neg, -ps[a] * (1 + tie), "left"))
        b2 = int(np.searchsorted(neg, -ps[b] * (1 - tie), "right")) - 1
        toks |= set(order[min(a, a2):max(b, b2) + 1].tolist())
    return tok, toks


def _logits(kind, n, rng):
    if kind == "peaked":     # LM-like: a few tokens hold most of the mass
        return rng.standard_normal(n) * 4.0
    if kind == "flat":       # nucleus of thousands of tokens
        return rng.standard_normal(n) * 0.5
    return rng.integers(-6, 7, n).astype(np.float64)   # "tied": exact ties


CASES = [(n, kind) for n in (2, 50, 1000, 32000, 128256) for kind in ("peaked", "flat", "tied")]


@pytest.mark.parametrize("n,kind", CASES)
def test_sample_matches_oracle(pkg, dev, n, kind):
    import torch
    rng = np.random.default_rng(n * 7 + len(kind))
    for dt in (np.float16, np.float32):
        lg = _logits(kind, n, rng).astype(dt)
        x = _t(lg, dev)
        seen_np = np.concatenate([rng.integers(0, n, 12), [0, 0, n, n + 5, -3]]).astype(np.int32)
        seen = _t(seen_np, dev)
        for T, top_p, pen in ((0.7, 0.9, 1.1), (1.0, 0.5, 1.3), (1.3, 1.0, 1.0), (0.7, 2.0, 1.1),
                              (0.9, 0.99, 1.1)):
            for u in (0.0, 0.173, 0.5, 0.871, 0.9999):
                got = int(pkg.sample(x, T, top_p, pen, seen, u).item())
                case = (dt.__name__, T, top_p, pen, u, got)
                exact, ok = acceptable(lg, T, top_p, pen, seen_np, u, gpu_sums=True, tol=5e-7,
                                       tie=5e-7)
                assert got in ok, case + (exact,)
                if len(ok) == 1:   # no token boundary within rounding of the draw
                    assert got == exact, case + (exact,)
                ref, ok = acceptable(lg, T, top_p, pen, seen_np, u)
                assert got in ok, case + (ref,)
    torch.cuda.synchronize()


def _dense(kind, n, rng):
    if kind == "near_flat":      # one level-0 bin: the range histogram narrows it
        return rng.standard_normal(n) * 1e-3
    if kind == "two_clusters":   # two dense bins; the draw lands in either
        return np.where(rng.random(n) < 0.5, 0.0, 0.3) + rng.standard_normal(n) * 1e-3
    if kind == "half_tied":      # a tied bucket inside a dense bin
        v = rng.standard_normal(n) * 1e-3
        v[rng.random(n) < 0.5] = 0.0
        return v
    return rng.standard_normal(n) * 2e-6   # "one_bucket": keys within one range bucket


@pytest.mark.parametrize("kind,dt", [("near_flat", np.float16), ("near_flat", np.float32),
                                     ("two_clusters", np.float32), ("half_tied", np.float32),
                                     ("half_tied", np.float16), ("one_bucket", np.float32)])
def test_sample_dense_nucleus(pkg, dev, kind, dt):
    """Nuclei of tens of thousands of nearly equal probabilities: more
    candidates than the select kernel holds in LDS, so the gather kernel
    builds the range histogram and the narrow kernel compacts only the
    buckets the cutoff and the draw can reach ("one_bucket": every key in
    one bucket, the select kernel's levels over the candidates in HBM).
    Checked against the oracle as in test_sample_matches_oracle."""
    import torch
    n = 128256
    rng = np.random.default_rng(zlib.crc32(kind.encode()) % 1000 + dt(0).itemsize)
    lg = _dense(kind, n, rng).astype(dt)
    x = _t(lg, dev)
    seen_np = rng.integers(0, n, 40).astype(np.int32)
    seen = _t(seen_np, dev)
    for T, top_p, pen in ((0.7, 0.9, 1.1), (1.0, 0.5, 1.0), (1.3, 1.0, 1.0), (0.7, 2.0, 1.1)):
        for u in (0.0, 0.173, 0.5, 0.9999):
            got = int(pkg.sample(x, T, top_p, pen, seen, u).item())
            case = (kind, dt.__name__, T, top_p, pen, u, got)
            exact, ok = acceptable(lg, T, top_p, pen, seen_np, u, gpu_sums=True, tol=5e-7,
                                   tie=5e-7)
            assert got in ok, case + (exact,)
            if len(ok) == 1:
                assert got == exact, case + (exact,)
            ref, ok = acceptable(lg, T, top_p, pen, seen_np, u)
            assert got in ok, case + (ref,)
    torch.cuda.synchronize()


def test_sample_tiny_top_p_is_argmax_of_penalised(pkg, dev):
    rng = np.random.default_rng(31)
    n = 128256
    lg = (rng.standard_normal(n) * 2).astype(np.float16)
    top = np.argsort(-lg.astype(np.float32), kind="stable")[:3]
    seen = _t(np.array([top[0], top[0]], np.int32), dev)
    x = _t(lg, dev)
    ref = o.argmax_ref(lg)
    for u in (0.0, 0.5, 0.99):
        assert int(pkg.sample(x, 1.0, 1e-9, 1.0, None, u).item()) == ref
        pen = lg.astype(np.float32).copy()
        t = int(top[0])
        pen[t] = pen[t] / np.float32(3.0) if pen[t] > 0 else pen[t] * np.float32(3.0)
        assert int(pkg.sample(x, 1.0, 1e-9, 3.0, seen, u).item()) == int(np.argmax(pen))


def test_sample_u_grid_distribution(pkg, dev):
    """Inverse-CDF check on the device: over u = (j + 1/2) / G with top_p
    above 1, token t is drawn G * p_t times (p = fp64 softmax(logits / T))."""
    rng = np.random.default_rng(32)
    lg = rng.standard_normal(10).astype(np.float32)
    x = _t(lg, dev)
    G = 2000
    counts = np.zeros(10, np.int64)
    for j in range(G):
        counts[int(pkg.sample(x, 0.8, 1.5, 1.0, None, (j + 0.5) / G).item())] += 1
    z = lg.astype(np.float64) / np.float64(np.float32(0.8))
    p = np.exp(z - z.max())
    p /= p.sum()
    assert np.all(np.abs(counts - G * p) <= 2.0), (counts, G * p)


def test_sample_graph_replay(pkg, dev):
    """Captured after one eager call on the same stream, the graph replays
    with new logits copied into its input and matches eager calls."""
    import torch
    rng = np.random.default_rng(33)
    n = 128256
    s = torch.cuda.Stream()
    x = torch.empty(n, dtype=torch.float16, device=dev)
    out = torch.empty(1, dtype=torch.int32, device=dev)
    first = (rng.standard_normal(n) * 3).astype(np.float16)
    x.copy_(_t(first, dev))
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        pkg.sample(x, 0.7, 0.9, 1.0, None, 0.42, out=out, stream=s)
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        pkg.sample(x, 0.7, 0.9, 1.0, None, 0.42, out=out, stream=s)
    for rep in range(4):
        lg = (rng.standard_normal(n) * (2 + rep)).astype(np.float16)
        x.copy_(_t(lg, dev))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = int(out.item())
        eager = int(pkg.sample(x, 0.7, 0.9, 1.0, None, 0.42).item())
        torch.cuda.synchronize()
        ref, ok = acceptable(lg, 0.7, 0.9, 1.0, [], 0.42, gpu_sums=True, tol=5e-7, tie=5e-7)
        assert got == eager and got in ok, (rep, got, eager, ref)


def test_sample_degenerate_logits(pkg, dev):
    """All-equal logits (a 128256-way tie, ranked by id at every select
    level, and the worst case for the select kernel) give exactly the
    oracle's token with the GPU's sums; all-NaN logits give index 0, as the
    reference's scan does when every comparison fails (Ops.swift:2082-2097)."""
    import torch
    n = 128256
    for dt in (np.float16, np.float32):
        eq = np.zeros(n, dt)
        x = _t(eq, dev)
        for u in (0.0, 0.3, 0.77, 0.9999):
            got = int(pkg.sample(x, 0.7, 0.9, 1.1, None, u).item())
            assert got == o.sample_ref(eq, 0.7, 0.9, 1.1, [], u, gpu_sums=True), (dt, u, got)
        nan = np.full(n, np.nan, dt)
        for u in (0.0, 0.5, 0.9999):
            got = int(pkg.sample(_t(nan, dev), 0.7, 0.9, 1.1, None, u).item())
            assert got == 0 == o.sample_ref(nan, 0.7, 0.9, 1.1, [], u), (dt, u, got)
    torch.cuda.synchronize()


# ------------------------------------------------- device-resident state --

def _state(pkg, dev, cap, draws, history):
    return pkg.SamplerState(cap, draws=np.asarray(draws, np.float32), history=history, device=dev)


def _lm_logits(rng, n, hist, scale):
    """Peaked logits whose largest values include the history's tokens, so
    the repetition penalty changes the draw."""
    lg = rng.standard_normal(n) * scale
    lg[np.asarray(hist) % n] += 3 * scale
    return lg.astype(np.float16)


def test_sample_state_matches_host_form(pkg, dev):
    """sltx_sample_top_p_state reads the seen ids from the device history and
    the draw from draws[next_draw]; each call appends its token and advances
    the draw, as the reference's generate loop grows seenTokens
    (LlamaModel.swift:150-161).  The kernels are the host-argument form's,
    so the tokens agree exactly, and each lies in the oracle's window."""
    import torch
    rng = np.random.default_rng(34)
    n = 128256
    draws = [0.13, 0.77, 0.42, 0.91, 0.05]
    prompt = [5, 17, 99, 17, 128000]
    st = _state(pkg, dev, 64, draws, prompt)
    hist = list(prompt)
    for i in range(12):
        lg = _lm_logits(rng, n, hist, 2.0 + i % 3)
        x = _t(lg, dev)
        got = int(pkg.sample_with_state(x, 0.8, 0.9, 1.3, st).item())
        u = draws[i % len(draws)]
        seen_np = np.array(hist, np.int32)
        host = int(pkg.sample(x, 0.8, 0.9, 1.3, _t(seen_np, dev), u).item())
        assert got == host, (i, got, host)
        exact, ok = acceptable(lg, 0.8, 0.9, 1.3, seen_np, u, gpu_sums=True, tol=5e-7, tie=5e-7)
        assert got in ok, (i, got, exact)
        hist.append(got)
        assert st.tokens() == hist, i
        assert int(st.next_draw.item()) == (i + 1) % len(draws), i
    torch.cuda.synchronize()


def test_sample_state_full_history_and_clamped_draws(pkg, dev):
    """A full history stops growing (and a length beyond the capacity counts
    as the capacity); draws outside [0, 1) and NaN are clamped into it; a
    negative length counts as an empty history."""
    import torch
    rng = np.random.default_rng(35)
    n = 32000
    top = float(np.float32(1.0) - np.float32(2.0 ** -24))
    st = _state(pkg, dev, 3, [1.5, -0.25, float("nan"), 0.5], [7, 8])
    hist = [7, 8]
    for i, u in enumerate([top, 0.0, 0.0, 0.5, top]):
        lg = _lm_logits(rng, n, hist, 2.0)
        x = _t(lg, dev)
        got = int(pkg.sample_with_state(x, 1.0, 0.95, 1.5, st).item())
        host = int(pkg.sample(x, 1.0, 0.95, 1.5, _t(np.array(hist, np.int32), dev), u).item())
        assert got == host, (i, got, host)
        if len(hist) < 3:
            hist.append(got)
        assert st.tokens() == hist, i
    assert int(st.history_len.item()) == 3
    # five calls so far: the next draw is draws[1] = -0.25 (-> 0), then NaN (-> 0)
    assert int(st.next_draw.item()) == 1
    st.history_len.fill_(1000)            # counts as 3, nothing appended
    lg = _lm_logits(rng, n, hist, 2.0)
    x = _t(lg, dev)
    got = int(pkg.sample_with_state(x, 1.0, 0.95, 1.5, st).item())
    host = int(pkg.sample(x, 1.0, 0.95, 1.5, _t(np.array(hist, np.int32), dev), 0.0).item())
    assert got == host and int(st.history_len.item()) == 1000
    assert st.history[:3].tolist() == hist
    st.history_len.fill_(-4)              # empty: the token lands at index 0
    got = int(pkg.sample_with_state(x, 1.0, 0.95, 1.5, st).item())
    host = int(pkg.sample(x, 1.0, 0.95, 1.5, None, 0.0).item())
    assert got == host, (got, host)
    assert int(st.history_len.item()) == 1 and int(st.history[0].item()) == got
    torch.cuda.synchronize()


def test_sample_state_graph_replay(pkg, dev):
    """One captured state-form call, replayed with new logits copied into its
    input: each replay takes the next draw and appends to the history, equal
    to eager calls on a twin state, step by step."""
    import torch
    rng = np.random.default_rng(36)
    n = 128256
    draws = rng.random(7).astype(np.float32)
    prompt = [1, 2, 3, 500, 9000]
    st = _state(pkg, dev, 40, draws, prompt)
    twin = _state(pkg, dev, 40, draws, prompt)
    s = torch.cuda.Stream()
    x = torch.empty(n, dtype=torch.float16, device=dev)
    out = torch.empty(1, dtype=torch.int32, device=dev)
    x.copy_(_t(_lm_logits(rng, n, prompt, 3.0), dev))
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        pkg.sample_with_state(x, 0.7, 0.9, 1.2, st, out=out, stream=s)
    s.synchronize()
    pkg.sample_with_state(x, 0.7, 0.9, 1.2, twin)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        pkg.sample_with_state(x, 0.7, 0.9, 1.2, st, out=out, stream=s)
    torch.cuda.synchronize()
    assert st.tokens() == twin.tokens()   # capture records, it does not run
    for rep in range(10):
        x.copy_(_t(_lm_logits(rng, n, twin.tokens(), 2.0 + rep % 4), dev))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = int(out.item())
        eager = int(pkg.sample_with_state(x, 0.7, 0.9, 1.2, twin).item())
        torch.cuda.synchronize()
        assert got == eager, (rep, got, eager)
        assert st.tokens() == twin.tokens(), rep
        assert int(st.next_draw.item()) == int(twin.next_draw.item()) == (rep + 2) % 7


def test_sample_capture_without_workspace_is_an_error(pkg, dev):
    """A stream that never sampled has no workspace; capture must not
    allocate, so the call fails (and the capture is abandoned)."""
    import torch
    s = torch.cuda.Stream()
    # larger than any workspace an earlier test gave a (pooled) stream
    x = torch.zeros(1 << 22, dtype=torch.float32, device=dev)
    g = torch.cuda.CUDAGraph()
    with pytest.raises(pkg.SltxError) as ei:
        with torch.cuda.graph(g, stream=s):
            pkg.sample(x, 0.7, 0.9, 1.0, None, 0.5, stream=s)
    assert "captured" in str(ei.value)
