"""GPU check of sltx_sample_top_p_noalloc (the sampler with a fixed per-GPU
scratch, allocating nothing) against sltx_sample_top_p through the C ABI.

Token selection is index work, so the bar is bit-exact: the same token for
the same logits, seen ids and draw.  Two calls in a row on one GPU, the
second over a smaller vocabulary (the scratch keeps the first call's
contents), then the same pair captured into a HIP graph on a fresh stream
that never ran the sampler eagerly (where the workspace entry point cannot
run) and replayed.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _logits(torch, gen, dev, n, kind):
    if kind == "peaked":
        return (3.0 * torch.randn(n, generator=gen, device=dev)).half()
    if kind == "flat":
        return (0.05 * torch.randn(n, generator=gen, device=dev)).float()
    return torch.randint(-4, 5, (n,), generator=gen, device=dev).half()   # fp16 ties


def _pair(pkg, torch, logits, seen, u, stream):
    """(noalloc token, workspace-sampler token) for one input."""
    a = pkg.sample_noalloc(logits, 0.7, 0.9, 1.1, seen, u, stream=stream)
    b = pkg.sample(logits, 0.7, 0.9, 1.1, seen, u, stream=stream)
    return a, b


@pytest.mark.parametrize("kind", ["peaked", "flat", "ties"])
def test_noalloc_matches_workspace_sampler(pkg, dev, kind):
    import torch
    gen = torch.Generator(device=dev)
    gen.manual_seed({"peaked": 1, "flat": 2, "ties": 3}[kind])
    rng = np.random.default_rng(7)
    s = torch.cuda.Stream()
    # two calls in a row, the second over fewer logits
    for n in (128256, 50000):
        logits = _logits(torch, gen, dev, n, kind)
        seen = torch.randint(0, n, (64,), generator=gen, device=dev, dtype=torch.int32)
        for u in rng.random(4):
            with torch.cuda.stream(s):
                a, b = _pair(pkg, torch, logits, seen, float(u), s)
            s.synchronize()
            assert int(a.item()) == int(b.item()), (kind, n, u)


def test_noalloc_at_the_limit_and_past_it(pkg, dev):
    import torch
    gen = torch.Generator(device=dev)
    gen.manual_seed(9)
    n = 262144
    logits = (2.0 * torch.randn(n, generator=gen, device=dev)).float()
    a = pkg.sample_noalloc(logits, 1.0, 0.95, 1.0, None, 0.25)
    b = pkg.sample(logits, 1.0, 0.95, 1.0, None, 0.25)
    torch.cuda.synchronize()
    assert int(a.item()) == int(b.item())
    big = torch.zeros(n + 1, device=dev)
    with pytest.raises(pkg.SltxError, match="262144"):
        pkg.sample_noalloc(big, 1.0, 0.9, 1.0, None, 0.5)


def test_noalloc_under_capture_on_a_fresh_stream(pkg, dev):
    """Captured on a stream that never ran the sampler (so it has no
    workspace): the noalloc call captures and each replay gives the eager
    workspace sampler's token, for two calls in a row (the second smaller),
    with eager work and synchronisation between the replays."""
    import torch
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    l1 = (3.0 * torch.randn(128256, generator=gen, device=dev)).half()
    l2 = (3.0 * torch.randn(40000, generator=gen, device=dev)).half()
    seen = torch.randint(0, 40000, (32,), generator=gen, device=dev, dtype=torch.int32)
    o1 = torch.empty(1, dtype=torch.int32, device=dev)
    o2 = torch.empty(1, dtype=torch.int32, device=dev)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        pkg.sample_noalloc(l1, 0.8, 0.9, 1.1, seen, 0.3, out=o1, stream=s)
        pkg.sample_noalloc(l2, 0.8, 0.9, 1.1, seen, 0.6, out=o2, stream=s)
    torch.cuda.synchronize()
    r1 = int(pkg.sample(l1, 0.8, 0.9, 1.1, seen, 0.3).item())
    r2 = int(pkg.sample(l2, 0.8, 0.9, 1.1, seen, 0.6).item())
    for rep in range(3):
        o1.fill_(-1)
        o2.fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        assert (int(o1.item()), int(o2.item())) == (r1, r2), rep
        # eager work on the GPU between replays
        pkg.sample(l2, 0.8, 0.9, 1.1, seen, 0.1)
        torch.cuda.synchronize()
