"""GPU parity of sltx_decode_layer_q4: one Llama decode layer after attention
in a single launch (o_proj, residual + RMSNorm, gate/up + SiLU x up, down +
residual, and the next layer's RMSNorm + q|k|v; LlamaModel.swift:324-331 then
:288-292), through the C ABI.

* Against the same layer built from this library's per-projection entry
  points (each pinned to the fp64 oracle by tests/test_gpu_gemv.py and
  tests/test_gpu_fused.py): the fused kernel sums the squares of the norms in
  another order, so a normalized value may move by one fp16 ulp; the outputs
  may therefore differ by twice the GEMV bound of tests/helpers.py plus one
  fp16 ulp (the "two paths" allowance of tests/test_gpu_fused.py).
* Against the numpy pipeline of oracle functions (fp64 matmuls, the
  reference's fp16 rounding points) at Llama-3.2-1B shapes: the BASELINE gate
  (max|d| / max|ref| <= 1e-2), an allowance propagated through the three
  chained matmuls on the residual stream, and the q|k|v phase alone at the
  GEMV bound.
* In place as a decode loop uses it (residual_out = residual, attn a view of
  next_qkv_out) and replayed from a HIP graph: bit-identical to eager calls.
* The kernel's bounded waits never ran out (fault counter 0).
"""
import numpy as np
import pytest

from helpers import GATE, TOL_GEMV, assert_parity, gpu_inputs, host
from oracle import q4_oracle as o

pytestmark = pytest.mark.gpu

EPS = 1e-5
SHAPES = [(3072, 8192, 5120), (2048, 8192, 3072)]   # (hidden, ffn, q|k|v rows)


def _norm(torch, gen, dev, K):
    return (1.0 + 0.1 * torch.randn(K, generator=gen, device=dev)).float()


def _layer(pkg, dev, H, F, NQ, seed):
    import torch
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    Q = lambda t, k: pkg.Q4Weight(*t, k, 64)
    _, [wo] = gpu_inputs(1, H, H, 64, seed=seed + 1, dev=dev)
    _, [wg, wu] = gpu_inputs(1, F, H, 64, seed=seed + 2, dev=dev, n_weights=2)
    _, [wd] = gpu_inputs(1, H, F, 64, seed=seed + 3, dev=dev)
    _, [wq] = gpu_inputs(1, NQ, H, 64, seed=seed + 4, dev=dev)
    L = dict(o=Q(wo, H), g=Q(wg, H), u=Q(wu, H), d=Q(wd, F), q=Q(wq, H),
             n2=_norm(torch, gen, dev, H), n1=_norm(torch, gen, dev, H),
             attn=torch.randn(1, H, generator=gen, device=dev).half(),
             h=(4.0 * torch.randn(1, H, generator=gen, device=dev)).half())
    return L


def _unfused(pkg, L, H, F, NQ, last):
    o_ = pkg.linear(L["attn"], L["o"], 1, H, H)
    res, act = pkg.residual_rmsnorm_matmul_q4_silu_mul(L["h"], o_, L["n2"], EPS, L["g"], L["u"], F)
    d = pkg.linear(act, L["d"], 1, F, H)
    h2 = pkg.matmul_q4_residual(act, L["d"], res, 1, H)
    qkv = None if last else pkg.rmsnorm_matmul_q4(h2, L["n1"], EPS, L["q"], NQ)
    return h2, qkv, d


def _two_paths(a, b, tol, what, ref_scale=None):
    """a, b: fp16 results of the same exact value by two kernels (see the
    module docstring); ref_scale: the values whose GEMV bound applies (b by
    default)."""
    a = a.float().cpu().numpy().astype(np.float64)
    b16 = b.cpu().numpy()
    b = b16.astype(np.float64)
    v = b if ref_scale is None else ref_scale.float().cpu().numpy().astype(np.float64)
    allow = (2 * (tol["rtol"] * np.abs(v) + tol["atol_rms"] * np.sqrt(np.mean(v ** 2)))
             + np.spacing(np.abs(b16)).astype(np.float64))
    d = np.abs(a - b)
    assert np.all(d <= allow), f"{what}: worst {np.max(d / allow):.2f}x the allowance"
    assert o.max_rel_err(a, b) <= GATE, what


@pytest.mark.parametrize("H,F,NQ", SHAPES)
@pytest.mark.parametrize("last", [False, True])
def test_decode_layer_matches_per_projection_calls(pkg, dev, H, F, NQ, last):
    import torch
    L = _layer(pkg, dev, H, F, NQ, seed=H + NQ)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        res_f, qkv_f = pkg.decode_layer(L["attn"], L["h"], L["o"], L["n2"], L["g"], L["u"], L["d"],
                                        EPS, next_norm=None if last else L["n1"],
                                        next_qkv=None if last else L["q"], stream=s)
    s.synchronize()
    assert pkg.decode_layer_faults(s) == 0
    h2, qkv, d = _unfused(pkg, L, H, F, NQ, last)
    torch.cuda.synchronize()
    # residual stream: the down projection carries the two-path allowance
    _two_paths(res_f, h2, TOL_GEMV, f"residual_out H={H} last={last}", ref_scale=d)
    if last:
        assert qkv_f is None
    else:
        _two_paths(qkv_f, qkv, TOL_GEMV, f"next q|k|v H={H}")


def test_decode_layer_matches_oracle_pipeline(pkg, dev):
    """Llama-3.2-1B shapes (hidden 2048, ffn 8192, 3072 q|k|v rows) against
    the numpy pipeline: o = half(attn.Wo); residualRmsNorm; act =
    half(silu(g) * u); h2 = half(h1 + half(act.Wd)); rmsNorm(h2).Wqkv.

    The residual stream goes through three chained matmuls, so its allowance
    is propagated: one fp16 ulp per rounding point (o, h1, d, h2), the GEMV
    bound of each product, and the error of act carried through the 8192-term
    down products as a 4-sigma random walk (independent roundings).  act's
    error is its GEMV bound plus the effect of the normalized vector, each of
    whose elements may differ from the oracle's by one fp16 ulp (its sum of
    squares is fp32), again as a 4-sigma walk through gate and up.  The q|k|v
    phase is checked on its own, against the oracle fed the kernel's residual
    stream."""
    import torch
    H, F, NQ = 2048, 8192, 3072
    L = _layer(pkg, dev, H, F, NQ, seed=77)
    res_f, qkv_f = pkg.decode_layer(L["attn"], L["h"], L["o"], L["n2"], L["g"], L["u"], L["d"], EPS,
                                    next_norm=L["n1"], next_qkv=L["q"])
    torch.cuda.synchronize()
    assert pkg.decode_layer_faults() == 0
    W = {k: (host(L[k].weight), host(L[k].scales), host(L[k].biases)) for k in "ougdq"}
    lin = lambda x, k: o.matmul_q4_f64(x, *W[k], 64)
    sq = lambda k: o.dequant_f64(*W[k], 64) ** 2
    ulp = lambda v: np.spacing(np.abs(np.asarray(v, np.float64)).astype(np.float16)).astype(np.float64)
    bound = lambda v: TOL_GEMV["rtol"] * np.abs(v) + TOL_GEMV["atol_rms"] * np.sqrt(np.mean(v ** 2))
    attn, h = host(L["attn"]), host(L["h"])
    n2, n1 = L["n2"].cpu().numpy(), L["n1"].cpu().numpy()
    ov = lin(attn, "o")
    res, xn2 = o.residual_rms_norm_ref(h, ov.astype(np.float16), n2, EPS)
    gv, uv = lin(xn2, "g"), lin(xn2, "u")
    a64 = o.silu_mul_f64(gv, uv)
    act = a64.astype(np.float16)
    dv = lin(act, "d")
    h2 = o.residual_add_ref(res, dv)
    got_h2 = res_f.float().cpu().numpy().astype(np.float64)
    assert o.max_rel_err(got_h2, h2.astype(np.float64)) <= GATE
    dn2 = ulp(xn2)[0] ** 2
    err_g = bound(gv) + 4 * np.sqrt(sq("g") @ dn2)
    err_u = bound(uv) + 4 * np.sqrt(sq("u") @ dn2)
    sig = 1.0 / (1.0 + np.exp(-gv))
    err_act = (np.abs(uv * sig * (1 + gv * (1 - sig))) * err_g + np.abs(gv * sig) * err_u
               + ulp(act))
    prop = 4 * np.sqrt(sq("d") @ (err_act[0] ** 2))
    allow = ulp(ov) + bound(ov) + ulp(res) + ulp(dv) + bound(dv) + prop + ulp(h2)
    dd = np.abs(got_h2 - h2.astype(np.float64))
    assert np.all(dd <= allow), f"residual stream: worst {np.max(dd / allow):.2f}x the allowance"
    # Q phase on its own: the oracle fed the kernel's residual stream
    qkv_own = lin(o.rms_norm_ref(res_f.cpu().numpy(), n1, EPS), "q")
    got_q = qkv_f.float().cpu().numpy().astype(np.float64)
    assert_parity(got_q, qkv_own, TOL_GEMV, "next q|k|v")
    assert o.max_rel_err(got_q, lin(o.rms_norm_ref(h2, n1, EPS), "q")) <= GATE


def test_decode_layer_in_place_chain_and_graph(pkg, dev):
    """Three layers chained as a decode loop calls them: the residual stream
    updated in place and each layer's attention stand-in a view of the q|k|v
    the previous call wrote.  In place equals out of place bit for bit, and a
    graph of the chain replays the eager chain exactly (eager work and
    synchronisation between replays)."""
    import torch
    H, F, NQ = 3072, 8192, 5120
    layers = [_layer(pkg, dev, H, F, NQ, seed=100 + i) for i in range(3)]
    for L in layers:   # norm weights ~0.05 keep the random-weight stream inside fp16
        L["n1"].mul_(0.05)
        L["n2"].mul_(0.05)
    qkv0 = torch.randn(1, NQ, device=dev).half()
    h0 = (4.0 * torch.randn(1, H, device=dev)).half()
    same = lambda a, b: torch.equal(a.view(torch.int16), b.view(torch.int16))

    def chain(h, qkv, stream, in_place):
        for i, L in enumerate(layers):
            nxt = layers[(i + 1) % 3]
            attn = qkv[:, :H]
            if in_place:
                pkg.decode_layer(attn, h, L["o"], L["n2"], L["g"], L["u"], L["d"], EPS,
                                 next_norm=nxt["n1"], next_qkv=nxt["q"], residual_out=h,
                                 next_qkv_out=qkv, stream=stream)
            else:
                h2, q2 = pkg.decode_layer(attn.contiguous(), h, L["o"], L["n2"], L["g"], L["u"],
                                          L["d"], EPS, next_norm=nxt["n1"], next_qkv=nxt["q"],
                                          stream=stream)
                h, qkv = h2, q2
        return h, qkv

    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        h_ref, q_ref = chain(h0.clone(), qkv0.clone(), s, in_place=False)
        h, qkv = h0.clone(), qkv0.clone()
        chain(h, qkv, s, in_place=True)
    s.synchronize()
    assert torch.isfinite(h_ref).all() and torch.isfinite(q_ref).all()
    assert same(h, h_ref) and same(qkv, q_ref)
    # graph of the in-place chain, captured on the stream that ran it eagerly
    hb, qb = h0.clone(), qkv0.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        chain(hb, qb, s, in_place=True)
    for rep in range(3):
        hb.copy_(h0)
        qb.copy_(qkv0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert same(hb, h_ref) and same(qb, q_ref), rep
        with torch.cuda.stream(s):
            chain(h0.clone(), qkv0.clone(), s, in_place=False)   # eager work between replays
        s.synchronize()
    assert pkg.decode_layer_faults(s) == 0


def test_decode_layer_unsupported_shape(pkg, dev):
    import torch
    H, F = 256, 512
    _, [wo] = gpu_inputs(1, H, H, 64, seed=1, dev=dev)
    _, [wg, wu] = gpu_inputs(1, F, H, 64, seed=2, dev=dev, n_weights=2)
    _, [wd] = gpu_inputs(1, H, F, 64, seed=3, dev=dev)
    Q = lambda t, k: pkg.Q4Weight(*t, k, 64)
    x = torch.randn(1, H, device=dev).half()
    n = torch.ones(H, device=dev)
    with pytest.raises(pkg.SltxError) as ei:
        pkg.decode_layer(x, x, Q(wo, H), n, Q(wg, H), Q(wu, H), Q(wd, F), EPS)
    assert ei.value.code == pkg.SLTX_ERR_UNSUPPORTED


def _synthetic_model(pkg, dev, L=2, H=3072, F=8192, heads=24, kv=8, hd=128, V=4096, seed=300):
    """A Llama-shaped model with random 4-bit weights in ModelWeights' form
    (q|k|v concatenated, tied embedding / lm_head over a small vocabulary)."""
    import torch
    from types import SimpleNamespace
    from swiftltx_amd.weights import LayerWeights
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    Q = lambda N, K, sd: pkg.Q4Weight(*gpu_inputs(1, N, K, 64, seed=sd, dev=dev)[1][0], K, 64)
    norm = lambda: (0.05 * (1.0 + 0.1 * torch.randn(H, generator=gen, device=dev))).float()
    nq = (heads + 2 * kv) * hd
    layers = [LayerWeights(q_proj=None, k_proj=None, v_proj=None, o_proj=Q(H, H, seed + 10 * i),
                           gate_proj=Q(F, H, seed + 10 * i + 1), up_proj=Q(F, H, seed + 10 * i + 2),
                           down_proj=Q(H, F, seed + 10 * i + 3), input_norm_weight=norm(),
                           post_norm_weight=norm(), qkv_proj=Q(nq, H, seed + 10 * i + 4))
              for i in range(L)]
    emb = Q(V, H, seed + 99)
    cfg = SimpleNamespace(hidden_size=H, intermediate_size=F, num_attention_heads=heads,
                          num_key_value_heads=kv, head_dim=hd, vocab_size=V, rms_norm_eps=EPS)
    fnorm = (1.0 + 0.1 * torch.randn(H, generator=gen, device=dev)).float()
    return SimpleNamespace(config=cfg, embed_tokens=emb, lm_head=emb, norm_weight=fnorm,
                           layers=layers)


def test_decode_step_single_launch_layers(pkg, dev):
    """DecodeStep with single_launch_layers (one sltx_decode_layer_q4 launch
    per layer) against the per-projection DecodeStep on a two-layer
    Llama-3.2-3B-shaped model: logits within the two-path allowance of the
    lm_head GEMV (plus the norms' one-ulp effects, bounded by the BASELINE
    gate), the same greedy token where the top two logits are apart, and a
    captured graph replaying the eager tokens."""
    import torch
    from swiftltx_amd.decode import DecodeStep
    mw = _synthetic_model(pkg, dev)
    s = torch.cuda.Stream()
    a = DecodeStep(mw, stream=s)
    b = DecodeStep(mw, stream=s, single_launch_layers=True)
    tok = 11
    toks = []
    for step in range(4):
        with torch.cuda.stream(s):
            a.token.fill_(tok)
            b.token.fill_(tok)
            a.step()
            b.step()
        s.synchronize()
        la = a.logits.float().cpu().numpy().astype(np.float64)
        lb = b.logits.float().cpu().numpy().astype(np.float64)
        assert np.isfinite(la).all()
        assert o.max_rel_err(lb, la) <= GATE, step
        top2 = np.sort(la[0])[-2:]
        if top2[1] - top2[0] > 2e-2 * np.max(np.abs(la)):
            assert int(b.token.item()) == int(a.token.item()), step
        toks.append(int(b.token.item()))
        tok = toks[-1]
    assert pkg.decode_layer_faults(s) == 0
    with torch.cuda.stream(s):
        b.token.fill_(11)
    b.capture()                  # one eager step (11 -> toks[0]) first
    s.synchronize()
    assert int(b.token.item()) == toks[0]
    b.token.fill_(11)
    torch.cuda.synchronize()
    replayed = []
    for _ in range(4):
        b.replay()
        torch.cuda.synchronize()
        replayed.append(int(b.token.item()))
    assert replayed == toks
    assert pkg.decode_layer_faults(s) == 0
