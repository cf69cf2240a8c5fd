"""A whole greedy decode step (swiftltx_amd.decode.DecodeStep) on a small
MLX-4bit Llama (two layers, two safetensors shards, tied lm_head) against the
same pipeline run in numpy from the oracle's functions
(LlamaModel.swift:213-236, 284-331; attention replaced on both sides by the
q rows, as DecodeStep's stand-in does):

* each step's logits within the parity gate (max|d|/max|ref| <= 1e-2) of the
  numpy pipeline fed the same token, and the same argmax wherever the
  reference's top two logits are further apart than that;
* graph replays reproduce the eager token sequence exactly.
"""
import numpy as np
import pytest

from oracle import q4_oracle as o
from test_gpu_loader import CFG, _write_model

pytestmark = pytest.mark.gpu


def _bf16(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _ref_logits(src, tok):
    c = CFG
    eps, g = c["rms_norm_eps"], 64
    qd = c["num_attention_heads"] * c["head_dim"]
    lin = lambda x, p: o.matmul_q4_f64(x, src[p + ".weight"], src[p + ".scales"],
                                       src[p + ".biases"], g)
    e = "model.embed_tokens"
    h = o.embedding_q4_ref(src[e + ".weight"], src[e + ".scales"], src[e + ".biases"], [tok], g)
    for i in range(c["num_hidden_layers"]):
        p = f"model.layers.{i}"
        xn = o.rms_norm_ref(h, src[p + ".input_layernorm.weight"], eps)
        qkv = np.concatenate([lin(xn, f"{p}.self_attn.{x}_proj") for x in "qkv"], axis=1)
        attn = qkv.astype(np.float16)[:, :qd]
        ov = lin(attn, f"{p}.self_attn.o_proj")
        res, xn2 = o.residual_rms_norm_ref(h, ov.astype(np.float16),
                                           _bf16(src[p + ".post_attention_layernorm.weight"]), eps)
        act = o.silu_mul_f64(lin(xn2, f"{p}.mlp.gate_proj"), lin(xn2, f"{p}.mlp.up_proj"))
        h = o.residual_add_ref(res, lin(act.astype(np.float16), f"{p}.mlp.down_proj"))
    xn = o.rms_norm_ref(h, src["model.norm.weight"].astype(np.float32), eps)
    return lin(xn, e)[0]


def test_decode_steps_match_numpy_and_graph(pkg, dev, tmp_path):
    import torch
    from swiftltx_amd.decode import DecodeStep
    from swiftltx_amd.weights import ModelWeights
    src = _write_model(tmp_path)
    mw = ModelWeights.from_directory(str(tmp_path), device=dev)
    s = torch.cuda.Stream()
    ds = DecodeStep(mw, stream=s)
    tokens = []
    tok = 7
    for step in range(5):
        with torch.cuda.stream(s):
            ds.token.fill_(tok)
            ds.step()
        s.synchronize()
        logits = ds.logits[0].float().cpu().numpy()
        got = int(ds.token.item())
        ref = _ref_logits(src, tok)
        err = np.max(np.abs(logits - ref)) / np.max(np.abs(ref))
        assert err <= 1e-2, (step, err)
        top2 = np.sort(ref)[-2:]
        if top2[1] - top2[0] > 2e-2 * np.max(np.abs(ref)):
            assert got == int(np.argmax(ref)), (step, got, int(np.argmax(ref)))
        assert got == o.argmax_ref(logits.astype(np.float16)), step
        tokens.append(got)
        tok = got
    # the captured greedy step replays the same sequence from the same start
    with torch.cuda.stream(s):
        ds.token.fill_(7)
    ds.capture()                  # runs one eager step (7 -> tokens[0]) on the stream first
    s.synchronize()
    assert int(ds.token.item()) == tokens[0]
    ds.token.fill_(7)
    torch.cuda.synchronize()
    replayed = []
    for _ in range(5):
        ds.replay()
        torch.cuda.synchronize()
        replayed.append(int(ds.token.item()))
    assert replayed == tokens


def test_decode_sampled_graph_matches_eager(pkg, dev, tmp_path):
    """A sampled step (temperature 0.9, top-p 0.95, penalty 1.2) with the
    seen tokens and draws in a SamplerState: each eager step's token is the
    host-argument sampler's on the same logits with the history so far and
    that step's draw; a captured step replays the eager sequence exactly
    from the same start, its history growing on the device."""
    import torch
    from swiftltx_amd.decode import DecodeStep
    from swiftltx_amd.weights import ModelWeights
    _write_model(tmp_path)
    mw = ModelWeights.from_directory(str(tmp_path), device=dev)
    s = torch.cuda.Stream()
    ds = DecodeStep(mw, stream=s)
    draws = np.random.default_rng(40).random(16).astype(np.float32)
    prompt = [7, 3, 7]
    kw = dict(temperature=0.9, top_p=0.95, repetition_penalty=1.2)
    st = pkg.SamplerState(32, draws=draws, history=prompt, device=dev)
    tokens = []
    with torch.cuda.stream(s):
        ds.token.fill_(7)
    for step in range(6):
        with torch.cuda.stream(s):
            ds.step(state=st, **kw)
        s.synchronize()
        got = int(ds.token.item())
        seen = torch.tensor(prompt + tokens, dtype=torch.int32, device=dev)
        host = int(pkg.sample(ds.logits[0], u=float(draws[step]), seen_tokens=seen, **kw).item())
        assert got == host, (step, got, host)
        tokens.append(got)
    assert st.tokens() == prompt + tokens
    replay_state = pkg.SamplerState(32, draws=draws, history=prompt, device=dev)
    with torch.cuda.stream(s):
        ds.token.fill_(7)
    ds.capture(state=replay_state, **kw)    # one eager step first: 7 -> tokens[0]
    s.synchronize()
    replayed = [int(ds.token.item())]
    for _ in range(5):
        ds.replay()
        torch.cuda.synchronize()
        replayed.append(int(ds.token.item()))
    assert replayed == tokens
    assert replay_state.tokens() == prompt + tokens
    with pytest.raises(ValueError):
        ds.capture(temperature=0.5)          # sampling in a graph needs a SamplerState
