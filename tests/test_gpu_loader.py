"""Device reads of safetensors weights and the ModelWeights mirror on the GPU.

* sltx_st_read_device: bit-exact against the host read for every dtype,
  including a tensor larger than the 16 MB staging chunk with an odd size;
* sltx_st_read_device_f32: F16 (normals, subnormals, +-0, inf, NaN), BF16 and
  F32 widened exactly as numpy widens them (loadFloat, ModelWeights.swift:96-108);
* ModelWeights (ModelWeights.swift:40-154) on a small MLX-4bit Llama directory
  written here in two shards: every 4-bit linear, norm and the tied lm_head
  land byte-exact on the device, q|k|v concatenate by rows, and the loaded
  weights drive the kernels (embedding gather, norm + q|k|v GEMV) to the
  oracle's results.
"""
import json
import os

import numpy as np
import pytest

from helpers import TOL_GEMV, assert_parity
from oracle import q4_oracle as o
from test_safetensors import write_st

pytestmark = pytest.mark.gpu


def _dev_bytes(t):
    import torch
    return t.contiguous().view(torch.uint8).cpu().numpy().tobytes()


def test_read_device_every_dtype(pkg, dev, tmp_path):
    import torch
    rng = np.random.default_rng(3)
    arrays = {"f32": ("F32", rng.standard_normal((33, 7)).astype(np.float32)),
              "f16": ("F16", rng.standard_normal((5, 9)).astype(np.float16)),
              "bf16": ("BF16", rng.integers(0, 65535, (6,)).astype(np.uint16)),
              "i8": ("I8", rng.integers(-128, 127, (17,)).astype(np.int8)),
              "u8": ("U8", rng.integers(0, 255, (3, 3)).astype(np.uint8)),
              "i32": ("I32", rng.integers(-9, 9, (4,)).astype(np.int32)),
              "u32": ("U32", rng.integers(0, 2**32 - 1, (8, 2), dtype=np.uint64).astype(np.uint32))}
    path = write_st(tmp_path / "d.safetensors",
                    {k: (dt, a.shape, a.tobytes()) for k, (dt, a) in arrays.items()})
    f = pkg.SafeTensorsFile(path)
    for name, (dt, a) in arrays.items():
        t = torch.empty(a.nbytes, dtype=torch.uint8, device=dev)
        f.read_device(name, t)
        assert _dev_bytes(t) == a.tobytes(), name


def test_read_device_multi_chunk(pkg, dev, tmp_path):
    """40 MB + 6 bytes: three staging chunks, the last partial; read into an
    offset of a larger allocation."""
    import torch
    rng = np.random.default_rng(4)
    a = rng.integers(0, 255, 40 * 2 ** 20 + 6).astype(np.uint8)
    path = write_st(tmp_path / "big.safetensors", {"big": ("U8", a.shape, a.tobytes())})
    f = pkg.SafeTensorsFile(path)
    t = torch.zeros(a.nbytes + 64, dtype=torch.uint8, device=dev)
    f.read_device("big", t, byte_offset=32)
    host = t.cpu().numpy()
    assert np.array_equal(host[32:32 + a.nbytes], a)
    assert not host[:32].any() and not host[32 + a.nbytes:].any()


def test_read_device_f32(pkg, dev, tmp_path):
    import torch
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 6.0e-8, -3.0e-6, 65504.0, 1.0],
                       dtype=np.float16)
    h = np.concatenate([special, np.random.default_rng(5).standard_normal(1000).astype(np.float16)])
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    bf = np.random.default_rng(6).integers(0, 65535, 999).astype(np.uint16)
    f32 = np.random.default_rng(7).standard_normal(77).astype(np.float32)
    path = write_st(tmp_path / "f.safetensors",
                    {"h": ("F16", h.shape, h.tobytes()), "allh": ("F16", allh.shape, allh.tobytes()),
                     "bf": ("BF16", bf.shape, bf.tobytes()), "f32": ("F32", f32.shape, f32.tobytes())})
    f = pkg.SafeTensorsFile(path)
    for name, ref in (("h", h.astype(np.float32)), ("allh", allh.astype(np.float32)),
                      ("bf", (bf.astype(np.uint32) << 16).view(np.float32)), ("f32", f32)):
        t = torch.empty(ref.size, dtype=torch.float32, device=dev)
        f.read_device_f32(name, t)
        got = t.cpu().numpy()
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(got), nan), name
        assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32)), name


# ----------------------------------------------------------- model directory --

CFG = dict(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
           num_key_value_heads=2, head_dim=64, vocab_size=300, max_position_embeddings=2048,
           rms_norm_eps=1e-5, rope_theta=500000.0, tie_word_embeddings=True,
           quantization={"group_size": 64, "bits": 4})


def _q4(rng, N, K, g=64):
    q = rng.integers(0, 16, (N, K))
    s = (np.abs(rng.standard_normal((N, K // g))) * 0.02).astype(np.float16)
    b = (-8 * s.astype(np.float32)).astype(np.float16)
    return o.pack_q4(q), s, b


def _write_model(root, bf16_k_scales=False):
    rng = np.random.default_rng(8)
    c = CFG
    h, F, V = c["hidden_size"], c["intermediate_size"], c["vocab_size"]
    qd = c["num_attention_heads"] * c["head_dim"]
    kvd = c["num_key_value_heads"] * c["head_dim"]
    t = {}

    def lin(prefix, N, K):
        w, s, b = _q4(rng, N, K)
        t[prefix + ".weight"], t[prefix + ".scales"], t[prefix + ".biases"] = w, s, b

    lin("model.embed_tokens", V, h)
    t["model.norm.weight"] = rng.standard_normal(h).astype(np.float16)   # f16 on disk
    for i in range(c["num_hidden_layers"]):
        p = f"model.layers.{i}"
        lin(f"{p}.self_attn.q_proj", qd, h)
        lin(f"{p}.self_attn.k_proj", kvd, h)
        lin(f"{p}.self_attn.v_proj", kvd, h)
        lin(f"{p}.self_attn.o_proj", h, qd)
        lin(f"{p}.mlp.gate_proj", F, h)
        lin(f"{p}.mlp.up_proj", F, h)
        lin(f"{p}.mlp.down_proj", h, F)
        t[f"{p}.input_layernorm.weight"] = rng.standard_normal(h).astype(np.float32)
        bfn = rng.integers(0x3F00, 0x3FC0, h).astype(np.uint16)   # bf16 bits near 1
        t[f"{p}.post_attention_layernorm.weight"] = bfn
    names = sorted(t)
    dt = {np.dtype(np.uint32): "U32", np.dtype(np.float16): "F16", np.dtype(np.float32): "F32"}
    half = len(names) // 2
    for k, part in enumerate((names[:half], names[half:])):
        write_st(root / f"model-0000{k + 1}-of-00002.safetensors",
                 {n: ("BF16" if n.endswith("post_attention_layernorm.weight")
                      or (bf16_k_scales and n == "model.layers.0.self_attn.k_proj.scales")
                      else dt[t[n].dtype], t[n].shape, t[n].tobytes()) for n in part},
                 metadata={"format": "mlx"})
    (root / "config.json").write_text(json.dumps(c))
    return t


def test_model_weights_directory(pkg, dev, tmp_path):
    import torch
    from swiftltx_amd.weights import ModelWeights
    src = _write_model(tmp_path)
    mw = ModelWeights.from_directory(str(tmp_path), device=dev)
    assert mw.is_quantized and len(mw.files) == 2
    assert mw.lm_head is mw.embed_tokens   # tied (no lm_head.weight)
    emb = mw.embed_tokens
    assert (emb.K, emb.group_size) == (256, 64)
    assert _dev_bytes(emb.weight) == src["model.embed_tokens.weight"].tobytes()
    assert np.array_equal(mw.norm_weight.cpu().numpy(), src["model.norm.weight"].astype(np.float32))
    for i, lw in enumerate(mw.layers):
        p = f"model.layers.{i}"
        for attr, name in (("q_proj", "self_attn.q_proj"), ("k_proj", "self_attn.k_proj"),
                           ("v_proj", "self_attn.v_proj"), ("o_proj", "self_attn.o_proj"),
                           ("gate_proj", "mlp.gate_proj"), ("up_proj", "mlp.up_proj"),
                           ("down_proj", "mlp.down_proj")):
            w = getattr(lw, attr)
            for part, field in (("weight", w.weight), ("scales", w.scales), ("biases", w.biases)):
                assert _dev_bytes(field) == src[f"{p}.{name}.{part}"].tobytes(), (attr, part)
        assert np.array_equal(lw.input_norm_weight.cpu().numpy(), src[f"{p}.input_layernorm.weight"])
        bf = (src[f"{p}.post_attention_layernorm.weight"].astype(np.uint32) << 16).view(np.float32)
        assert np.array_equal(lw.post_norm_weight.cpu().numpy(), bf)
        for part, field in (("weight", lw.qkv_proj.weight), ("scales", lw.qkv_proj.scales),
                            ("biases", lw.qkv_proj.biases)):
            cat = np.concatenate([src[f"{p}.self_attn.{x}_proj.{part}"] for x in "qkv"])
            assert _dev_bytes(field) == cat.tobytes()

    # the loaded weights drive the kernels
    ids = np.array([0, 5, 299, 17], dtype=np.int32)
    e = pkg.embedding_q4(emb, CFG["vocab_size"], torch.from_numpy(ids).to(dev))
    ref = o.embedding_q4_ref(src["model.embed_tokens.weight"], src["model.embed_tokens.scales"],
                             src["model.embed_tokens.biases"], ids, 64)
    torch.cuda.synchronize()
    assert np.array_equal(e.cpu().numpy(), ref)
    x = e[1:2].contiguous()
    lw = mw.layers[0]
    N = lw.qkv_proj.weight.shape[0]
    y = pkg.rmsnorm_matmul_q4(x, lw.input_norm_weight, 1e-5, lw.qkv_proj, N)
    torch.cuda.synchronize()
    xn = o.rms_norm_ref(ref[1:2], src["model.layers.0.input_layernorm.weight"], 1e-5)
    wq = np.concatenate([src[f"model.layers.0.self_attn.{x}_proj.weight"] for x in "qkv"])
    sq = np.concatenate([src[f"model.layers.0.self_attn.{x}_proj.scales"] for x in "qkv"])
    bq = np.concatenate([src[f"model.layers.0.self_attn.{x}_proj.biases"] for x in "qkv"])
    assert_parity(y.cpu().numpy(), o.matmul_q4_f64(xn, wq, sq, bq, 64), TOL_GEMV, "loaded qkv")


def test_concat_rejects_mismatched_part(pkg, dev, tmp_path):
    """q|k|v concatenation reads every part by byte offset into one weight, so
    a part whose scales are not F16 (here k_proj's tagged BF16) must be
    rejected, not copied at the wrong row width."""
    from swiftltx_amd.weights import ModelWeights
    _write_model(tmp_path, bf16_k_scales=True)
    with pytest.raises(ValueError, match="k_proj.scales"):
        ModelWeights.from_directory(str(tmp_path), device=dev)
