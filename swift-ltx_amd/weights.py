"""Host mirror of swift-ltx's model configuration and 4-bit weight loader.

ModelConfig   <- ModelConfig (ModelConfig.swift:5-73), parsed from config.json
ModelWeights  <- ModelWeights(config:files:) (ModelWeights.swift:40-154)

The weights land in device memory (torch tensors on the GPU) through the
native safetensors reader (include/swiftltx_q4.h, sltx_st_*):
  * a 4-bit linear (its ".scales" exists) becomes a Q4Weight with the raw
    uint32 / fp16 bytes (loadLinear, ModelWeights.swift:111-122) -- the layout
    the kernels read, so nothing is repacked;
  * norm weights are widened to fp32 (loadFloat, ModelWeights.swift:96-108);
  * the lm_head falls back to the embedding when "lm_head.weight" is absent
    (tied, ModelWeights.swift:126-130);
  * optionally (concat_qkv) q, k and v rows are read into one [q+k+v, K/8]
    weight (with matching scales/biases), so a decode layer's three
    projections are one launch.
Float (non-quantized) linears load as fp32 device tensors; their matmul is the
reference's CPU path (LlamaModel.swift:478-493), outside this library.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field
from typing import Optional

from . import Q4Weight, SafeTensorsFile, load_safetensors


@dataclass
class QuantizationConfig:
    group_size: int
    bits: int


@dataclass
class ModelConfig:
    """ModelConfig (ModelConfig.swift:5-73); keys as in HuggingFace config.json.
    head_dim defaults to hidden_size / num_attention_heads when absent (the
    reference requires the key)."""
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    vocab_size: int
    max_position_embeddings: int = 0
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    head_dim: int = 0
    tie_word_embeddings: bool = False
    quantization: Optional[QuantizationConfig] = None
    rope_scaling: Optional[dict] = None

    @classmethod
    def from_dict(cls, d: dict) -> "ModelConfig":
        q = d.get("quantization")
        heads = int(d["num_attention_heads"])
        return cls(
            hidden_size=int(d["hidden_size"]),
            intermediate_size=int(d["intermediate_size"]),
            num_hidden_layers=int(d["num_hidden_layers"]),
            num_attention_heads=heads,
            num_key_value_heads=int(d["num_key_value_heads"]),
            vocab_size=int(d["vocab_size"]),
            max_position_embeddings=int(d.get("max_position_embeddings", 0)),
            rms_norm_eps=float(d.get("rms_norm_eps", 1e-5)),
            rope_theta=float(d.get("rope_theta", 10000.0)),
            head_dim=int(d.get("head_dim", int(d["hidden_size"]) // heads)),
            tie_word_embeddings=bool(d.get("tie_word_embeddings", False)),
            quantization=(QuantizationConfig(int(q["group_size"]), int(q["bits"]))
                          if q else None),
            rope_scaling=d.get("rope_scaling"),
        )

    @classmethod
    def from_file(cls, path) -> "ModelConfig":
        with open(path) as f:
            return cls.from_dict(json.load(f))

    @property
    def kv_repeat_factor(self) -> int:
        """kvRepeatFactor (ModelConfig.swift:71-72)."""
        return self.num_attention_heads // self.num_key_value_heads


@dataclass
class LayerWeights:
    """LayerWeights (ModelWeights.swift:14-30) plus the optional q|k|v weight."""
    q_proj: object
    k_proj: object
    v_proj: object
    o_proj: object
    gate_proj: object
    up_proj: object
    down_proj: object
    input_norm_weight: object
    post_norm_weight: object
    qkv_proj: Optional[Q4Weight] = None


class ModelWeights:
    """ModelWeights(config:files:) (ModelWeights.swift:40-154)."""

    def __init__(self, config: ModelConfig, files, device="cuda", concat_qkv=True,
                 stream=None):
        import torch
        self.config = config
        self.files = files
        self.device = torch.device(device)
        self._stream = stream
        first = "model.layers.0.self_attn.q_proj"
        # quantization detection (ModelWeights.swift:43-52)
        self.is_quantized = any(
            (first + ".weight") in f.tensors and
            (f.tensors[first + ".weight"].dtype in ("U8", "I8") or (first + ".scales") in f.tensors)
            for f in files)
        c = config
        self.embed_tokens = self.load_linear("model.embed_tokens", c.hidden_size)
        self.norm_weight = self.load_float("model.norm.weight")
        self.lm_head = (self.load_linear("lm_head", c.hidden_size)
                        if self.exists("lm_head.weight") else self.embed_tokens)
        qdim = c.num_attention_heads * c.head_dim
        self.layers = []
        for i in range(c.num_hidden_layers):
            p = f"model.layers.{i}"
            h = c.hidden_size
            lw = LayerWeights(
                q_proj=self.load_linear(f"{p}.self_attn.q_proj", h),
                k_proj=self.load_linear(f"{p}.self_attn.k_proj", h),
                v_proj=self.load_linear(f"{p}.self_attn.v_proj", h),
                o_proj=self.load_linear(f"{p}.self_attn.o_proj", qdim),
                gate_proj=self.load_linear(f"{p}.mlp.gate_proj", h),
                up_proj=self.load_linear(f"{p}.mlp.up_proj", h),
                down_proj=self.load_linear(f"{p}.mlp.down_proj", c.intermediate_size),
                input_norm_weight=self.load_float(f"{p}.input_layernorm.weight"),
                post_norm_weight=self.load_float(f"{p}.post_attention_layernorm.weight"))
            if concat_qkv and isinstance(lw.q_proj, Q4Weight):
                lw.qkv_proj = self.load_linear_concat(
                    [f"{p}.self_attn.q_proj", f"{p}.self_attn.k_proj", f"{p}.self_attn.v_proj"], h)
            self.layers.append(lw)

    @classmethod
    def from_directory(cls, directory, device="cuda", concat_qkv=True) -> "ModelWeights":
        config = ModelConfig.from_file(os.path.join(directory, "config.json"))
        return cls(config, load_safetensors(directory), device, concat_qkv)

    # -- helpers mirroring the reference's closures --------------------------

    def _find(self, name) -> SafeTensorsFile:
        for f in self.files:
            if name in f.tensors:
                return f
        raise KeyError(f"Weight not found: {name}")

    def exists(self, name) -> bool:
        return any(name in f.tensors for f in self.files)

    def _torch_dtype(self, code):
        import torch
        return {"F32": torch.float32, "F16": torch.float16, "BF16": torch.bfloat16,
                "I8": torch.int8, "U8": torch.uint8, "I32": torch.int32,
                "U32": torch.int32}[code]

    def load_raw(self, name):
        """loadRaw (ModelWeights.swift:58-92) for integer / fp16 tensors: raw
        bytes to the device (U32 held as int32)."""
        import torch
        f = self._find(name)
        info = f.tensors[name]
        t = torch.empty(info.shape, dtype=self._torch_dtype(info.dtype), device=self.device)
        f.read_device(name, t, stream=self._stream)
        return t

    def load_float(self, name):
        """loadFloat (ModelWeights.swift:96-108): fp32 on the device."""
        import torch
        f = self._find(name)
        info = f.tensors[name]
        t = torch.empty(info.shape, dtype=torch.float32, device=self.device)
        f.read_device_f32(name, t, stream=self._stream)
        return t

    def _group(self, prefix, K, scales_shape):
        """Group size: the config's (default 64, ModelWeights.swift:117), checked
        against the scales' shape."""
        g = self.config.quantization.group_size if self.config.quantization else 64
        groups = scales_shape[-1]
        if groups * g != K:
            raise ValueError(f"{prefix}: {groups} groups of {g} do not cover K = {K}")
        return g

    def load_linear(self, prefix, K):
        """loadLinear (ModelWeights.swift:111-122)."""
        if not self.exists(f"{prefix}.scales"):
            return self.load_float(f"{prefix}.weight")
        w = self.load_raw(f"{prefix}.weight")
        s = self.load_raw(f"{prefix}.scales")
        b = self.load_raw(f"{prefix}.biases")
        if w.shape[-1] * 8 != K:
            raise ValueError(f"{prefix}: packed width {w.shape[-1]} x 8 != K = {K}")
        return Q4Weight(w, s, b, K, self._group(prefix, K, tuple(s.shape)))

    def load_linear_concat(self, prefixes, K):
        """Rows of several 4-bit linears with the same K and group size read
        into one weight (row-major [N, K/8], so rows concatenate by byte
        offset); used for q|k|v."""
        import torch
        infos = []
        for p in prefixes:
            parts = [(self._find(f"{p}.{n}"), f"{p}.{n}") for n in ("weight", "scales", "biases")]
            infos.append(parts)
        rows = [parts[0][0].tensors[parts[0][1]].shape[0] for parts in infos]
        N = sum(rows)
        sshape = infos[0][1][0].tensors[infos[0][1][1]].shape
        g = self._group("+".join(prefixes), K, sshape)
        w = torch.empty((N, K // 8), dtype=torch.int32, device=self.device)
        s = torch.empty((N, K // g), dtype=torch.float16, device=self.device)
        b = torch.empty((N, K // g), dtype=torch.float16, device=self.device)
        # Every part must have the destination's row layout: packed I32/U32
        # words of width K/8 and F16 scales/biases with K/g groups, and the
        # same row count in all three tensors (else its rows would land at
        # the wrong byte offsets with no error).
        want = (({"I32", "U32"}, K // 8 * 4), ({"F16"}, K // g * 2), ({"F16"}, K // g * 2))
        for parts, n in zip(infos, rows):
            for (f, name), (dtypes, row_bytes) in zip(parts, want):
                info = f.tensors[name]
                if info.dtype not in dtypes:
                    raise ValueError(f"{name}: dtype {info.dtype}, expected {sorted(dtypes)}")
                if len(info.shape) != 2 or info.shape[0] != n:
                    raise ValueError(f"{name}: shape {info.shape}, expected {n} rows")
                if info.byte_count != n * row_bytes:
                    raise ValueError(f"{name}: {info.byte_count} bytes, expected {n} rows of "
                                     f"{row_bytes} bytes")
        r0 = 0
        for parts, n in zip(infos, rows):
            for (f, name), t in zip(parts, (w, s, b)):
                row_bytes = t.shape[1] * t.element_size()
                f.read_device(name, t, byte_offset=r0 * row_bytes, stream=self._stream)
            r0 += n
        return Q4Weight(w, s, b, K, g)
