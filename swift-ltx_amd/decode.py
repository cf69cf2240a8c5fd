"""The 4-bit matmul path of Llama decode steps, as device work on one stream.

Mirrors LlamaModel.generate / forward / transformerBlock
(LlamaModel.swift:150-161, 213-236, 284-331) with this library's entry points:

  embeddingQ4 (Ops.swift:189-208)              sltx_embedding_q4, token id read on the device
  per layer:
    rmsNorm + q, k, v linear                   sltx_rmsnorm_matmul_q4 (q|k|v rows concatenated)
    rope, KV cache, attention                  the caller's `attention` (outside this library)
    o linear                                   sltx_linear
    residualRmsNorm + gate, up, siluMul        sltx_residual_rmsnorm_matmul_q4_silu_mul
    down linear + elemAdd                      sltx_matmul_q4_residual (in place on the residual)
  final rmsNorm + lm_head linear               sltx_rmsnorm_matmul_q4
  argmax / sample                              sltx_argmax / sltx_sample_top_p

The chosen token id stays in device memory and is the next step's input, so a
step can be captured once as a HIP graph and replayed per token: greedy
(temperature 0, argmax as the reference uses), or sampled with a SamplerState,
which keeps the seen tokens and the uniform draws in device memory.  Sampling
with host arguments (seen list, u) runs eagerly.

`attention(layer, qkv)` receives the layer index and the [1, q+k+v] fp16
projections and returns the [1, heads * head_dim] fp16 attention output (a
tensor that stays valid until the step ends; a view is fine).  The default is
a stand-in with no attention: the q rows themselves, a view of qkv, so the
data dependency is kept and nothing is launched.
"""
from __future__ import annotations

import random

from . import (Q4Weight, argmax, embedding_q4, linear, matmul_q4_residual,
               rmsnorm_matmul_q4, residual_rmsnorm_matmul_q4_silu_mul, sample, sample_with_state)


def q_rows_attention(q_dim):
    """Stand-in attention: the q projection rows (no RoPE, no cache)."""
    def attention(layer, qkv):
        return qkv[:, :q_dim]
    return attention


class DecodeStep:
    """One decode step over device buffers it owns.

    weights: a ModelWeights (swiftltx_amd.weights) loaded with concat_qkv, or
    any object with the same fields (embed_tokens, lm_head, norm_weight,
    layers[i].{qkv_proj, o_proj, gate_proj, up_proj, down_proj,
    input_norm_weight, post_norm_weight}) and a config with hidden_size,
    intermediate_size, num_attention_heads, num_key_value_heads, head_dim,
    vocab_size, rms_norm_eps."""

    def __init__(self, weights, attention=None, stream=None):
        import torch
        c = weights.config
        self.w = weights
        self.c = c
        self.stream = stream
        self.hidden = c.hidden_size
        self.q_dim = c.num_attention_heads * c.head_dim
        self.qkv_rows = self.q_dim + 2 * c.num_key_value_heads * c.head_dim
        for i, lw in enumerate(weights.layers):
            if lw.qkv_proj is None:
                raise ValueError(f"layer {i}: q|k|v weights not concatenated (load with concat_qkv)")
            for name in ("o_proj", "gate_proj", "up_proj", "down_proj"):
                if not isinstance(getattr(lw, name), Q4Weight):
                    raise ValueError(f"layer {i}: {name} is not a 4-bit weight")
        self.attention = attention or q_rows_attention(self.q_dim)
        dev = weights.embed_tokens.weight.device
        f16 = torch.float16
        self.token = torch.zeros(1, dtype=torch.int32, device=dev)       # input / chosen token
        self.h = torch.empty(1, self.hidden, dtype=f16, device=dev)      # residual stream
        self.qkv = torch.empty(1, self.qkv_rows, dtype=f16, device=dev)
        self.o = torch.empty(1, self.hidden, dtype=f16, device=dev)
        self.act = torch.empty(1, c.intermediate_size, dtype=f16, device=dev)
        self.logits = torch.empty(1, c.vocab_size, dtype=f16, device=dev)
        self.res = torch.empty(1, self.hidden, dtype=f16, device=dev)   # h + attention out
        self.graph = None
        # the zeroed token must be in place before work on self.stream reads it
        torch.cuda.current_stream(dev).synchronize()

    def _select(self, temperature, top_p, repetition_penalty, seen, u, state):
        s = self.stream
        if temperature <= 0:
            argmax(self.logits, out=self.token, stream=s)
        elif state is not None:
            sample_with_state(self.logits, temperature, top_p, repetition_penalty, state,
                              out=self.token, stream=s)
        else:
            sample(self.logits, temperature, top_p, repetition_penalty, seen,
                   random.random() if u is None else u, out=self.token, stream=s)

    def forward(self):
        """Embedding of self.token through the lm_head into self.logits."""
        c, w, s = self.c, self.w, self.stream
        embedding_q4(w.embed_tokens, c.vocab_size, self.token, out=self.h, stream=s)
        self._layers()
        rmsnorm_matmul_q4(self.h, w.norm_weight, c.rms_norm_eps, w.lm_head, c.vocab_size,
                          out=self.logits, stream=s)

    def _layers(self):
        c, w, s = self.c, self.w, self.stream
        K, F, eps = self.hidden, c.intermediate_size, c.rms_norm_eps
        for i, lw in enumerate(w.layers):
            rmsnorm_matmul_q4(self.h, lw.input_norm_weight, eps, lw.qkv_proj, self.qkv_rows,
                              out=self.qkv, stream=s)
            attn = self.attention(i, self.qkv)
            linear(attn, lw.o_proj, 1, self.q_dim, K, out=self.o, stream=s)
            # res = h + o (the residual stream); gate/up read its norm; h = res + down
            residual_rmsnorm_matmul_q4_silu_mul(self.h, self.o, lw.post_norm_weight, eps,
                                                lw.gate_proj, lw.up_proj, F,
                                                residual_out=self.res, out=self.act, stream=s)
            matmul_q4_residual(self.act, lw.down_proj, self.res, 1, K, out=self.h, stream=s)

    def step(self, temperature=0.0, top_p=0.9, repetition_penalty=1.1, seen=None, u=None,
             state=None):
        """Run one step eagerly: self.token -> logits -> next token in self.token.
        temperature > 0 samples, with `state` (a SamplerState) if given, else
        with the host's seen tokens and draw u."""
        self.forward()
        self._select(temperature, top_p, repetition_penalty, seen, u, state)
        return self.token

    def capture(self, temperature=0.0, top_p=0.9, repetition_penalty=1.1, state=None):
        """Capture one step as a HIP graph on self.stream (a torch stream;
        required): greedy, or sampled from `state` (a SamplerState, required
        when temperature > 0).  Runs one eager step there first, which
        consumes a token, a draw and a history entry like any other step."""
        import torch
        if self.stream is None:
            raise ValueError("capture needs a dedicated stream")
        if temperature > 0 and state is None:
            raise ValueError("a sampled step in a graph needs a SamplerState")
        kw = dict(temperature=temperature, top_p=top_p, repetition_penalty=repetition_penalty,
                  state=state)
        with torch.cuda.stream(self.stream):
            self.step(**kw)
        self.stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=self.stream):
            self.step(**kw)
        self.graph = g
        return g

    def replay(self):
        """One captured step, enqueued on the current stream.  Replays and eager
        steps of one object share its buffers and the capture stream's
        workspace: the caller keeps them in order (one stream, or
        synchronization between them).  Moving the replay onto the capture
        stream with cross-stream waits around it cost ~130 us per decode
        token."""
        if self.graph is None:
            raise RuntimeError("capture() first")
        self.graph.replay()
        return self.token
