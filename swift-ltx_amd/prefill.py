"""The 4-bit matmul path of a Llama prefill (a prompt of S tokens in one
batched pass), as device work on one stream.

Mirrors LlamaModel.prefill / transformerBlockBatch (LlamaModel.swift:168-203,
230-282) with this library's entry points:

  embeddingQ4Batch (Ops.swift:163-185)          sltx_embedding_q4, S device token ids
  per layer:
    rmsNorm                                     layer 0: sltx_rms_norm (all S rows); later
                                                layers: the previous down step's call
    q, k, v linear                              sltx_linear, fast (GEMM; q|k|v rows concatenated)
    RoPE, KV cache append, attention            the caller's `attention` (outside this library)
    o linear + residualRmsNorm                  sltx_matmul_q4_residual_rms_norm (unrounded sum)
    gate, up linear + siluMul                   sltx_matmul_q4_silu_mul (GEMM, fused epilogue)
    down linear + elemAdd (+ next rmsNorm)      sltx_matmul_q4_residual_rms_norm (rounded sum,
                                                the next layer's input norm); last layer:
                                                sltx_matmul_q4_residual (GEMM, residual epilogue)
  final rmsNorm + lm_head on the last row       sltx_rmsnorm_matmul_q4 (GEMV)

The reference normalizes all S rows before slicing the last one
(LlamaModel.swift:191-195); only the last row reaches the lm_head, so here the
norm runs on that row alone, fused into the lm_head's GEMV.

`attention(layer, qkv)` receives the layer index and the [S, q+k+v] fp16
projections and returns the [S, heads * head_dim] fp16 attention output
(row-contiguous).  The default stand-in has no attention: a copy of the q
columns (torch; it is not part of this path), so every row depends on its own
token only.
"""
from __future__ import annotations

from . import (Q4Weight, embedding_q4, linear, matmul_q4_residual, matmul_q4_residual_rms_norm,
               matmul_q4_silu_mul, rms_norm, rmsnorm_matmul_q4)


def q_columns_attention(q_dim):
    """Stand-in attention: a contiguous copy of the q projection columns."""
    def attention(layer, qkv):
        return qkv[:, :q_dim].contiguous()
    return attention


class PrefillStep:
    """A prefill over buffers it owns, for prompts of exactly `seq_len` tokens.

    weights: a ModelWeights (swiftltx_amd.weights) loaded with concat_qkv, or
    any object with the same fields (see DecodeStep)."""

    def __init__(self, weights, seq_len, attention=None, stream=None):
        import torch
        c = weights.config
        if seq_len < 1:
            raise ValueError("seq_len must be >= 1")
        self.w = weights
        self.c = c
        self.S = int(seq_len)
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
        self.attention = attention or q_columns_attention(self.q_dim)
        dev = weights.embed_tokens.weight.device
        f16 = torch.float16
        S, K, F = self.S, self.hidden, c.intermediate_size
        self.tokens = torch.zeros(S, dtype=torch.int32, device=dev)
        self.h = torch.empty(S, K, dtype=f16, device=dev)        # residual stream
        self.normed = torch.empty(S, K, dtype=f16, device=dev)
        self.qkv = torch.empty(S, self.qkv_rows, dtype=f16, device=dev)
        self.res = torch.empty(S, K, dtype=f16, device=dev)
        self.act = torch.empty(S, F, dtype=f16, device=dev)
        self.logits = torch.empty(1, c.vocab_size, dtype=f16, device=dev)
        self.graph = None
        torch.cuda.current_stream(dev).synchronize()   # zeroed tokens before other streams read them

    def forward(self):
        """self.tokens (S ids) -> the last token's logits in self.logits."""
        c, w, s = self.c, self.w, self.stream
        S, K, F, eps = self.S, self.hidden, c.intermediate_size, c.rms_norm_eps
        embedding_q4(w.embed_tokens, c.vocab_size, self.tokens, out=self.h, stream=s)
        layers = w.layers
        rms_norm(self.h, layers[0].input_norm_weight, eps, S, K, out=self.normed, stream=s)
        for i, lw in enumerate(layers):
            linear(self.normed, lw.qkv_proj, S, K, self.qkv_rows, fast=True, out=self.qkv, stream=s)
            attn = self.attention(i, self.qkv)
            # res = h + o (the residual stream); gate/up read its norm
            matmul_q4_residual_rms_norm(attn, lw.o_proj, self.h, lw.post_norm_weight, eps, S, K,
                                        False, residual_out=self.res, norm_out=self.normed,
                                        stream=s)
            matmul_q4_silu_mul(self.normed, lw.gate_proj, lw.up_proj, S, K, F, out=self.act,
                               stream=s)
            # h = res + down, and the next layer's input norm of h
            if i + 1 < len(layers):
                matmul_q4_residual_rms_norm(self.act, lw.down_proj, self.res,
                                            layers[i + 1].input_norm_weight, eps, S, K, True,
                                            residual_out=self.h, norm_out=self.normed, stream=s)
            else:
                matmul_q4_residual(self.act, lw.down_proj, self.res, S, K, out=self.h, stream=s)
        rmsnorm_matmul_q4(self.h[S - 1:], w.norm_weight, eps, w.lm_head, c.vocab_size,
                          out=self.logits, stream=s)
        return self.logits

    def capture(self):
        """Capture forward() as a HIP graph on self.stream (a torch stream;
        required), after one eager run there (which sizes the workspace the
        split-K GEMMs and the fused residual + norm calls use in the graph)."""
        import torch
        if self.stream is None:
            raise ValueError("capture needs a dedicated stream")
        with torch.cuda.stream(self.stream):
            self.forward()
        self.stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=self.stream):
            self.forward()
        self.graph = g
        return g

    def replay(self):
        """One captured prefill (of the ids now in self.tokens), enqueued on the current stream.  Replays and eager
        steps of one object share its buffers and the capture stream's
        workspace: the caller keeps them in order (one stream, or
        synchronization between them).  Moving the replay onto the capture
        stream with cross-stream waits around it cost ~130 us per decode
        token."""
        if self.graph is None:
            raise RuntimeError("capture() first")
        self.graph.replay()
        return self.logits
