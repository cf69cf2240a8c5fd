"""Shared helpers for the GPU parity tests.

Tolerances (fp64 oracle = reference semantics w = s*q + b, exact):
  GATE        the parity bar: max|y - ref| / max|ref| <= 1e-2.
  elementwise |y - ref| <= rtol*|ref| + atol_rms*rms(ref), per path:
    GEMV, fp16 out      rtol 6e-4 (fp16 store, half ulp = 4.9e-4), atol 1e-4*rms
    GEMM, fp16 weights  rtol 1e-3, atol 3e-3*rms  (weights rounded to fp16 before
                        the MFMA: relative 2^-11 per product)
    GEMM, bf16 weights  rtol 4e-3, atol 1.2e-2*rms (bf16: relative 2^-9 per product)
  The GEMM is also compared with a "rounded-weight" reference (the fp64
  product with the weights rounded exactly as the kernel rounds them), which
  it must match to fp32-accumulation accuracy.
"""
from __future__ import annotations

import os

import numpy as np
from safetensors.numpy import load_file
from safetensors import safe_open

from oracle import q4_oracle as o

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

GATE = 1e-2
TOL_GEMV = dict(rtol=6e-4, atol_rms=1e-4)
TOL_GEMM_F16 = dict(rtol=1e-3, atol_rms=3e-3)
TOL_GEMM_BF16 = dict(rtol=4e-3, atol_rms=1.2e-2)
TOL_ROUNDED_W = dict(rtol=6e-4, atol_rms=2e-5)


def load_golden(name):
    path = os.path.join(GOLDEN, name + ".safetensors")
    with safe_open(path, framework="numpy") as f:
        meta = f.metadata()
    return load_file(path), meta


def to_dev(a, dev):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).to(dev)


def q4w(pkg, w, s, b, K, g, dev):
    return pkg.Q4Weight(to_dev(w, dev), to_dev(s, dev), to_dev(b, dev), K, g)


def assert_parity(y, ref, tol, what=""):
    y = np.asarray(y, dtype=np.float64)
    err = o.max_rel_err(y, ref)
    assert err <= GATE, f"{what}: max_rel_err {err:.3e} > {GATE}"
    ok, worst = o.elementwise_ok(y, ref, **tol)
    assert ok, f"{what}: elementwise error {worst:.2f}x the allowance ({tol}); max_rel_err {err:.2e}"
    return err


def rounded_weights_f16(w, s, b, g):
    """fp16(s*q + b) rounded once, as the GEMM's fp16 FMA does (exact value
    computed in fp64, then one rounding to fp16)."""
    return o.dequant_f64(w, s, b, g).astype(np.float16).astype(np.float64)


def rounded_weights_bf16(w, s, b, g):
    """bf16(fp32(s*q + b)): the bf16 GEMM computes q*s+b with one fp32 FMA and
    rounds that to bf16."""
    f32 = o.dequant_f64(w, s, b, g).astype(np.float32)
    return o.bf16_bits_to_f32(o.f32_to_bf16_bits(f32)).astype(np.float64)


def gpu_inputs(M, N, K, g, seed, dev, x_dtype="f16", n_weights=1):
    """Large synthetic inputs generated on the device (the benchmark's input distributions):
    x ~ N(0,1); codes uniform (random 32-bit words); scales |N(0,0.02)|;
    biases -8*scales.  Returns torch tensors (x, [(w, s, b)])."""
    import torch
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    x = torch.randn(M, K, generator=gen, device=dev, dtype=torch.float32)
    x = x.to(torch.bfloat16 if x_dtype == "bf16" else torch.float16)
    sets = []
    for _ in range(n_weights):
        w = torch.randint(-2**31, 2**31 - 1, (N, K // 8), generator=gen, device=dev,
                          dtype=torch.int64).to(torch.int32)
        s = (torch.randn(N, K // g, generator=gen, device=dev) * 0.02).abs().to(torch.float16)
        b = (s.float() * -8.0).to(torch.float16)
        sets.append((w, s, b))
    return x, sets


def host(t):
    """torch device tensor -> numpy with the oracle's dtypes."""
    import torch
    if t.dtype == torch.int32:
        return t.cpu().numpy().view(np.uint32)
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()
