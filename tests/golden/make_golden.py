"""Write the golden fixtures for the 4-bit dequant matmul path.

    python tests/golden/make_golden.py

Each case is one safetensors file in the MLX 4-bit layout the reference
loader reads (ModelWeights.swift:109-120: <name>.weight U32 [N, K/8],
<name>.scales F16 [N, K/g], <name>.biases F16 [N, K/g]) plus:
    x          F16 [M, K]  (or U16 bf16 bit patterns when meta x_dtype=bf16)
    y_f64      F64 [M, N]  fp64 oracle (numpy and C restatements must agree)
    y_emu      F16 [M, N]  fp32 emulation of matmul_q4's summation order
                           (GEMV cases only; Kernels.swift:444-620)
    bias       F32 [N]     (epilogue cases)
The reference holds no vectors for this path (its tests never call the
quantized matmul), so these are produced by the oracle in oracle/ and pinned
by that oracle's own checks in tests/test_oracle.py.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
from safetensors.numpy import save_file

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
from oracle import q4_oracle as o  # noqa: E402

# name, M, N, K, group, seed, kind
CASES = [
    ("gemv_n64_k128_g64", 1, 64, 128, 64, 0, "plain"),
    ("gemv_n128_k3072_g64", 1, 128, 3072, 64, 1, "plain"),
    ("gemv_n96_k256_g32", 1, 96, 256, 32, 2, "plain"),
    ("gemv_n64_k512_g128", 1, 64, 512, 128, 3, "plain"),
    ("gemv_n50_k160_g32", 1, 50, 160, 32, 4, "plain"),
    ("gemm_m3_n96_k256_g64", 3, 96, 256, 64, 5, "plain"),
    ("gemm_m37_n160_k384_g64", 37, 160, 384, 64, 6, "plain"),
    ("swiglu_m1_n64_k192_g64", 1, 64, 192, 64, 7, "swiglu"),
    ("swiglu_m5_n80_k256_g64", 5, 80, 256, 64, 8, "swiglu"),
    ("dit_m9_n64_k128_g64_bf16_gelu", 9, 64, 128, 64, 9, "bf16_gelu"),
]


def make_case(name, M, N, K, g, seed, kind):
    tensors = {}
    meta = {"M": str(M), "N": str(N), "K": str(K), "group_size": str(g), "kind": kind,
            "seed": str(seed)}
    if kind == "swiglu":
        x, sets = o.make_inputs(M, N, K, g, seed=seed, n_weights=2)
        (wg, sg, bg), (wu, su, bu) = sets
        for pre, (w, s, b) in (("gate_proj", sets[0]), ("up_proj", sets[1])):
            tensors[pre + ".weight"] = w
            tensors[pre + ".scales"] = s
            tensors[pre + ".biases"] = b
        gate = o.matmul_q4_f64(x, wg, sg, bg, g)
        up = o.matmul_q4_f64(x, wu, su, bu, g)
        cg = o.c_matmul_q4_f64(x, wg, sg, bg, g)
        cu = o.c_matmul_q4_f64(x, wu, su, bu, g)
        assert np.allclose(gate, cg, rtol=1e-12, atol=1e-12)
        assert np.allclose(up, cu, rtol=1e-12, atol=1e-12)
        tensors["y_f64"] = o.silu_mul_f64(gate, up)
        # reference semantics: gate, up rounded to fp16, then silu_mul (Kernels.swift:90-98)
        ge = o.c_matmul_q4_emu(x, wg, sg, bg, g)
        ue = o.c_matmul_q4_emu(x, wu, su, bu, g)
        tensors["y_emu"] = o.c_silu_mul(ge, ue).reshape(M, N)
        tensors["x"] = x
    elif kind == "bf16_gelu":
        x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=seed, x_dtype="bf16")
        rng = np.random.default_rng(seed + 1000)
        bias = (0.5 * rng.standard_normal(N)).astype(np.float32)
        pre = o.matmul_q4_f64(o.x_values(x, "bf16"), w, s, b, g) + bias.astype(np.float64)
        cpre = o.c_matmul_q4_f64(x, w, s, b, g, x_dtype="bf16") + bias.astype(np.float64)
        assert np.allclose(pre, cpre, rtol=1e-12, atol=1e-12)
        tensors.update({"proj.weight": w, "proj.scales": s, "proj.biases": b, "x": x,
                        "bias": bias, "y_pre_f64": pre, "y_f64": o.gelu_tanh_f64(pre)})
        meta["x_dtype"] = "bf16"
    else:
        x, [(w, s, b)] = o.make_inputs(M, N, K, g, seed=seed)
        y = o.matmul_q4_f64(x, w, s, b, g)
        cy = o.c_matmul_q4_f64(x, w, s, b, g)
        assert np.allclose(y, cy, rtol=1e-12, atol=1e-12)
        tensors.update({"proj.weight": w, "proj.scales": s, "proj.biases": b, "x": x, "y_f64": y,
                        "y_emu": o.c_matmul_q4_emu(x, w, s, b, g)})
    tensors = {k: np.ascontiguousarray(v) for k, v in tensors.items()}
    save_file(tensors, os.path.join(HERE, name + ".safetensors"), metadata=meta)


def main():
    o.build_c()
    for case in CASES:
        make_case(*case)
    with open(os.path.join(HERE, "cases.json"), "w") as f:
        json.dump([{"name": c[0], "M": c[1], "N": c[2], "K": c[3], "group_size": c[4],
                    "seed": c[5], "kind": c[6]} for c in CASES], f, indent=1)
    print("wrote", len(CASES), "cases")


if __name__ == "__main__":
    main()
