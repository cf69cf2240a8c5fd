// q4_common.hpp -- shared definitions for the MLX 4-bit dequant matmul kernels
// (gfx950 / CDNA4).
//
// Weight layout (swift-ltx ModelWeights.swift:7-11, LinearWeight.quantized):
//   weight  uint32 [N, K/8]  nibble k of row n = bits 4*(k%8)..+3 of word k/8
//   scales  fp16   [N, K/g]
//   biases  fp16   [N, K/g]
//   w[n,k] = scales[n,k/g] * q[n,k] + biases[n,k/g]   (Kernels.swift:392-395)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sltx {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kCUs = 256;   // compute units of an MI355X (8 XCDs x 32)

// fp16 bit pattern of 1024.0: OR-ing a value v < 1024 into its mantissa gives
// the fp16 number 1024 + v exactly (Kim et al. 2022, "Who Says Elephants
// Can't Run", int4 -> fp16 conversion by mantissa insertion).
constexpr uint32_t kMagic1024x2 = 0x64006400u;

__device__ __forceinline__ f16x2 as_f16x2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
__device__ __forceinline__ uint32_t as_u32(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// v_and_or_b32: (a & mask) | magic.  Written as one instruction: for two
// 32-bit literal operands the compiler emits v_and_b32 + v_or_b32 (this
// VOP3 form takes no literal, and at most one scalar operand), so both
// constants are passed in VGPRs, where they are loop-invariant.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t orv) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(mask), "v"(orv));
    return r;
}

// v_dot2_f32_f16: a.x*b.x + a.y*b.y + c with fp32 accumulation.
__device__ __forceinline__ float dot2(f16x2 a, f16x2 b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
}

__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(f16, h);
}

__device__ __forceinline__ uint16_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, (f16)f);  // v_cvt_f16_f32, round to nearest even
}

__device__ __forceinline__ float bf2f(uint16_t h) {
    return __builtin_bit_cast(float, (uint32_t)h << 16);
}

__device__ __forceinline__ uint16_t f2bf(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);  // round to nearest even
}

// Epilogue activations, fp32, with the hardware exp2 (__expf) and reciprocal
// (about 1e-6 relative; the outputs are rounded to 16 bits).
// silu_mul (Kernels.swift:90-98): v / (1 + exp(-v)) * u
__device__ __forceinline__ float silu_mul_f32(float v, float u) {
    return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)) * u;
}

// gelu_approximate_f32 (Kernels.swift:1774-1783), inner clamped to +-10:
// 0.5 v (1 + tanh(inner)) written as v / (1 + exp(-2 inner)).
__device__ __forceinline__ float gelu_tanh_f32(float v) {
    float inner = 0.7978845608f * (v + 0.044715f * v * v * v);
    inner = fminf(fmaxf(inner, -10.0f), 10.0f);
    return v * __builtin_amdgcn_rcpf(1.0f + __expf(-2.0f * inner));
}

// Status codes shared with the C ABI (include/swiftltx_q4.h).
enum : int {
    kOk = 0,
    kErrInvalid = -1,
    kErrUnsupported = -2,
    kErrHip = -3,
};

// Element types at the boundary.
enum DType : int { kF16 = 0, kBF16 = 1, kF32 = 2 };

// Epilogues applied to the fp32 accumulator before the store.
enum Epilogue : int {
    kEpiNone = 0,
    kEpiSiluMul = 1,   // y = silu(x.Wg^T) * (x.Wu^T)  (two weight sets)
    kEpiGeluTanh = 2,  // y = gelu_tanh(x.W^T + bias)
    kEpiResidual = 3,  // y = half(residual + half(x.W^T))  (linear + elemAdd, fp16 out)
    kEpiGeluMul = 4,   // y = gelu_tanh(x.Wg^T) * (x.Wu^T)  (two weight sets; T5 GeGLU)
};

// Gated activations of the two-weight-set epilogues: SiLU (Llama MLP) or
// GELU-tanh (T5 GeGLU, T5Encoder.swift:191-199), on fp32 products.
__device__ __forceinline__ float glu_f32(bool gelu, float gate, float up) {
    return gelu ? gelu_tanh_f32(gate) * up : silu_mul_f32(gate, up);
}

// linear(...) then elemAdd(residual, .) (LlamaModel.swift:330-331): the
// projection is rounded to fp16 first, then added in fp32 and rounded again
// (the reference's add kernel, Kernels.swift:121-128).
__device__ __forceinline__ uint16_t residual_add_f16(uint16_t residual, float acc) {
    return f2h(h2f(residual) + h2f(f2h(acc)));
}

}  // namespace sltx
