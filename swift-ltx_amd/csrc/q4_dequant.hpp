// q4_dequant.hpp -- the register dequantization shared by the MFMA kernels
// (q4_gemm.hip, q4_mid.hip, q4_skinny.hip, q4_narrow.hip): one packed word of
// 8 nibbles -> 8 fp16 weights s * q + b, each rounded once (matmulQ4Fast's
// fp16 dequant, Ops.swift:312-381), in k order or in an order that a matching
// reorder of 8 activations follows, and the XOR-swizzled 128-byte LDS rows
// of a 64-wide k-tile.
#pragma once

#include "q4_common.hpp"
#include "q4_launch.hpp"

namespace sltx {

// s_waitcnt immediates (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt
// 6:4, lgkmcnt 11:8; a field at its maximum does not wait)
__host__ __device__ constexpr int vmcnt_only(int n) {
    return (n & 0xF) | (0x7 << 4) | (0xF << 8) | (((n >> 4) & 0x3) << 14);
}

// x[k .. k+7] as four fp16 pairs (x0,x1) (x2,x3) (x4,x5) (x6,x7) -> the
// pairs (x0,x2) (x1,x3) (x4,x6) (x5,x7) of the dequantized word's order.
__device__ __forceinline__ u32x4 permute_x(u32x4 r) {
    u32x4 a;
    a[0] = __builtin_amdgcn_perm(r[1], r[0], 0x05040100u);
    a[1] = __builtin_amdgcn_perm(r[1], r[0], 0x07060302u);
    a[2] = __builtin_amdgcn_perm(r[3], r[2], 0x05040100u);
    a[3] = __builtin_amdgcn_perm(r[3], r[2], 0x07060302u);
    return a;
}

// One packed word -> 8 fp16 s*q+b in the order q0,q2,q1,q3,q4,q6,q5,q7.
// The nibbles are spread to bytes (q0 q2 q4 q6 and q1 q3 q5 q7), and
// v_cvt_scalef32_pk_f16_fp8 turns two bytes into two fp16 at a time: read as
// fp8 e4m3, a byte b < 16 is b * 2^-9 exactly (the subnormals and the first
// binade share one spacing), and the instruction's scale, of which only the
// exponent counts, is 2^9.  One v_pk_fma_f16 per pair then gives s * q + b
// with a single rounding.
__device__ __forceinline__ u32x4 dequant_word(uint32_t w, f16x2 s2, f16x2 b2) {
    const uint32_t lo = w & 0x0F0F0F0Fu;          // bytes q0 q2 q4 q6
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;   // bytes q1 q3 q5 q7
    const float k512 = 512.0f;                    // 2^9: fp8 byte b -> b
    f16x2 q[4];
    q[0] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, k512, false);   // q0, q2
    q[1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, k512, false);   // q1, q3
    q[2] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, k512, true);    // q4, q6
    q[3] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, k512, true);    // q5, q7
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = as_u32(__builtin_elementwise_fma(q[e], s2, b2));
    return o;
}

// LDS layout of a 64-wide k-tile: 128-byte rows of eight 16-byte columns.
// Logical column c of row r sits at physical column c ^ (r & 7) ^ ((r >> 3) & 1).
// A ds_read_b128 is served 16 lanes at a time by 64 4-byte banks (256 B): 16
// consecutive rows reading one logical column hit 16 distinct (row parity,
// column) slots, i.e. no bank conflicts.
__device__ __forceinline__ int swz(int row, int col16) {
    return row * 8 + (col16 ^ (row & 7) ^ ((row >> 3) & 1));
}

// One 32-bit word (8 nibbles, k order) -> 8 fp16 values s*q+b.  Nibbles are
// spread to bytes and interleaved back into k order with v_perm_b32; then
// v_cvt_scalef32_pk_f16_fp8 turns two bytes into two exact fp16 integers (an
// fp8 e4m3 byte b < 16 is b * 2^-9, and the instruction's scale, of which only
// the exponent counts, is 2^9) and one fp16 FMA q*s+b rounds once.
__device__ __forceinline__ u32x4 dequant_word_f16(uint32_t w, f16x2 s2, f16x2 b2) {
    const uint32_t lo = w & 0x0F0F0F0Fu;          // bytes q6 q4 q2 q0
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;   // bytes q7 q5 q3 q1
    const uint32_t q03 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);   // bytes q3 q2 q1 q0
    const uint32_t q47 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);   // bytes q7 q6 q5 q4
    const float k512 = 512.0f;
    f16x2 q[4];
    q[0] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(q03, k512, false);   // q0, q1
    q[1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(q03, k512, true);    // q2, q3
    q[2] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(q47, k512, false);   // q4, q5
    q[3] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(q47, k512, true);    // q6, q7
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = as_u32(__builtin_elementwise_fma(q[e], s2, b2));   // v_pk_fma_f16
    return o;
}

// An output in the launch's dtype.
__device__ __forceinline__ void store_one(const GemmParams& p, size_t o, float v) {
    if (p.y_dtype == kF32)
        reinterpret_cast<float*>(p.y)[o] = v;
    else if (p.y_dtype == kBF16)
        reinterpret_cast<uint16_t*>(p.y)[o] = f2bf(v);
    else
        reinterpret_cast<uint16_t*>(p.y)[o] = f2h(v);
}

}  // namespace sltx
