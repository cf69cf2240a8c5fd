// q4_gemv_ops.hpp -- the GEMV's per-lane building blocks (q4_gemv.hip): x
// preparation into dot order, the dequantizing dot over one 32-nibble chunk,
// and the DPP / permlane row reductions.
#pragma once

#include "q4_common.hpp"

namespace sltx {

// Build the dot-order pairs for 8 consecutive x values (one weight word).
__device__ __forceinline__ void pair_word(const f16x8& xv, uint32_t out[4], float& corr,
                                          float& sum) {
    const f16 sixteenth = (f16)0.0625f;
    f16 a0 = xv[0], a1 = xv[1] * sixteenth, a2 = xv[2], a3 = xv[3] * sixteenth;
    f16 a4 = xv[4], a5 = xv[5] * sixteenth, a6 = xv[6], a7 = xv[7] * sixteenth;
    f16x2 p0 = {a0, a4}, p1 = {a1, a5}, p2 = {a2, a6}, p3 = {a3, a7};
    out[0] = as_u32(p0);
    out[1] = as_u32(p1);
    out[2] = as_u32(p2);
    out[3] = as_u32(p3);
    corr += 1024.0f * ((float)a0 + (float)a1 + (float)a2 + (float)a3 + (float)a4 + (float)a5 +
                       (float)a6 + (float)a7);
    sum += (float)xv[0] + (float)xv[1] + (float)xv[2] + (float)xv[3] + (float)xv[4] +
           (float)xv[5] + (float)xv[6] + (float)xv[7];
}

// sum_k q[k]*x[k] over one 32-nibble chunk, starting from -corr.  The first
// dot of each of the two chains is the untied v_dot2_f32_f16 with its start
// value as an operand: left to the compiler, every chain becomes
// v_dot2c_f32_f16 (accumulator tied to the destination) and needs a copy of
// its start value first (two per chunk; measured: gate/up 6.66-6.70 ->
// 6.62-6.64 us, fused decode layer 19.0 -> 18.8 us).
__device__ __forceinline__ float chunk_dot(const u32x4 w, const u32x4 xq[4], float negcorr) {
    float d0, d1;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t wj = w[j];
        const uint32_t w8 = wj >> 8;
        const uint32_t p0 = and_or(wj, 0x000F000Fu, kMagic1024x2);
        const uint32_t p1 = and_or(wj, 0x00F000F0u, kMagic1024x2);
        const uint32_t p2 = and_or(w8, 0x000F000Fu, kMagic1024x2);
        const uint32_t p3 = and_or(w8, 0x00F000F0u, kMagic1024x2);
        if (j == 0) {
            asm("v_dot2_f32_f16 %0, %1, %2, %3" : "=v"(d0) : "v"(p0), "v"(xq[j][0]), "v"(negcorr));
            asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(d1) : "v"(p1), "v"(xq[j][1]));
        } else {
            d0 = dot2(as_f16x2(p0), as_f16x2(xq[j][0]), d0);
            d1 = dot2(as_f16x2(p1), as_f16x2(xq[j][1]), d1);
        }
        d0 = dot2(as_f16x2(p2), as_f16x2(xq[j][2]), d0);
        d1 = dot2(as_f16x2(p3), as_f16x2(xq[j][3]), d1);
    }
    return d0 + d1;
}

// chunk_dot for two x rows over the same weight chunk: each word is
// dequantized once and dotted with both rows' pairs (four chains).
__device__ __forceinline__ void chunk_dot_x2(const u32x4 w, const u32x4 xa[4], const u32x4 xb[4],
                                             float nca, float ncb, float& ra, float& rb) {
    float a0, a1, b0, b1;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t wj = w[j];
        const uint32_t w8 = wj >> 8;
        const uint32_t p0 = and_or(wj, 0x000F000Fu, kMagic1024x2);
        const uint32_t p1 = and_or(wj, 0x00F000F0u, kMagic1024x2);
        const uint32_t p2 = and_or(w8, 0x000F000Fu, kMagic1024x2);
        const uint32_t p3 = and_or(w8, 0x00F000F0u, kMagic1024x2);
        if (j == 0) {
            asm("v_dot2_f32_f16 %0, %1, %2, %3" : "=v"(a0) : "v"(p0), "v"(xa[j][0]), "v"(nca));
            asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(a1) : "v"(p1), "v"(xa[j][1]));
            asm("v_dot2_f32_f16 %0, %1, %2, %3" : "=v"(b0) : "v"(p0), "v"(xb[j][0]), "v"(ncb));
            asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(b1) : "v"(p1), "v"(xb[j][1]));
        } else {
            a0 = dot2(as_f16x2(p0), as_f16x2(xa[j][0]), a0);
            a1 = dot2(as_f16x2(p1), as_f16x2(xa[j][1]), a1);
            b0 = dot2(as_f16x2(p0), as_f16x2(xb[j][0]), b0);
            b1 = dot2(as_f16x2(p1), as_f16x2(xb[j][1]), b1);
        }
        a0 = dot2(as_f16x2(p2), as_f16x2(xa[j][2]), a0);
        a1 = dot2(as_f16x2(p3), as_f16x2(xa[j][3]), a1);
        b0 = dot2(as_f16x2(p2), as_f16x2(xb[j][2]), b0);
        b1 = dot2(as_f16x2(p3), as_f16x2(xb[j][3]), b1);
    }
    ra = a0 + a1;
    rb = b0 + b1;
}

// v + (v from another lane of the same 16-lane row), by DPP.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    const int m = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false);
    return v + __builtin_bit_cast(float, m);
}

// Sum over each aligned group of L lanes (L = 16, 32 or 64), result in every
// lane of the group.  Within a 16-lane row: DPP quad_perm [1,0,3,2] and
// [2,3,0,1], then row_half_mirror and row_mirror (each pairs lanes whose
// partial sums are disjoint).  Across rows: v_permlane16_swap (row pairs)
// and v_permlane32_swap (wave halves), each returning the two halves to add.
template <int L>
__device__ __forceinline__ float row_reduce(float v) {
    if (L >= 2) v = dpp_add<0xB1>(v);
    if (L >= 4) v = dpp_add<0x4E>(v);
    if (L >= 8) v = dpp_add<0x141>(v);
    if (L >= 16) v = dpp_add<0x140>(v);
    if (L >= 32) {
        const unsigned u = __builtin_bit_cast(unsigned, v);
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        v = __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
    }
    if (L >= 64) {
        const unsigned u = __builtin_bit_cast(unsigned, v);
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        v = __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
    }
    return v;
}

}  // namespace sltx
