// q4_epilogue.hpp -- the MFMA kernels' output stage on eight consecutive
// columns of one row (q4_gemm.hip, q4_wide.hip): the fp32 bias, GELU-tanh
// and residual epilogues, 16-byte vector stores when the row allows them, and
// raw fp32 partial sums for split-K workspaces.
#pragma once

#include "q4_common.hpp"
#include "q4_launch.hpp"

namespace sltx {

__device__ __forceinline__ void store_out(const GemmParams& p, size_t o, float v) {
    if (p.y_dtype == kF32)
        reinterpret_cast<float*>(p.y)[o] = v;
    else if (p.y_dtype == kBF16)
        reinterpret_cast<uint16_t*>(p.y)[o] = f2bf(v);
    else
        reinterpret_cast<uint16_t*>(p.y)[o] = f2h(v);
}

// Whether rows of y (and of the residual) can take 16-byte vector stores.
__device__ __forceinline__ bool out_vec_ok(const GemmParams& p) {
    return (p.N & 7) == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0 &&
           (p.epilogue != kEpiResidual || (reinterpret_cast<uintptr_t>(p.residual) & 15) == 0);
}

// Eight consecutive outputs row[n0 .. n0+7] (columns past N dropped): one
// 16-byte store (two for fp32) when `vec` (N % 8 == 0, 16-byte aligned y),
// else one store per element.
__device__ __forceinline__ void store_out8(const GemmParams& p, size_t row, int n0,
                                           const float* v, bool vec) {
    if (vec && n0 + 8 <= p.N) {
        if (p.y_dtype == kF32) {
            f32x4* d = reinterpret_cast<f32x4*>(reinterpret_cast<float*>(p.y) + row + n0);
            d[0] = f32x4{v[0], v[1], v[2], v[3]};
            d[1] = f32x4{v[4], v[5], v[6], v[7]};
        } else {
            u32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t lo = p.y_dtype == kBF16 ? f2bf(v[2 * e]) : f2h(v[2 * e]);
                const uint32_t hi = p.y_dtype == kBF16 ? f2bf(v[2 * e + 1]) : f2h(v[2 * e + 1]);
                o[e] = lo | (hi << 16);
            }
            *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(p.y) + row + n0) = o;
        }
        return;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e)
        if (n0 + e < p.N) store_out(p, row + n0 + e, v[e]);
}

// Non-SiLU epilogue (bias, GELU-tanh, residual add) on eight consecutive
// outputs, then stored as store_out8 does.
__device__ __forceinline__ void epi_store8(const GemmParams& p, size_t row, int n0, float* v,
                                           bool vec) {
    if (p.bias) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] += p.bias[n0 + e < p.N ? n0 + e : 0];
    }
    if (p.epilogue == kEpiGeluTanh) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = gelu_tanh_f32(v[e]);
    }
    if (p.epilogue == kEpiResidual) {
        if (vec && n0 + 8 <= p.N) {
            const u32x4 r = *reinterpret_cast<const u32x4*>(p.residual + row + n0);
            u32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t lo = residual_add_f16((uint16_t)(r[e] & 0xFFFFu), v[2 * e]);
                const uint32_t hi = residual_add_f16((uint16_t)(r[e] >> 16), v[2 * e + 1]);
                o[e] = lo | (hi << 16);
            }
            *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(p.y) + row + n0) = o;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (n0 + e < p.N)
                    reinterpret_cast<uint16_t*>(p.y)[row + n0 + e] =
                        residual_add_f16(p.residual[row + n0 + e], v[e]);
        }
        return;
    }
    store_out8(p, row, n0, v, vec);
}

// Eight raw fp32 partial sums into a workspace row (16-byte aligned rows when
// N % 4 == 0).
__device__ __forceinline__ void store_f32x8(float* wsr, int n0, int N, const float* v) {
    if ((N & 3) == 0 && n0 + 8 <= N) {
        f32x4* d = reinterpret_cast<f32x4*>(wsr + n0);
        d[0] = f32x4{v[0], v[1], v[2], v[3]};
        d[1] = f32x4{v[4], v[5], v[6], v[7]};
        return;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e)
        if (n0 + e < N) wsr[n0 + e] = v[e];
}

// NV (2 or 4) consecutive outputs row[n0 .. n0+NV-1] (columns past N
// dropped): one 4- to 16-byte store when N % NV == 0 and y is 16-byte
// aligned, else one store per element.
template <int NV>
__device__ __forceinline__ void store_outv(const GemmParams& p, size_t row, int n0, const float* v) {
    static_assert(NV == 2 || NV == 4, "2 or 4 outputs");
    if ((p.N % NV) == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0 && n0 + NV <= p.N) {
        if (p.y_dtype == kF32) {
            float* d = reinterpret_cast<float*>(p.y) + row + n0;
            if constexpr (NV == 4) *reinterpret_cast<f32x4*>(d) = f32x4{v[0], v[1], v[2], v[3]};
            else *reinterpret_cast<float2*>(d) = make_float2(v[0], v[1]);
        } else {
            uint32_t w[NV / 2];
#pragma unroll
            for (int e = 0; e < NV / 2; ++e) {
                const uint32_t lo = p.y_dtype == kBF16 ? f2bf(v[2 * e]) : f2h(v[2 * e]);
                const uint32_t hi = p.y_dtype == kBF16 ? f2bf(v[2 * e + 1]) : f2h(v[2 * e + 1]);
                w[e] = lo | (hi << 16);
            }
            uint16_t* d = reinterpret_cast<uint16_t*>(p.y) + row + n0;
            if constexpr (NV == 4) *reinterpret_cast<uint2*>(d) = make_uint2(w[0], w[1]);
            else *reinterpret_cast<uint32_t*>(d) = w[0];
        }
        return;
    }
#pragma unroll
    for (int e = 0; e < NV; ++e)
        if (n0 + e < p.N) store_out(p, row + n0 + e, v[e]);
}

// The non-gated epilogues (bias, GELU-tanh, residual add) on NV consecutive
// outputs, stored as store_outv does.
template <int NV>
__device__ __forceinline__ void epi_storev(const GemmParams& p, size_t row, int n0, float* v) {
    if (p.bias) {
#pragma unroll
        for (int e = 0; e < NV; ++e) v[e] += p.bias[n0 + e < p.N ? n0 + e : 0];
    }
    if (p.epilogue == kEpiGeluTanh) {
#pragma unroll
        for (int e = 0; e < NV; ++e) v[e] = gelu_tanh_f32(v[e]);
    }
    if (p.epilogue == kEpiResidual) {
        // fp16 output only: the projection rounded, added to the residual, rounded
        if (NV == 4 && (p.N & 3) == 0 && n0 + 4 <= p.N &&
            ((reinterpret_cast<uintptr_t>(p.y) | reinterpret_cast<uintptr_t>(p.residual)) & 7) == 0) {
            const uint2 r = *reinterpret_cast<const uint2*>(p.residual + row + n0);
            const uint32_t o0 = residual_add_f16((uint16_t)(r.x & 0xFFFFu), v[0]) |
                                ((uint32_t)residual_add_f16((uint16_t)(r.x >> 16), v[1]) << 16);
            const uint32_t o1 = residual_add_f16((uint16_t)(r.y & 0xFFFFu), v[2]) |
                                ((uint32_t)residual_add_f16((uint16_t)(r.y >> 16), v[3]) << 16);
            *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.y) + row + n0) = make_uint2(o0, o1);
            return;
        }
#pragma unroll
        for (int e = 0; e < NV; ++e)
            if (n0 + e < p.N)
                reinterpret_cast<uint16_t*>(p.y)[row + n0 + e] =
                    residual_add_f16(p.residual[row + n0 + e], v[e]);
        return;
    }
    store_outv<NV>(p, row, n0, v);
}

// NV raw fp32 partial sums into a workspace row.
template <int NV>
__device__ __forceinline__ void store_f32v(float* wsr, int n0, int N, const float* v) {
    if ((N % NV) == 0 && n0 + NV <= N) {
        if constexpr (NV == 4) *reinterpret_cast<f32x4*>(wsr + n0) = f32x4{v[0], v[1], v[2], v[3]};
        else *reinterpret_cast<float2*>(wsr + n0) = make_float2(v[0], v[1]);
        return;
    }
#pragma unroll
    for (int e = 0; e < NV; ++e)
        if (n0 + e < N) wsr[n0 + e] = v[e];
}

}  // namespace sltx
