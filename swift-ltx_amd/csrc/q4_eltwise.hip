// q4_eltwise.hip -- standalone SiLU x up for API parity with siluMul, and
// the fp32 -> fp16 activation cast of sltx_matmul_q4_ex.
//
// out[i] = half((v / (1 + exp(-v))) * float(b[i])), v = float(a[i]):
// swift-ltx silu_mul (Kernels.swift:90-98) dispatched by siluMul (Ops.swift:44-56).
// The fused GEMV/GEMM epilogues make this op unnecessary on the hot path; it is
// kept so callers that still run gate and up separately have a drop-in.
// Eight elements per thread with 16-byte loads when the pointers allow it.
#include "q4_common.hpp"
#include "q4_launch.hpp"

namespace sltx {

__global__ __launch_bounds__(256) void silu_mul_vec8_kernel(const f16x8* __restrict__ a,
                                                            const f16x8* __restrict__ b,
                                                            f16x8* __restrict__ out, long n8) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n8) return;
    const f16x8 va = a[i], vb = b[i];
    f16x8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (f16)silu_mul_f32((float)va[e], (float)vb[e]);
    out[i] = r;
}

__global__ __launch_bounds__(256) void silu_mul_scalar_kernel(const uint16_t* __restrict__ a,
                                                              const uint16_t* __restrict__ b,
                                                              uint16_t* __restrict__ out,
                                                              long begin, long n) {
    const long i = begin + (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[i] = f2h(silu_mul_f32(h2f(a[i]), h2f(b[i])));
}

hipError_t launch_silu_mul(const uint16_t* a, const uint16_t* b, uint16_t* out, long count,
                           hipStream_t st) {
    if (count <= 0) return hipSuccess;
    const bool aligned = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                           reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    long done = 0;
    if (aligned) {
        const long n8 = count / 8;
        if (n8 > 0) {
            const long grid = (n8 + 255) / 256;
            hipLaunchKernelGGL(silu_mul_vec8_kernel, dim3((unsigned)grid), dim3(256), 0, st,
                               reinterpret_cast<const f16x8*>(a), reinterpret_cast<const f16x8*>(b),
                               reinterpret_cast<f16x8*>(out), n8);
            done = n8 * 8;
        }
    }
    if (done < count) {
        const long rest = count - done;
        const long grid = (rest + 255) / 256;
        hipLaunchKernelGGL(silu_mul_scalar_kernel, dim3((unsigned)grid), dim3(256), 0, st, a, b,
                           out, done, count);
    }
    return hipGetLastError();
}

// cast_f32_to_f16 (Kernels.swift:816-822): out[i] = half(clamp(x[i], -65504,
// 65504)), round to nearest even; the activation cast DiTLinear.applyF32in
// runs before matmulQ4FastF32 (DiTModel.swift:104-110).  Eight elements per
// thread per step (two 16-byte loads, one 16-byte store), grid-stride;
// count % 8 == 0 and 16-byte aligned pointers (the callers' rows are
// K % 32 == 0 elements long).
__global__ __launch_bounds__(256) void cast_f32_f16_kernel(const f32x4* __restrict__ x,
                                                           u32x4* __restrict__ out, long n8) {
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n8;
         i += (long)gridDim.x * blockDim.x) {
        const f32x4 a = x[2 * i], b = x[2 * i + 1];
        const float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            o[e] = (uint32_t)f2h(fminf(fmaxf(v[2 * e], -65504.0f), 65504.0f)) |
                   ((uint32_t)f2h(fminf(fmaxf(v[2 * e + 1], -65504.0f), 65504.0f)) << 16);
        out[i] = o;
    }
}

hipError_t launch_cast_f32_f16(const float* x, uint16_t* out, long count, hipStream_t st) {
    if (count <= 0) return hipSuccess;
    if (count % 8 != 0 || ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) & 15))
        return hipErrorInvalidValue;
    const long n8 = count / 8;
    long grid = (n8 + 255) / 256;
    if (grid > 4 * kCUs * 8) grid = 4 * kCUs * 8;
    hipLaunchKernelGGL(cast_f32_f16_kernel, dim3((unsigned)grid), dim3(256), 0, st,
                       reinterpret_cast<const f32x4*>(x), reinterpret_cast<u32x4*>(out), n8);
    return hipGetLastError();
}

}  // namespace sltx
