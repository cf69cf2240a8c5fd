// q4_norm.hip -- row-wise RMS norm and fused residual add + RMS norm, the
// operators on either side of the quantized projections in swift-ltx's Llama
// layer (rmsNorm, Ops.swift:8-27, kernel rms_norm, Kernels.swift:40-86;
// residualRmsNorm, Ops.swift:256-279, kernel residual_rms_norm,
// Kernels.swift:238-290).  fp16 in/out, fp32 weight and arithmetic.  These
// serve M > 1 (prefill); at M = 1 the same math runs as a prologue inside the
// GEMV (q4_gemv.hip).
#include "q4_common.hpp"
#include "q4_launch.hpp"

namespace sltx {

// One block per row.  v = a (or a + b, whose fp16 rounding is written to
// res_out); rms = rsqrt(mean(v^2) + eps) over the unrounded v; out = half(r *
// rms * w) with r the (rounded) input.
__global__ __launch_bounds__(256) void rms_norm_kernel(const uint16_t* a, const uint16_t* b,
                                                       const float* w, float eps, uint16_t* res_out,
                                                       uint16_t* out, int dim) {
    __shared__ float red[4];
    const size_t off = (size_t)blockIdx.x * dim;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < dim; i += 256) {
        float v = h2f(a[off + i]);
        if (b) {
            v += h2f(b[off + i]);
            res_out[off + i] = f2h(v);
        }
        ss += v * v;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float rms = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)dim + eps);
    // r is the stored residual element (written above by this same thread),
    // as residual_rms_norm reads it back; residual_out may be a or b itself.
    for (int i = threadIdx.x; i < dim; i += 256) {
        const float r = b ? h2f(res_out[off + i]) : h2f(a[off + i]);
        out[off + i] = f2h(r * rms * w[i]);
    }
}

// The same row norm with 16-byte accesses, for dim % 8 == 0 and 16-byte
// aligned rows: thread t holds pieces t, t + 256, ... (VPT of them, 8 values
// each) in registers between the sum of squares and the output, so a and b are
// read once.  Same arithmetic and order as rms_norm_kernel.
template <int VPT>
__global__ __launch_bounds__(256) void rms_norm_vec_kernel(const uint16_t* a, const uint16_t* b,
                                                           const float* w, float eps,
                                                           uint16_t* res_out, uint16_t* out,
                                                           int dim) {
    __shared__ float red[4];
    const int nv = dim / 8;
    const size_t off = (size_t)blockIdx.x * dim;
    const f16x8* A = reinterpret_cast<const f16x8*>(a + off);
    const f16x8* B = reinterpret_cast<const f16x8*>(b ? b + off : nullptr);
    f16x8 r[VPT];
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
        const int v = threadIdx.x + 256 * u;
        if (v >= nv) continue;
        const f16x8 x = A[v];
        if (b) {
            const f16x8 y = B[v];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float t = (float)x[e] + (float)y[e];
                ss += t * t;
                r[u][e] = (f16)t;
            }
            reinterpret_cast<f16x8*>(res_out + off)[v] = r[u];
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float t = (float)x[e];
                ss += t * t;
            }
            r[u] = x;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float rms = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)dim + eps);
    const f32x4* W = reinterpret_cast<const f32x4*>(w);
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
        const int v = threadIdx.x + 256 * u;
        if (v >= nv) continue;
        const f32x4 w0 = W[2 * v], w1 = W[2 * v + 1];
        f16x8 o8;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            o8[e] = (f16)((float)r[u][e] * rms * w0[e]);
            o8[4 + e] = (f16)((float)r[u][4 + e] * rms * w1[e]);
        }
        reinterpret_cast<f16x8*>(out + off)[v] = o8;
    }
}

hipError_t launch_rms_norm(const uint16_t* a, const uint16_t* b, const float* w, float eps,
                           uint16_t* res_out, uint16_t* out, int rows, int dim, hipStream_t st) {
    if (rows <= 0 || dim <= 0) return hipSuccess;
    if ((long)rows * 256 > 0xffffffffL) return hipErrorInvalidValue;   // one 256-thread block per row
    auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const bool vec = dim % 8 == 0 && al16(a) && al16(out) && al16(w) && (!b || (al16(b) && al16(res_out)));
    const int vpt = (dim / 8 + 255) / 256;
    if (vec && vpt <= 8) {
        const dim3 g(rows), t(256);
        if (vpt == 1) hipLaunchKernelGGL(rms_norm_vec_kernel<1>, g, t, 0, st, a, b, w, eps, res_out, out, dim);
        else if (vpt == 2) hipLaunchKernelGGL(rms_norm_vec_kernel<2>, g, t, 0, st, a, b, w, eps, res_out, out, dim);
        else if (vpt <= 4) hipLaunchKernelGGL(rms_norm_vec_kernel<4>, g, t, 0, st, a, b, w, eps, res_out, out, dim);
        else hipLaunchKernelGGL(rms_norm_vec_kernel<8>, g, t, 0, st, a, b, w, eps, res_out, out, dim);
    } else {
        hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(256), 0, st, a, b, w, eps, res_out, out, dim);
    }
    return hipGetLastError();
}

}  // namespace sltx
