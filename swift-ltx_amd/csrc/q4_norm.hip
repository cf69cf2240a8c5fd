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
    for (int i = threadIdx.x; i < dim; i += 256) {
        const float r = b ? h2f(f2h(h2f(a[off + i]) + h2f(b[off + i]))) : h2f(a[off + i]);
        out[off + i] = f2h(r * rms * w[i]);
    }
}

hipError_t launch_rms_norm(const uint16_t* a, const uint16_t* b, const float* w, float eps,
                           uint16_t* res_out, uint16_t* out, int rows, int dim, hipStream_t st) {
    if (rows <= 0 || dim <= 0) return hipSuccess;
    hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(256), 0, st, a, b, w, eps, res_out, out, dim);
    return hipGetLastError();
}

}  // namespace sltx
