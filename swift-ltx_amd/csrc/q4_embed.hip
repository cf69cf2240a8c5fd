// q4_embed.hip -- 4-bit embedding gather (dequantized rows of the quantized
// token-embedding table, which Llama also ties to the lm_head weight,
// ModelWeights.swift:126-130).  Semantics of embedding_q4_batch /
// embedding_q4 (Kernels.swift:368-434), dispatched by embeddingQ4Batch /
// embeddingQ4 (Ops.swift:163-208): out[t, k] = half(float(q) * s + b), the
// product and sum in fp32.
#include "q4_common.hpp"
#include "q4_launch.hpp"

namespace sltx {

// One thread per 8-nibble word of a row: 8 outputs, one 16-byte store.
// Block b covers token b / bpr, words (b % bpr) * 256 + [0, 256).  Ids
// outside [0, vocab) write a zero row.
__global__ __launch_bounds__(256) void embedding_q4_kernel(EmbedParams p, int bpr) {
    const int t = blockIdx.x / bpr;
    const int i = (blockIdx.x % bpr) * 256 + threadIdx.x;   // word within the row
    const int words = p.K / 8;
    if (i >= words) return;
    const int id = p.ids[t];
    u32x4* dst = reinterpret_cast<u32x4*>(p.out + (size_t)t * p.K + (size_t)i * 8);
    if (id < 0 || id >= p.vocab) {
        *dst = u32x4{0u, 0u, 0u, 0u};
        return;
    }
    const uint32_t w = p.w[(size_t)id * words + i];
    const size_t gi = (size_t)id * p.groups + ((i * 8) >> p.glog2);
    const float s = h2f(p.s[gi]), b = h2f(p.b[gi]);
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float lo = fmaf((float)((w >> (8 * e)) & 0xFu), s, b);
        const float hi = fmaf((float)((w >> (8 * e + 4)) & 0xFu), s, b);
        o[e] = (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16);
    }
    *dst = o;
}

hipError_t launch_embedding_q4(const EmbedParams& p, int n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const int bpr = (p.K / 8 + 255) / 256;
    const long grid = (long)n * bpr;
    if (grid > 0x7fffffffL) return hipErrorInvalidValue;
    hipLaunchKernelGGL(embedding_q4_kernel, dim3((unsigned)grid), dim3(256), 0, st, p, bpr);
    return hipGetLastError();
}

}  // namespace sltx
