// q4_probe.hip -- HBM read ceiling of the device (measurement utility).
//
// The weight GEMVs are pure read streams, so the ceiling they are judged
// against is the rate at which this GPU streams a large buffer into
// registers, not a copy (which also writes).  Each thread keeps four 16-byte
// nontemporal loads in flight per grid-stride step (the GEMV's own load
// shape) and XORs every 32-bit word it reads; each block writes the XOR of
// its words to sink[block], so the loads cannot be removed and the result can
// be checked against the host's XOR of the buffer.
#include "q4_common.hpp"
#include "q4_launch.hpp"

namespace sltx {

constexpr int kReadThreads = 256;
constexpr int kReadUnroll = 4;

__global__ __launch_bounds__(kReadThreads) void hbm_read_kernel(const u32x4* __restrict__ src,
                                                                long n16, uint32_t* sink) {
    __shared__ uint32_t red[kReadThreads / 64];
    const long step = (long)kReadThreads * kReadUnroll;   // words of one block step
    const long stride = (long)gridDim.x * step;
    u32x4 acc = {0u, 0u, 0u, 0u};
    long base = (long)blockIdx.x * step;
    // whole steps: unconditional loads, all four in flight
    for (; base + step <= n16; base += stride) {
        u32x4 v[kReadUnroll];
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u)
            v[u] = __builtin_nontemporal_load(&src[base + u * kReadThreads + threadIdx.x]);
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u) acc ^= v[u];
    }
    // the partial step at the end (one block at most)
    if (base < n16)
        for (long i = base + threadIdx.x; i < n16; i += kReadThreads) acc ^= src[i];
    uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t s = 0u;
        for (int w = 0; w < kReadThreads / 64; ++w) s ^= red[w];
        sink[blockIdx.x] = s;
    }
}

int hbm_read_blocks() { return 4 * kCUs; }

hipError_t launch_hbm_read(const void* src, long n16, uint32_t* sink, hipStream_t st) {
    hipLaunchKernelGGL(hbm_read_kernel, dim3(hbm_read_blocks()), dim3(kReadThreads), 0, st,
                       static_cast<const u32x4*>(src), n16, sink);
    return hipGetLastError();
}

}  // namespace sltx
