// hbm_read.hip -- the HBM read ceiling the weight streams are judged against
// (bench.py's measured_ceiling).  Built into its own library,
// lib/libswiftltx_bench.so: it is a measurement tool, not part of the
// drop-in C ABI in include/swiftltx_q4.h.
//
// The weight GEMVs are pure read streams, so the ceiling is the rate at which
// this GPU streams a large buffer into registers, not a copy (which also
// writes).  Each thread keeps four 16-byte nontemporal loads in flight per
// grid-stride step (the GEMV's own load shape) and XORs every 32-bit word it
// reads; each block writes the XOR of its words to sink[block], so the loads
// cannot be removed and the result can be checked against the host's XOR of
// the buffer.
//
// The same stream through direct global -> LDS copies (global_load_lds, 16
// bytes a lane): the same grid and the same four copies per thread and step,
// into a two-stage ring per wave, each copy read back from LDS by the lane
// that issued it and XOR-ed: the rate at which a kernel can stream weights
// from HBM into LDS.
#include <type_traits>

#include "../q4_common.hpp"
#include "../q4_dequant.hpp"

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


typedef __attribute__((address_space(3))) void* lds_ptr_t;

__global__ __launch_bounds__(kReadThreads) void hbm_read_lds_kernel(const u32x4* __restrict__ src,
                                                                    long n16, uint32_t* sink) {
    // two stages, each kReadUnroll copies of the block's threads; separate
    // arrays, so that a read of one stage does not wait for copies into the other
    __shared__ u32x4 st0[kReadUnroll * kReadThreads], st1[kReadUnroll * kReadThreads];
    __shared__ uint32_t red[kReadThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, w64 = tid & ~63;
    const long step = (long)kReadThreads * kReadUnroll;
    const long nsteps = n16 / step;   // whole steps; step j of this block: j * grid + block
    const long mine = nsteps > blockIdx.x ? (nsteps - blockIdx.x + gridDim.x - 1) / gridDim.x : 0;
    auto issue = [&](auto sc, long j) {   // kReadUnroll vector-memory ops
        u32x4* stg = decltype(sc)::value ? st1 : st0;
        const long base = (blockIdx.x + j * gridDim.x) * step;
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u)
            __builtin_amdgcn_global_load_lds((const void*)(src + base + u * kReadThreads + tid),
                                             (lds_ptr_t)(stg + u * kReadThreads + w64), 16, 0, 0);
    };
    u32x4 acc = {0u, 0u, 0u, 0u};
    auto drain = [&](auto sc) {   // this lane's copies of one stage
        const u32x4* stg = decltype(sc)::value ? st1 : st0;
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u) acc ^= stg[u * kReadThreads + w64 + lane];
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    // a stage is refilled only after the lane's reads of it returned
    // (lgkmcnt(0)); the copies are waited for with vmcnt, in issue order
    if (mine > 0) issue(S0{}, 0);
    for (long j = 0; j < mine; j += 2) {
        if (j + 1 < mine) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue(S1{}, j + 1);
            __builtin_amdgcn_s_waitcnt(vmcnt_only(kReadUnroll));
        } else {
            __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
        }
        drain(S0{});
        if (j + 1 < mine) {
            if (j + 2 < mine) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                issue(S0{}, j + 2);
                __builtin_amdgcn_s_waitcnt(vmcnt_only(kReadUnroll));
            } else {
                __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
            }
            drain(S1{});
        }
    }
    // the partial step at the end (one block at most), as in hbm_read_kernel
    const long tail = nsteps * step;
    if (tail < n16 && blockIdx.x == nsteps % gridDim.x)
        for (long i = tail + tid; i < n16; i += kReadThreads) acc ^= src[i];
    uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o, 64);
    if (lane == 0) red[tid >> 6] = x;
    __syncthreads();
    if (tid == 0) {
        uint32_t s = 0u;
        for (int w = 0; w < kReadThreads / 64; ++w) s ^= red[w];
        sink[blockIdx.x] = s;
    }
}

}  // namespace sltx

extern "C" {

// Words of sink: one per block of the read grid (4 per CU).
int sltx_bench_hbm_read_blocks(void) { return 4 * sltx::kCUs; }

// Reads `bytes` (a multiple of 16, src 16-byte aligned) into registers
// (lds = 0) or through direct-to-LDS copies (lds = 1) and writes the per-block
// XOR words to sink.  Returns 0, -1 for bad arguments, else the hipError_t.
int sltx_bench_hbm_read(const void* src, uint64_t bytes, uint32_t* sink, int32_t lds,
                        void* stream) {
    if (bytes == 0) return 0;
    if (!src || !sink || bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(src) & 15) != 0 ||
        (reinterpret_cast<uintptr_t>(sink) & 3) != 0)
        return -1;
    const long n16 = (long)(bytes / 16);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int blocks = sltx_bench_hbm_read_blocks();
    if (lds)
        hipLaunchKernelGGL(sltx::hbm_read_lds_kernel, dim3(blocks), dim3(sltx::kReadThreads), 0, st,
                           static_cast<const sltx::u32x4*>(src), n16, sink);
    else
        hipLaunchKernelGGL(sltx::hbm_read_kernel, dim3(blocks), dim3(sltx::kReadThreads), 0, st,
                           static_cast<const sltx::u32x4*>(src), n16, sink);
    return (int)hipGetLastError();
}

}  // extern "C"
