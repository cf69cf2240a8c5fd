// q4_probe.hip -- measurement utilities: the HBM read ceiling, the launch
// floor, the register-only MFMA rate and shader clock, and the cost of a
// grid-wide hand-off inside one launch.  None has a counterpart in the
// reference; they bound what the kernels of this library can reach.
//
// HBM read ceiling.
// The weight GEMVs are pure read streams, so the ceiling they are judged
// against is the rate at which this GPU streams a large buffer into
// registers, not a copy (which also writes).  Each thread keeps four 16-byte
// nontemporal loads in flight per grid-stride step (the GEMV's own load
// shape) and XORs every 32-bit word it reads; each block writes the XOR of
// its words to sink[block], so the loads cannot be removed and the result can
// be checked against the host's XOR of the buffer.
//
// The same stream through direct global -> LDS copies (global_load_lds, 16
// bytes a lane): the same grid and the same four copies per thread and step,
// into a two-stage ring per wave, each copy read back from LDS by the lane
// that issued it and XOR-ed.  It gives the rate at which a kernel can stream
// weights from HBM into LDS, against the register-load rate above.
#include <type_traits>

#include "q4_common.hpp"
#include "q4_dequant.hpp"
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

// ---- launch floor: a kernel that does nothing (one wave) ----
__global__ __launch_bounds__(64) void probe_empty_kernel() {}

// ---- register-only MFMA: each wave runs `iters` rounds of four independent
// v_mfma_f32_32x32x16_f16 on operands read once from `ab` (random bits keep
// the datapath toggling, as real data does).  Lane 0 of each block records
// the shader-clock cycles (s_memtime) and the 100 MHz wall-clock ticks
// (s_memrealtime) of its loop, so clock = cycles / ticks * 100 MHz.
constexpr int kMfmaThreads = 256;

__global__ __launch_bounds__(kMfmaThreads) void probe_mfma_kernel(const f16x8* __restrict__ ab,
                                                                  int iters, float* sink,
                                                                  unsigned long long* clocks) {
    const int lane = threadIdx.x & 63;
    const f16x8 a0 = ab[lane], a1 = ab[64 + lane], b0 = ab[128 + lane], b1 = ab[192 + lane];
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    __syncthreads();
    const unsigned long long t0 = clock64(), w0 = wall_clock64();
    for (int i = 0; i < iters; ++i) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b0, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b0, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b1, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b1, c3, 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) s += c0[k] + c1[k] + c2[k] + c3[k];
    const unsigned long long t1 = clock64(), w1 = wall_clock64();
    sink[blockIdx.x * kMfmaThreads + threadIdx.x] = s;
    if (threadIdx.x == 0) {
        clocks[2 * blockIdx.x] = t1 - t0;
        clocks[2 * blockIdx.x + 1] = w1 - w0;
    }
}

// ---- grid-wide hand-off inside one launch: `rounds` grid barriers among
// `blocks` one-wave blocks (all co-resident; the launcher checks), arrival
// by
//   mode 0  one agent-scope counter: every block adds 1, then polls it;
//   mode 1  per-XCD counters first (block b on XCD b % 8), the last arrival
//           of each XCD adds 1 to the global counter, every block polls it;
//   mode 2  tagged words: block b stores round + 1 to word b (agent scope),
//           then polls all `blocks` words until each holds round + 1 (the
//           decode-layer kernel's exchange: no atomics, no fence);
//   mode 3  a data hand-off without fences: block b stores 16 data words
//           with agent-scope (write-through) stores and waits for them to
//           complete, arrives as in mode 1, and after the wait reads all
//           16 * blocks words back with agent-coherent 16-byte buffer loads;
// with `fence`, an agent-scope release fence before arriving and an
// acquire fence after the wait (what handing data over through plain stores
// needs).  Every wait is bounded: after kProbeSpin polls the block adds one
// to *faults and leaves the loop, so the kernel always finishes.
// sync: kProbeSyncWords(blocks) zeroed words.
constexpr int kProbeSpin = 1 << 18;
constexpr int kXcds = 8;

int probe_sync_words(int blocks) { return 16 * (kXcds + 1) + 16 * blocks; }

__global__ __launch_bounds__(64) void probe_sync_kernel(int mode, int fence, int rounds,
                                                        uint32_t* sync, int* faults) {
    const int lane = threadIdx.x, G = gridDim.x, b = blockIdx.x;
    uint32_t* gcnt = sync;                               // own 64-byte line
    uint32_t* xcnt = sync + 16 + 16 * (b % kXcds);       // this XCD's line
    uint32_t* words = sync + 16 * (kXcds + 1);
    const int x = b % kXcds;
    const uint32_t gx = (uint32_t)((G - x + kXcds - 1) / kXcds);   // blocks on this XCD
    const uint32_t nx = (uint32_t)(G < kXcds ? G : kXcds);         // XCDs with blocks
    for (int r = 0; r < rounds; ++r) {
        if (fence) __atomic_thread_fence(__ATOMIC_RELEASE);
        bool ok = true;
        if (mode == 2) {
            const uint32_t tag = (uint32_t)r + 1u;
            if (lane == 0) __hip_atomic_store(&words[b], tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            int polls = 0;
            for (;;) {
                bool mine = true;
                for (int i = lane; i < G; i += 64)
                    mine &= __hip_atomic_load(&words[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= tag;
                if (__all(mine)) break;
                if (++polls >= kProbeSpin) {
                    ok = false;
                    break;
                }
            }
        } else {
            uint32_t target;
            if (mode == 3) {
                // this block's 16 words, then wait until they have completed
                if (lane < 16)
                    __hip_atomic_store(&words[16 * b + lane], (uint32_t)r + 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
            }
            if (lane == 0) {
                if (mode == 1 || mode == 3) {
                    const uint32_t old = __hip_atomic_fetch_add(xcnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (old + 1u == ((uint32_t)r + 1u) * gx)
                        __hip_atomic_fetch_add(gcnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                } else {
                    __hip_atomic_fetch_add(gcnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            target = ((uint32_t)r + 1u) * (mode == 0 ? (uint32_t)G : nx);
            int polls = 0;
            uint32_t seen = 0u;
            if (lane == 0) {
                while ((seen = __hip_atomic_load(gcnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) < target)
                    if (++polls >= kProbeSpin) break;
            }
            ok = __shfl(seen, 0, 64) >= target;
            if (ok && mode == 3) {   // read every block's words back, 16 bytes a lane
                const auto rsrc = __builtin_amdgcn_make_buffer_rsrc(words, (short)0, 64 * G,
                                                                    0x00020000);
                uint32_t bad = 0u;
                for (int i0 = 0; i0 < 4 * G; i0 += 64 * 8) {   // 4 * G quads, 8 a lane in flight
                    u32x4 v[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u)   // agent-coherent (sc1); past the end: zeros
                        v[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                   rsrc, 16 * (i0 + 64 * u + lane), 0, 16));
#pragma unroll
                    for (int u = 0; u < 8; ++u)
                        if (i0 + 64 * u + lane < 4 * G)
                            bad |= (v[u].x < (uint32_t)r + 1u) | (v[u].y < (uint32_t)r + 1u) |
                                   (v[u].z < (uint32_t)r + 1u) | (v[u].w < (uint32_t)r + 1u);
                }
                ok = !__any(bad);
            }
        }
        if (!ok) {
            if (lane == 0) atomicAdd(faults, 1);
            return;
        }
        if (fence) __atomic_thread_fence(__ATOMIC_ACQUIRE);
    }
}

int probe_sync_max_blocks() {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, probe_sync_kernel, 64, 0) !=
        hipSuccess)
        return 0;
    return per_cu * kCUs;
}

hipError_t launch_probe_empty(hipStream_t st) {
    hipLaunchKernelGGL(probe_empty_kernel, dim3(1), dim3(64), 0, st);
    return hipGetLastError();
}

hipError_t launch_probe_mfma(const void* ab, int blocks, int iters, float* sink,
                             unsigned long long* clocks, hipStream_t st) {
    hipLaunchKernelGGL(probe_mfma_kernel, dim3(blocks), dim3(kMfmaThreads), 0, st,
                       static_cast<const f16x8*>(ab), iters, sink, clocks);
    return hipGetLastError();
}

hipError_t launch_probe_sync(int mode, int fence, int blocks, int rounds, uint32_t* sync,
                             int* faults, hipStream_t st) {
    hipLaunchKernelGGL(probe_sync_kernel, dim3(blocks), dim3(64), 0, st, mode, fence, rounds,
                       sync, faults);
    return hipGetLastError();
}

hipError_t launch_hbm_read(const void* src, long n16, uint32_t* sink, bool lds, hipStream_t st) {
    if (lds)
        hipLaunchKernelGGL(hbm_read_lds_kernel, dim3(hbm_read_blocks()), dim3(kReadThreads), 0, st,
                           static_cast<const u32x4*>(src), n16, sink);
    else
        hipLaunchKernelGGL(hbm_read_kernel, dim3(hbm_read_blocks()), dim3(kReadThreads), 0, st,
                           static_cast<const u32x4*>(src), n16, sink);
    return hipGetLastError();
}

}  // namespace sltx
