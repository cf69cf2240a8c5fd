// q4_split.hpp -- K splits across blocks with no second launch: each block
// stores its split's fp32 sums to the workspace, counts its arrival on its
// output tile's counter, and the block that arrives last adds the splits and
// runs the epilogue (q4_wide.hip, q4_mid.hip).
//
// The XCDs' L2s are not coherent with each other.  The partial sums are
// stored and loaded with the sc1 cache policy, the one the compiler gives
// agent-scope atomic loads and stores.  Every thread's stores have completed
// (vmcnt) before the block's barrier, thread 0 then adds to the counter with
// an agent-scope atomic, and the last block loads after reading the count
// and a second barrier, so no L2-wide write-back or invalidate is needed
// (agent-scope fences, which do both, made the wide route's split launches
// slower than a separate reduce pass).
#pragma once

#include "q4_common.hpp"

namespace sltx {

constexpr int kSc1 = 16;   // cache-policy operand: sc1

__device__ __forceinline__ __amdgpu_buffer_rsrc_t ws_rsrc(const float* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, 0x7fffffff, 0x00020000);
}

// NV consecutive partial sums into row[n .. n+NV-1] (element offset `row`
// in the workspace), columns past N dropped.
template <int NV>
__device__ __forceinline__ void store_f32v_sc1(__amdgpu_buffer_rsrc_t rs, size_t row, int n, int N,
                                               const float* v) {
    if ((N % NV) == 0 && n + NV <= N) {
        const int o = (int)((row + n) * sizeof(float));
        if constexpr (NV == 4) {
            const u32x4 d = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                             __float_as_uint(v[3])};
            __builtin_amdgcn_raw_buffer_store_b128(d, rs, o, 0, kSc1);
        } else if constexpr (NV == 2) {
            typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
            const u32x2 d = {__float_as_uint(v[0]), __float_as_uint(v[1])};
            __builtin_amdgcn_raw_buffer_store_b64(d, rs, o, 0, kSc1);
        } else {
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[0]), rs, o, 0, kSc1);
        }
        return;
    }
#pragma unroll
    for (int e = 0; e < NV; ++e)
        if (n + e < N)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[e]), rs,
                                                  (int)((row + n + e) * sizeof(float)), 0, kSc1);
}

// NV consecutive partial sums row[n .. n+NV-1], loaded whatever n (columns
// past N read an earlier column, to be discarded): no load sits behind a
// branch.  n is a multiple of NV, so with N % NV == 0 a group lies wholly
// before N or wholly past it, and clamping a group past N moves none of the
// columns that are kept.
template <int NV>
__device__ __forceinline__ void load_f32v_sc1(__amdgpu_buffer_rsrc_t rs, size_t row, int n, int N,
                                              float* v) {
    if ((N % NV) == 0) {
        const int o = (int)((row + min(n, N - NV)) * sizeof(float));
        if constexpr (NV == 4) {
            const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(rs, o, 0, kSc1);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = __uint_as_float(q[e]);
        } else if constexpr (NV == 2) {
            const auto q = __builtin_amdgcn_raw_buffer_load_b64(rs, o, 0, kSc1);
            v[0] = __uint_as_float(q[0]);
            v[1] = __uint_as_float(q[1]);
        } else {
            v[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, o, 0, kSc1));
        }
    } else {
#pragma unroll
        for (int e = 0; e < NV; ++e)
            v[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                rs, (int)((row + min(n + e, N - 1)) * sizeof(float)), 0, kSc1));
    }
}

// Arrival of this block on its output tile's counter `ticket` (after its
// sc1 partial stores): true in every thread of the block that arrives
// `nsplit`-th, which also resets the counter for the next launch.  Every
// thread of the block must call it.
__device__ __forceinline__ bool split_arrive_last(unsigned* ticket, unsigned nsplit) {
    __shared__ int last_block;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev =
            __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = prev + 1 == nsplit;
        if (last) __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_block = last;
    }
    __syncthreads();
    return last_block != 0;
}

}  // namespace sltx
