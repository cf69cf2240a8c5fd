// q4_narrow.hip -- 4-bit dequant matmul for M <= 8 activation rows (short
// prompts, batched decode, the T5 encoder at a few tokens) on CDNA4's
// 4x4x4 MFMA blocks, as a weight stream shaped like the GEMV.
//
// Same product as q4_gemm.hip, Y[M,N] = X[M,K] . dequant(W)[N,K]^T with the
// weights dequantized to fp16 (s * q + b, one rounding) and fp32 accumulation
// (matmulQ4Fast, Ops.swift:312-381).  At M <= 8 each weight byte feeds at
// most 8 multiply-adds: the launch is bound by the weight stream, and what
// decides its time is how the loads reach HBM and how little work is left
// once the last of them lands.
//  * v_mfma_f32_4x4x4_16b_f16 is 16 independent 4x4x4 products: lane
//    4b + i supplies row i of block b's A (4 k) and column i of its B, and
//    VGPR v of lane 4b + i receives D[v][i] of block b (checked on the GPU).
//    Here every block works on the same 4 weight rows (B columns) and the
//    same 4 activation rows (A rows), each on its own 32 k of a 512-k run:
//    lane 4 * pc + n covers weight row n and piece pc (16 bytes) of the
//    run.  One 16-byte load per lane is then 4 rows x 256 contiguous bytes,
//    whole 128-byte lines (a load of 16 rows x 64 bytes, the 16x16 MFMA's
//    operand shape, streams ~15% slower: every request is half a line).
//  * A wave owns 4 rows of each weight set (gate and up for the gated
//    epilogues) and 1/S of the runs of K, with every load in flight before
//    the first MFMA, in use order.  S (1, 2 or 4) is chosen so the launch
//    has about 16 waves per CU: a wave's loads come back close together,
//    behind those of the waves that started before it, so what is left
//    after the last load lands is one wave's dequantization, and smaller
//    waves leave less.  The 16 per-piece partials are summed across lanes
//    (DPP row rotations, then two cross-row shuffles), and the S waves of a
//    row group add theirs through LDS, in a fixed order.
//  * X's M rows are copied once per block to LDS (direct 16-byte copies,
//    1 KB per wave-wide copy).  Piece c of row m is stored at position
//    c ^ (m & 3) of its 1 KB chunk, so a fragment read -- 4 pieces of 4 rows
//    per 16 lanes -- hits 16 distinct bank groups.  A rows past M read row
//    M - 1: their outputs are never stored.
//  * Each weight word is dequantized in registers (q4_dequant.hpp) into
//    two B fragments of 4 k; with M <= 4 one A block serves them, with
//    M <= 8 two.  Per word that is 2 (or 4) MFMAs of 8 cycles each, the same
//    matrix time as one 16x16x32 MFMA.  The dequantization (~57 cycles of
//    VALU per wave-word) is the compute bound.
//  * A lane's scale and bias for a run are 2-byte loads issued with that
//    run's weights (its 32 k lie in one group: group sizes 32, 64, 128).
//    Copying each wave's slabs to LDS first instead measured slower: the
//    first MFMA then waits for the slabs as well as the first run.
#include "q4_common.hpp"
#include "q4_dequant.hpp"
#include "q4_launch.hpp"

namespace sltx {

namespace {

typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kNarrowMaxLds = 78 * 1024;   // X bytes a block may stage (two blocks per CU)
constexpr int kNarrowMaxWaves = 8;

// Dynamic LDS of a launch: X's rows.
size_t narrow_lds(const GemmParams& p) { return (size_t)p.M * p.K * 2; }

__device__ __forceinline__ f32x4 mfma4(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1,
                                       f32x4 c) {
    const u32x2 a = {a0, a1}, b = {b0, b1};
    return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(f16x4_t, a),
                                              __builtin_bit_cast(f16x4_t, b), c, 0, 0, 0);
}

// Sum over the 16 lanes that share lane % 4 (lane bits 2..5): two row
// rotations (by 4 and 8 lanes) inside each 16-lane row, then across rows.
__device__ __forceinline__ float sum_pieces(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               0x124, 0xF, 0xF, false));   // row_ror:4
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               0x128, 0xF, 0xF, false));   // row_ror:8
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

// RUNS 512-k runs of K split over S waves, PAIR: two weight sets and a
// gated epilogue, MB: A blocks of 4 activation rows (M <= 4 * MB).  A block
// is W = S * RG waves: RG row groups of 4 rows.
template <int RUNS, int S, bool PAIR, int MB>
__global__ __launch_bounds__(64 * kNarrowMaxWaves) void q4_narrow_kernel(GemmParams p) {
    constexpr int NS = PAIR ? 2 : 1;
    constexpr int R = RUNS / S;   // runs per wave
    static_assert(RUNS % S == 0, "runs split evenly");
    extern __shared__ u32x4 xl[];   // X rows [M][RUNS chunks of 64 pieces]
    __shared__ float red[kNarrowMaxWaves][NS * MB * 4][4];   // partials of waves ks > 0
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, W = blockDim.x >> 6;
    const int n = lane & 3, pc = lane >> 2;
    const int rg = wave / S, ks = wave - rg * S;
    const int K = p.K, M = p.M;

    // ---- X rows [0, M) -> LDS, one 1 KB chunk per wave-wide copy ----
    for (int c = wave; c < M * RUNS; c += W) {   // wave-uniform
        const int m = c / RUNS, j = c - m * RUNS;
        const char* src = reinterpret_cast<const char*>(p.a) + ((size_t)m * K + j * 512) * 2 +
                          (lane ^ (m & 3)) * 16;
        __builtin_amdgcn_global_load_lds((const void*)src, (lds_ptr_t)(xl + c * 64), 16, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- the wave's rows and runs: scale, bias and packed words per run and
    // set, in use order ----
    const int row0 = (blockIdx.x * (W / S) + rg) * 4;
    const int row = min(row0 + n, p.N - 1);   // clamped rows are computed and dropped
    const int gshift = 5 + p.gshift;          // log2(group size)
    const int j0 = ks * R;
    u32x4 wq[R][NS];
    uint32_t sv[R][NS], bv[R][NS];
#pragma unroll
    for (int jj = 0; jj < R; ++jj)
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int j = j0 + jj;
            const size_t gi = (size_t)row * p.groups + ((j * 512 + pc * 32) >> gshift);
            sv[jj][s] = (s ? p.s1 : p.s0)[gi];
            bv[jj][s] = (s ? p.b1 : p.b0)[gi];
            const uint32_t* wr = (s ? p.w1 : p.w0) + (size_t)row * (K / 8) + j * 64 + pc * 4;
            wq[jj][s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr));
            // keep the issue order: left free, the scheduler groups the loads
            // by kind, and the first run's scales then arrive with the last
            // run's weights
            __builtin_amdgcn_sched_barrier(0);
        }

    // X is in LDS once at most the loads issued after the copies are
    // outstanding; the barrier (assembly with a memory clobber, so no LDS
    // read moves above it) then covers the other waves' copies.
    __builtin_amdgcn_s_waitcnt(vmcnt_only(R * NS * 3));
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);

    // A rows past M read row M - 1 (their outputs are dropped).  Written as
    // a select, the second block's row made the compiler wait for every
    // load before the first MFMA.
    const int xm0 = min(n, M - 1);
    const int xm1 = min(4 + n, M - 1);
    const u32x4* xr0 = xl + xm0 * (RUNS * 64) + 4 * pc;
    const u32x4* xr1 = xl + xm1 * (RUNS * 64) + 4 * pc;
    const int sw0 = xm0 & 3, sw1 = xm1 & 3;

    // two accumulator chains per (set, A block): the halves of each word
    f32x4 acc[NS][MB][2];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[s][mb][0] = acc[s][mb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int jj = 0; jj < R; ++jj) {
        const int j = j0 + jj;
        u32x4 xa[MB][4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            xa[0][r] = permute_x(xr0[j * 64 + (r ^ sw0)]);
            if constexpr (MB == 2) xa[1][r] = permute_x(xr1[j * 64 + (r ^ sw1)]);
        }
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const f16x2 s2 = as_f16x2(sv[jj][s] | (sv[jj][s] << 16));
            const f16x2 b2 = as_f16x2(bv[jj][s] | (bv[jj][s] << 16));
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const u32x4 b = dequant_word(wq[jj][s][r], s2, b2);
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    acc[s][mb][0] = mfma4(xa[mb][r][0], xa[mb][r][1], b[0], b[1], acc[s][mb][0]);
                    acc[s][mb][1] = mfma4(xa[mb][r][2], xa[mb][r][3], b[2], b[3], acc[s][mb][1]);
                }
            }
            // one (run, set) at a time, in load order: work of later runs
            // scheduled early would wait for their loads
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // ---- sum the pieces; lanes 0..3 hold the wave's partials of rows
    // row0 .. row0 + 3 ----
    float v[NS][MB][4];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[s][mb][e] = sum_pieces(acc[s][mb][0][e] + acc[s][mb][1][e]);
    if constexpr (S > 1) {
        if (ks > 0 && pc == 0) {
#pragma unroll
            for (int s = 0; s < NS; ++s)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                    for (int e = 0; e < 4; ++e) red[wave][(s * MB + mb) * 4 + e][n] = v[s][mb][e];
        }
        __syncthreads();   // every load has landed: its wait for them costs nothing
        if (ks > 0) return;
#pragma unroll
        for (int k = 1; k < S; ++k)
#pragma unroll
            for (int s = 0; s < NS; ++s)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[s][mb][e] += red[wave + k][(s * MB + mb) * 4 + e][n];
    }
    const int rn = row0 + n;
    if (pc != 0 || rn >= p.N) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int m = 4 * mb + e;
            if (m >= M) continue;
            float out;
            if constexpr (PAIR) {
                out = glu_f32(p.epilogue == kEpiGeluMul, v[0][mb][e], v[NS - 1][mb][e]);
            } else {
                out = v[0][mb][e];
                if (p.bias) out += p.bias[rn];
                if (p.epilogue == kEpiGeluTanh) out = gelu_tanh_f32(out);
            }
            const size_t oi = (size_t)m * p.N + rn;
            if (!PAIR && p.epilogue == kEpiResidual)
                reinterpret_cast<uint16_t*>(p.y)[oi] = residual_add_f16(p.residual[oi], out);
            else
                store_one(p, oi, out);
        }
}

template <int RUNS, int S, bool PAIR, int MB>
hipError_t launch_cfg(const GemmParams& p, const NarrowPlan& pl, hipStream_t st) {
    const long groups4 = (p.N + 3) / 4;   // row groups
    const dim3 grid((unsigned)((groups4 + pl.RG - 1) / pl.RG)), block(64 * S * pl.RG);
    hipLaunchKernelGGL((q4_narrow_kernel<RUNS, S, PAIR, MB>), grid, block, narrow_lds(p), st, p);
    return hipGetLastError();
}

template <int RUNS, int S>
hipError_t launch_split(const GemmParams& p, const NarrowPlan& pl, hipStream_t st) {
    if constexpr (RUNS % S != 0) {
        return hipErrorInvalidValue;
    } else {
        if (p.w1 != nullptr) {
            if constexpr (RUNS <= 10)   // the pair's weights in flight fit the registers
                return pl.MB == 1 ? launch_cfg<RUNS, S, true, 1>(p, pl, st)
                                  : launch_cfg<RUNS, S, true, 2>(p, pl, st);
            return hipErrorInvalidValue;
        }
        return pl.MB == 1 ? launch_cfg<RUNS, S, false, 1>(p, pl, st)
                          : launch_cfg<RUNS, S, false, 2>(p, pl, st);
    }
}

template <int RUNS>
hipError_t launch_runs(const GemmParams& p, const NarrowPlan& pl, hipStream_t st) {
    switch (pl.S) {
        case 1: return launch_split<RUNS, 1>(p, pl, st);
        case 2: return launch_split<RUNS, 2>(p, pl, st);
        case 4: return launch_split<RUNS, 4>(p, pl, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace

bool narrow_plan(const GemmParams& p, bool a_bf16, NarrowPlan* out) {
    if (a_bf16 || p.M < 1 || p.M > 8 || p.N < 1 || p.K <= 0 || p.K % 512 != 0) return false;
    if (p.gshift < 0 || p.gshift > 2) return false;
    const bool pair = p.w1 != nullptr;
    if (pair && p.epilogue != kEpiSiluMul && p.epilogue != kEpiGeluMul) return false;
    if (!pair && p.epilogue != kEpiNone && p.epilogue != kEpiGeluTanh &&
        p.epilogue != kEpiResidual)
        return false;
    const int runs = p.K / 512;
    switch (runs) {   // the instantiated run counts
        case 4: case 6: case 8: case 10: case 12: case 16: case 20: break;
        default: return false;
    }
    if (pair && runs > 10) return false;
    if (narrow_lds(p) > (size_t)kNarrowMaxLds) return false;
    NarrowPlan pl;
    pl.MB = p.M <= 4 ? 1 : 2;
    // split K until the launch has about 16 waves per CU
    const long groups4 = (p.N + 3) / 4;
    pl.S = 1;
    while (pl.S < 4 && groups4 * pl.S < 16L * kCUs && runs % (2 * pl.S) == 0) pl.S *= 2;
    // row groups per block: about one block per CU, at most 8 waves
    const long rg = (groups4 + kCUs - 1) / kCUs;
    const int max_rg = kNarrowMaxWaves / pl.S;
    pl.RG = (int)(rg < 1 ? 1 : rg > max_rg ? max_rg : rg);
    *out = pl;
    return true;
}

hipError_t launch_narrow(const GemmParams& p, const NarrowPlan& pl, hipStream_t st) {
    switch (p.K / 512) {
        case 4: return launch_runs<4>(p, pl, st);
        case 6: return launch_runs<6>(p, pl, st);
        case 8: return launch_runs<8>(p, pl, st);
        case 10: return launch_runs<10>(p, pl, st);
        case 12: return launch_runs<12>(p, pl, st);
        case 16: return launch_runs<16>(p, pl, st);
        case 20: return launch_runs<20>(p, pl, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace sltx
