// q4_narrow.hip -- 4-bit dequant matmul for M <= 4 activation rows and one
// weight set (short prompts, batched decode, the T5 encoder at a few
// tokens) on CDNA4's 4x4x4 MFMA blocks, as a weight stream shaped like the
// GEMV.
//
// Same product as q4_gemm.hip, Y[M,N] = X[M,K] . dequant(W)[N,K]^T with the
// weights dequantized to fp16 (s * q + b, one rounding) and fp32 accumulation
// (matmulQ4Fast, Ops.swift:312-381).  At M <= 4 each weight byte feeds at
// most 4 multiply-adds: the launch is bound by the weight stream, and what
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
//  * A wave owns 4 weight rows and 1/S of the runs of K, with every load in
//    flight before the first MFMA, in use order.  S (1, 2 or 4) is chosen
//    so the launch has about 16 waves per CU: a wave's loads come back close
//    together, behind those of the waves that started before it, so what is
//    left after the last load lands is one wave's dequantization, and
//    smaller waves leave less.  The 16 per-piece partials are summed across
//    lanes (DPP row rotations, then two cross-row shuffles), and the S waves
//    of a row group add theirs through LDS, in a fixed order.
//  * X's M rows are copied once per block to LDS (direct 16-byte copies,
//    1 KB per wave-wide copy).  Piece c of row m is stored at position
//    c ^ m of its 1 KB chunk, so a fragment read -- 4 pieces of 4 rows per
//    16 lanes -- hits 16 distinct bank groups.  A rows past M read row
//    M - 1: their outputs are never stored.
//  * Each weight word is dequantized in registers (q4_dequant.hpp) into two
//    B fragments of 4 k: 2 MFMAs of ~8 cycles per word, the same matrix time
//    as one 16x16x32 MFMA.  The dequantization (~57 cycles of VALU per
//    wave-word) is the compute bound.
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

// RUNS 512-k runs of K split over S waves.  A block is W = S * RG waves: RG
// row groups of 4 rows.
template <int RUNS, int S>
__global__ __launch_bounds__(64 * kNarrowMaxWaves) void q4_narrow_kernel(GemmParams p) {
    constexpr int R = RUNS / S;   // runs per wave
    static_assert(RUNS % S == 0, "runs split evenly");
    extern __shared__ u32x4 xl[];   // X rows [M][RUNS chunks of 64 pieces]
    __shared__ float red[kNarrowMaxWaves][4][4];   // partials of waves ks > 0
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, W = blockDim.x >> 6;
    const int n = lane & 3, pc = lane >> 2;
    const int rg = wave / S, ks = wave - rg * S;
    const int K = p.K, M = p.M;

    // ---- X rows [0, M) -> LDS, one 1 KB chunk per wave-wide copy ----
    for (int c = wave; c < M * RUNS; c += W) {   // wave-uniform
        const int m = c / RUNS, j = c - m * RUNS;
        const char* src = reinterpret_cast<const char*>(p.a) + ((size_t)m * K + j * 512) * 2 +
                          (lane ^ m) * 16;
        __builtin_amdgcn_global_load_lds((const void*)src, (lds_ptr_t)(xl + c * 64), 16, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- the wave's rows and runs: scale, bias and packed words per run, in
    // use order ----
    const int row0 = (blockIdx.x * (W / S) + rg) * 4;
    const int row = min(row0 + n, p.N - 1);   // clamped rows are computed and dropped
    const int gshift = 5 + p.gshift;          // log2(group size)
    const int j0 = ks * R;
    u32x4 wq[R];
    uint32_t sv[R], bv[R];
#pragma unroll
    for (int jj = 0; jj < R; ++jj) {
        const int j = j0 + jj;
        const size_t gi = (size_t)row * p.groups + ((j * 512 + pc * 32) >> gshift);
        sv[jj] = p.s0[gi];
        bv[jj] = p.b0[gi];
        const uint32_t* wr = p.w0 + (size_t)row * (K / 8) + j * 64 + pc * 4;
        wq[jj] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr));
        // keep the issue order: left free, the scheduler groups the loads by
        // kind, and the first run's scales then arrive with the last run's
        // weights
        __builtin_amdgcn_sched_barrier(0);
    }

    // X is in LDS once at most the loads issued after the copies are
    // outstanding; the barrier (assembly with a memory clobber, so no LDS
    // read moves above it) then covers the other waves' copies.
    __builtin_amdgcn_s_waitcnt(vmcnt_only(R * 3));
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);

    // A rows past M read row M - 1 (their outputs are dropped).
    const int xm = min(n, M - 1);
    const u32x4* xr = xl + xm * (RUNS * 64) + 4 * pc;

    // two accumulator chains: the halves of each word
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int jj = 0; jj < R; ++jj) {
        const int j = j0 + jj;
        u32x4 xa[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) xa[r] = permute_x(xr[j * 64 + (r ^ xm)]);
        const f16x2 s2 = as_f16x2(sv[jj] | (sv[jj] << 16));
        const f16x2 b2 = as_f16x2(bv[jj] | (bv[jj] << 16));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const u32x4 b = dequant_word(wq[jj][r], s2, b2);
            acc0 = mfma4(xa[r][0], xa[r][1], b[0], b[1], acc0);
            acc1 = mfma4(xa[r][2], xa[r][3], b[2], b[3], acc1);
        }
        // one run at a time, in load order: work of later runs scheduled
        // early would wait for their loads
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- sum the pieces; lanes 0..3 hold the wave's partials of rows
    // row0 .. row0 + 3, activation row e in element e ----
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = sum_pieces(acc0[e] + acc1[e]);
    if constexpr (S > 1) {
        if (ks > 0 && pc == 0) {
#pragma unroll
            for (int e = 0; e < 4; ++e) red[wave][e][n] = v[e];
        }
        __syncthreads();   // every load has landed: its wait for them costs nothing
        if (ks > 0) return;
#pragma unroll
        for (int k = 1; k < S; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] += red[wave + k][e][n];
    }
    const int rn = row0 + n;
    if (pc != 0 || rn >= p.N) return;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        if (m >= M) break;
        float out = v[m];
        if (p.bias) out += p.bias[rn];
        if (p.epilogue == kEpiGeluTanh) out = gelu_tanh_f32(out);
        const size_t oi = (size_t)m * p.N + rn;
        if (p.epilogue == kEpiResidual)
            reinterpret_cast<uint16_t*>(p.y)[oi] = residual_add_f16(p.residual[oi], out);
        else
            store_one(p, oi, out);
    }
}

template <int RUNS, int S>
hipError_t launch_cfg(const GemmParams& p, const NarrowPlan& pl, hipStream_t st) {
    if constexpr (RUNS % S != 0) {
        return hipErrorInvalidValue;
    } else {
        const long groups4 = (p.N + 3) / 4;   // row groups
        const dim3 grid((unsigned)((groups4 + pl.RG - 1) / pl.RG)), block(64 * S * pl.RG);
        hipLaunchKernelGGL((q4_narrow_kernel<RUNS, S>), grid, block, narrow_lds(p), st, p);
        return hipGetLastError();
    }
}

template <int RUNS>
hipError_t launch_runs(const GemmParams& p, const NarrowPlan& pl, hipStream_t st) {
    switch (pl.S) {
        case 1: return launch_cfg<RUNS, 1>(p, pl, st);
        case 2: return launch_cfg<RUNS, 2>(p, pl, st);
        case 4: return launch_cfg<RUNS, 4>(p, pl, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace

bool narrow_plan(const GemmParams& p, bool a_bf16, NarrowPlan* out) {
    if (a_bf16 || p.w1 != nullptr || p.M < 1 || p.M > 4 || p.N < 1 || p.K <= 0 ||
        p.K % 512 != 0)
        return false;
    if (p.gshift < 0 || p.gshift > 2) return false;
    if (p.epilogue != kEpiNone && p.epilogue != kEpiGeluTanh && p.epilogue != kEpiResidual)
        return false;
    switch (p.K / 512) {   // the instantiated run counts
        case 4: case 6: case 8: case 10: case 12: case 16: case 20: break;
        default: return false;
    }
    if (narrow_lds(p) > (size_t)kNarrowMaxLds) return false;
    const int runs = p.K / 512;
    NarrowPlan pl;
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
