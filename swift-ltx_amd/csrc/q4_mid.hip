// q4_mid.hip -- 4-bit dequant matmul for 16 < M <= 32 activation rows
// (T5 encoder layers at short sequence lengths, short prompts, batched
// decode) on CDNA4 MFMA, as a weight stream.
//
// Same product as q4_gemm.hip, Y[M,N] = X[M,K] . dequant(W)[N,K]^T with fp32
// accumulation (matmulQ4Fast, Ops.swift:312-381).  At these M a weight byte
// feeds at most 32 multiply-adds, so the kernel should run at the weight
// stream's rate; what it must not do is load X badly.  X is M x K fp16 (up to
// 256 KB at K = 4096) and every block needs all of it: the small-M route's
// per-wave X fragments (16 rows x 64 B per load, a K slice per wave) cost a
// CU more load issue than its weights.  Here:
//  * A block owns all K for 32 + 32 rows (gate and up of the same output
//    columns, for the gated epilogues) or 32 rows of one weight set.  It has
//    16 waves.  The 8 compute waves are 2 row tiles x 4 K-groups (gated,
//    rounds of 256 k: wave 2g + j computes row tile j over k-tile g of every
//    round) or 1 row tile x 8 K-groups (one set, rounds of 512 k: wave g over
//    k-tile g), each as one 32x32x16 MFMA tile (all 32 activation rows; rows
//    past M are copies of row M - 1, never stored).  Four copy waves copy the
//    weights, four copy X and the scales and biases, all by direct
//    global -> LDS copies in whole 128-byte lines.  One set in 32-row blocks
//    was measured faster than in 64-row blocks (2 tiles x 4 K-groups) at every
//    N tried: twice the blocks, half the weight bytes per block.
//  * Weights: the block's packed rows are copied in groups of 1024 k (512
//    contiguous bytes of two rows per wave-wide copy, the GEMV's pattern:
//    the DRAM pages of a row are read in long runs) into two LDS slots:
//    groups 0 and 1 at the start, then the slot of group G - 1 takes group
//    G + 1 once every wave is past group G - 1.  A round's compute waits
//    only for its group.  The 16-byte piece c of a row r lands at
//    c ^ (r & 15) of the row's 512 bytes, so that the fragment reads of 16
//    rows hit distinct banks.
//  * X: each round's 32 rows x 256 k, a few rounds ahead in a ring of
//    stages (the 16-byte column c of row r at c ^ (r & 7) ^ ((r >> 3) & 1)),
//    and first the block's scales and biases (one slab per array).  One
//    barrier per round hands a stage over.  Each copy role waits only for
//    its own copies: s_waitcnt counts a wave's memory operations in issue
//    order, so a wave that issued both streams would wait for weights issued
//    before the X copy it needs.
//  * Inside a k-tile the k order is permuted as in q4_gemm.hip: k-step s of
//    lane half h is packed word 4h + s of the row, so a lane's B fragments
//    over the k-tile are one 16-byte piece, dequantized in registers
//    (v_perm_b32 byte pairing, v_cvt_scalef32_pk_f16_fp8, one v_pk_fma_f16
//    per pair: s * q + b rounded once), and its A fragment is 16-byte column
//    4h + s of the X row.
//  * After the last round the four K-groups' accumulator tiles are summed in
//    LDS in a fixed order and the epilogue (gated SiLU / GELU-tanh pair,
//    bias, GELU-tanh, residual add) runs on the fp32 sums.
//  * One weight set over few blocks (N <= 4096: 128 blocks for 256 CUs) may
//    split K in two halves across blocks (SPLIT): each block stores its
//    half's sums to the workspace and the last of the two adds them, in
//    split order, and runs the epilogue (q4_split.hpp).
#include "q4_common.hpp"
#include "q4_dequant.hpp"
#include "q4_launch.hpp"
#include "q4_split.hpp"

namespace sltx {

namespace {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int NCW = 8;                     // compute waves
constexpr int NLW = 4;                     // copy waves per stream (weights, X)
constexpr int MTHREADS = 64 * (NCW + 2 * NLW);
constexpr int CTHREADS = 64 * NCW;
constexpr int LTHREADS = 64 * NLW;
constexpr int BM = 32;                     // activation rows (one MFMA tile)
constexpr size_t kMaxLds = 160 * 1024;
// Two shapes of block.  Gated pairs: 32 gate + 32 up rows, 2 row tiles x 4
// K-groups, rounds of 256 k.  KG8 (one weight set): 32 weight rows, 1 row
// tile x 8 K-groups, rounds of 512 k.  Either way a weight group is 512 bytes
// of every block row (4 or 2 rounds).
template <bool KG8>
struct MidShape {
    static constexpr int KG = KG8 ? 8 : 4;            // K-groups: k-tile g of each round
    static constexpr int RK = 64 * KG;                // k per round
    static constexpr int BROWS = KG8 ? 32 : 64;       // weight rows per block
    static constexpr int RPG = 1024 / RK;             // rounds per weight group (1024 k)
    static constexpr int XSLOTS = KG * BM * 8;        // 16-byte slots of an X stage
    static constexpr int NXC = XSLOTS / LTHREADS;     // X copies per X-copy thread per round
    static constexpr int GSLOTS = BROWS * 32;         // 16-byte slots of a weight group
    static constexpr int NWG = GSLOTS / LTHREADS;     // weight copies per W-copy thread per group
    static_assert(NXC * LTHREADS == XSLOTS && NWG * LTHREADS == GSLOTS, "whole copies");
    static_assert(RPG * RK == 1024 && 2 * KG * RPG == 32, "a group is 512 bytes of a row");
    // X ring stages: five for a gated pair (two weight slots), three for one
    // set
    static constexpr int nsx(int ng, int wsl) { return (!KG8 && wsl == 2) ? 5 : 3; }
    static constexpr size_t static_lds(int ng, int wsl) {
        return (size_t)wsl * GSLOTS * 16 + (size_t)nsx(ng, wsl) * XSLOTS * 16;
    }
    static_assert(nsx(3, 2) * XSLOTS * 4 >= NCW * 1024, "the K-group sums fit the ring");
};

__device__ __forceinline__ f32x16 mfma32_f16(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// 16-byte pieces of one scale / bias slab (rows x groups fp16), and the
// pieces reserved per slab in LDS (whole waves of 64).
__host__ __device__ constexpr int mid_slab_pieces(int rows, int groups) { return rows * groups / 8; }
__host__ __device__ constexpr int mid_slab_alloc(int rows, int groups) {
    return (mid_slab_pieces(rows, groups) + 63) / 64 * 64;
}

__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// NG weight groups of 1024 k in WSL = 2 LDS slots (the only count built):
// the slot of group G - 1 is refilled with group G + 1 once every wave has
// finished group G - 1.  SPLIT: block (x, y) covers groups y NG .. y NG +
// NG - 1 of K = 2 NG groups.
template <bool PAIR, bool KG8, int NG, int WSL, bool SPLIT>
__global__ __launch_bounds__(MTHREADS, 1) void q4_mid_kernel(GemmParams p) {
    using S = MidShape<KG8>;
    static_assert(PAIR != KG8, "gated pairs: two row tiles; one set: the 32-row block");
    static_assert(!SPLIT || KG8, "K splits: one weight set");
    constexpr int KG = S::KG, RK = S::RK, BROWS = S::BROWS, RPG = S::RPG;
    constexpr int XSLOTS = S::XSLOTS, NXC = S::NXC, GSLOTS = S::GSLOTS, NWG = S::NWG;
    constexpr int NR = NG * RPG;                // rounds
    constexpr int NSLAB = PAIR ? 4 : 2;         // s0, b0[, s1, b1]
    constexpr int SROWS = PAIR ? 32 : BROWS;    // rows per slab
    constexpr int NSX = S::nsx(NG, WSL);
    static_assert(WSL == 2 && WSL <= NG, "weight slots");
    // At the start of round q an X-copy wave has issued X(q + 1 .. q + NSX - 2)
    // after X(q).
    constexpr int WAIT_X = (NSX - 2) * NXC;
    static_assert(NSX >= 3, "rounds");
    __shared__ u32x4 wl[WSL * GSLOTS];          // weights [slot][row][32 pieces]
    __shared__ u32x4 xs[NSX * XSLOTS];          // X ring; after the loop, the K-group sums
    extern __shared__ u32x4 sb_lds[];           // [NSLAB][alloc] slabs

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = blockIdx.x * (PAIR ? 32 : BROWS);
    const int K = p.K, groups = p.groups;
    const int split = SPLIT ? (int)blockIdx.y : 0;
    const int kb = split * NG * 1024;           // this block's first k
    // scale groups of this block's K range: gblk from gbase
    const int gblk = SPLIT ? groups / 2 : groups, gbase = split * gblk;
    const int alloc = mid_slab_alloc(SROWS, gblk);
    f32x16 acc;

    if (wave >= NCW + NLW) {
        // ---- X-copy waves: the slabs, then X round by round ----
        const int lt = tid - CTHREADS - LTHREADS, lw = 64 * (wave - NCW - NLW);
        const int pieces = mid_slab_pieces(SROWS, gblk);
        const int valid = min(SROWS, p.N - n0) * gblk * 2;   // slab bytes inside the arrays
        for (int a = 0; a < NSLAB; ++a) {
            const uint16_t* arr = a == 0 ? p.s0 : a == 1 ? p.b0 : a == 2 ? p.s1 : p.b1;
            const char* src = reinterpret_cast<const char*>(arr + (size_t)n0 * groups);
            for (int c0 = lw; c0 < pieces; c0 += LTHREADS) {
                int off = (c0 + lane) * 16;
                if (off >= valid) off = 0;   // a spare copy of piece 0
                // SPLIT: the slab's row r is groups gbase .. of row n0 + r
                if (SPLIT) off = (off / (gblk * 2)) * (groups * 2) + gbase * 2 + off % (gblk * 2);
                __builtin_amdgcn_global_load_lds((const void*)(src + off),
                                                 (lds_ptr_t)(sb_lds + a * alloc + c0), 16, 0, 0);
            }
        }
        // X slot s of a stage: k-tile s / 256, row (s / 8) % 32, physical
        // column s % 8, i.e. logical column (s % 8) ^ (row & 7) ^ ((row >> 3) & 1)
        const uint16_t* A = reinterpret_cast<const uint16_t*>(p.a);
        const uint16_t* x_src[NXC];
#pragma unroll
        for (int i = 0; i < NXC; ++i) {
            const int s = lt + LTHREADS * i;
            const int kt = s / (BM * 8), row = (s >> 3) & (BM - 1);
            const int c16 = (s & 7) ^ (row & 7) ^ ((row >> 3) & 1);
            x_src[i] = A + (size_t)min(row, p.M - 1) * K + kb + kt * 64 + c16 * 8;
        }
        const char* spare_src = reinterpret_cast<const char*>(p.a) + lane * 4;
        auto issue_x = [&](int q) {   // NXC vector-memory ops
            if (q < NR) {
                u32x4* st = xs + (q % NSX) * XSLOTS + lw;
#pragma unroll
                for (int i = 0; i < NXC; ++i)
                    __builtin_amdgcn_global_load_lds((const void*)(x_src[i] + (size_t)q * RK),
                                                     (lds_ptr_t)(st + LTHREADS * i), 16, 0, 0);
            } else {
                // past the last round: 256 bytes per wave into the stage
                // round q - NSX + 1 read, which no later round reads
                uint32_t* spare_dst = reinterpret_cast<uint32_t*>(xs + (q % NSX) * XSLOTS) + lw;
#pragma unroll
                for (int i = 0; i < NXC; ++i)
                    __builtin_amdgcn_global_load_lds((const void*)spare_src, (lds_ptr_t)spare_dst, 4, 0, 0);
            }
        };
        for (int q = 0; q < NSX - 1; ++q) issue_x(q);
        for (int q = 0; q < NR; ++q) {
            __builtin_amdgcn_s_waitcnt(vmcnt_only(WAIT_X));
            lds_barrier();
            issue_x(q + NSX - 1);   // into the stage round q - 1 read
        }
        __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    } else if (wave >= NCW) {
        // ---- W-copy waves: every group at once, then one wait per group ----
        // Copy i of group G covers rows 2c, 2c + 1 (c = wave index + 4 i),
        // lane l: row 2c + l / 32, the row's piece (l % 32) ^ (row & 15) of
        // the group's 512 bytes, landing in slot l of the copy.
        const int lw = wave - NCW;
        const uint32_t* w_src[NWG];
#pragma unroll
        for (int i = 0; i < NWG; ++i) {
            const int row = 2 * (lw + NLW * i) + (lane >> 5);
            const uint32_t* W = (PAIR && row >= 32) ? p.w1 : p.w0;
            int n = PAIR ? n0 + (row & 31) : n0 + row;
            if (n >= p.N) n = 0;   // rows past N read row 0 (never stored)
            w_src[i] = W + (size_t)n * (K / 8) + kb / 8 + (((lane & 31) ^ (row & 15)) * 4);
        }
        auto issue_w = [&](int G) {   // NWG vector-memory ops: group G into slot G % WSL
            u32x4* slot = wl + (G % WSL) * GSLOTS;
#pragma unroll
            for (int i = 0; i < NWG; ++i)
                __builtin_amdgcn_global_load_lds((const void*)(w_src[i] + (size_t)G * 128),
                                                 (lds_ptr_t)(slot + 64 * (lw + NLW * i)), 16, 0, 0);
        };
        for (int G = 0; G < WSL; ++G) issue_w(G);
        for (int q = 0; q < NR; ++q) {
            const int G = q / RPG;
            if (q % RPG == 0) {
                // group G landed.  Issued after it: groups 1 .. WSL - 1 at
                // G = 0; later only group G + WSL - 2 (issued at the start of
                // group G - 1), if it exists and is not G itself
                const int later = G == 0 ? WSL - 1 : min(NG - 1 - G, WSL - 2);
                if (later == 0) __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
                else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_only(NWG));
                else __builtin_amdgcn_s_waitcnt(vmcnt_only(2 * NWG));
            }
            lds_barrier();
            // every wave is past group G - 1: its slot takes group G + WSL - 1
            if (q % RPG == 0 && G >= 1 && G + WSL - 1 < NG) issue_w(G + WSL - 1);
        }
    } else {
        // ---- compute waves ----
        const int j = KG8 ? 0 : wave & 1;        // row tile
        const int g = KG8 ? wave : wave >> 1;    // K-group
        const int r = lane & 31, h = lane >> 5;  // MFMA row / column, k half
        const int wrow = 32 * j + r;             // block row

        // this lane's scale / bias: slab (2e, 2e + 1), row srow, group of k
        // q * 256 + 64 g + 32 h
        const uint16_t* sbl = reinterpret_cast<const uint16_t*>(sb_lds);
        const int e = PAIR ? j : 0, srow = PAIR ? r : 32 * j + r;
        const uint16_t* s_row = sbl + (size_t)(2 * e) * alloc * 8 + srow * gblk;
        const uint16_t* b_row = s_row + (size_t)alloc * 8;
        const int glog2 = 5 + p.gshift;
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
#pragma unroll
        for (int q = 0; q < NR; ++q) {
            lds_barrier();
            const u32x4* xst = xs + (q % NSX) * XSLOTS + g * (BM * 8);
            const u32x4 wpc = wl[((q / RPG) % WSL) * GSLOTS + wrow * 32 +
                                 ((2 * KG * (q % RPG) + 2 * g + h) ^ (wrow & 15))];
            const int gi = (q * RK + 64 * g + 32 * h) >> glog2;   // of the block's groups
            const uint32_t sv = s_row[gi], bv = b_row[gi];
            const f16x2 s2 = as_f16x2(sv | (sv << 16));
            const f16x2 b2 = as_f16x2(bv | (bv << 16));
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const u32x4 a = xst[swz(r, 4 * h + s)];
                acc = mfma32_f16(a, dequant_word_f16(wpc[s], s2, b2), acc);
            }
        }
    }

    // ---- sum the K-groups' tiles (LDS, fixed order), epilogue ----
    __syncthreads();   // every copy landed, every ring read done
    float* red = reinterpret_cast<float*>(xs);   // wave w's tile at [w][v][lane]
    if (wave < NCW) {
#pragma unroll
        for (int v = 0; v < 16; ++v) red[wave * 1024 + v * 64 + lane] = acc[v];
    }
    __syncthreads();

    // D[m][c] of a 32x32 tile is element 4 (m / 8) + m % 4 of lane
    // c + 32 ((m / 4) % 2)
    constexpr int NCOLS = PAIR ? 32 : BROWS;
    static_assert(!SPLIT || BM * NCOLS == MTHREADS, "a split block: one output per thread");
    for (int o = tid; o < BM * NCOLS; o += MTHREADS) {
        const int m = o / NCOLS, c = o % NCOLS;
        const int n = n0 + c;
        const bool valid = m < p.M && n < p.N;
        if (!SPLIT && !valid) continue;
        const int jj = (PAIR || KG8) ? 0 : c >> 5;
        const int idx = (4 * (m >> 3) + (m & 3)) * 64 + (c & 31) + 32 * ((m >> 2) & 1);
        // the tile of (K-group gg, row tile t) is wave 2 gg + t (KG8: wave gg)
        auto wv = [&](int gg, int t) { return KG8 ? gg : 2 * gg + t; };
        float v0 = 0.0f, v1 = 0.0f;
#pragma unroll
        for (int gg = 0; gg < KG; ++gg) {
            v0 += red[wv(gg, jj) * 1024 + idx];
            if constexpr (PAIR) v1 += red[wv(gg, 1) * 1024 + idx];
        }
        if constexpr (SPLIT) {
            // this half's sum to the workspace; the block that arrives second
            // loads the other half's and adds the two in split order
            const __amdgpu_buffer_rsrc_t rs = ws_rsrc(p.ws);
            if (valid) store_f32v_sc1<1>(rs, ((size_t)split * p.M + m) * p.N, n, p.N, &v0);
            if (!split_arrive_last(p.tickets + blockIdx.x, 2)) return;
            if (!valid) return;
            float other;
            load_f32v_sc1<1>(rs, ((size_t)(1 - split) * p.M + m) * p.N, n, p.N, &other);
            float sum = 0.0f;
            sum += split == 0 ? v0 : other;
            sum += split == 0 ? other : v0;
            v0 = sum;
        }
        float out;
        if constexpr (PAIR) {
            out = glu_f32(p.epilogue == kEpiGeluMul, v0, v1);
        } else {
            out = v0;
            if (p.bias) out += p.bias[n];
            if (p.epilogue == kEpiGeluTanh) out = gelu_tanh_f32(out);
        }
        const size_t oi = (size_t)m * p.N + n;
        if (!PAIR && p.epilogue == kEpiResidual)
            reinterpret_cast<uint16_t*>(p.y)[oi] = residual_add_f16(p.residual[oi], out);
        else
            store_one(p, oi, out);
    }
}

// Dynamic LDS: the scale / bias slabs (32 rows each, the groups of a
// block's K range)
size_t mid_lds(const GemmParams& p, bool pair, int splits = 1) {
    return (size_t)(pair ? 4 : 2) * mid_slab_alloc(32, p.groups / splits) * 16;
}

size_t mid_static_lds(int ng, int wsl, bool pair) {
    return pair ? MidShape<false>::static_lds(ng, wsl) : MidShape<true>::static_lds(ng, wsl);
}

// (groups, slots) built: two slots, gated pairs at K = 2048, 3072, 4096 (with
// five X stages), one set at K = 2048 .. 10240.  At M = 32 three slots
// measured slower: 32.8 us against 31.6 on the T5 GeGLU pair, 9.90 against
// 9.61 on T5 q/k/v/o, 6.65 against 6.51 on Llama q|k|v; the Llama gate/up
// pair with the whole K in three slots and three X stages 11.6 against 11.0.
bool mid_built(bool pair, int ng, int wsl) {
    if (pair) return (ng == 2 || ng == 3 || ng == 4) && wsl == 2;
    return wsl == 2 && (ng == 2 || ng == 3 || ng == 4 || ng == 8 || ng == 10);
}

// Weight-group slots: 2, refilled as the groups are used, when that build
// exists for K and fits LDS beside the X ring and the slabs; 0 otherwise.
int mid_wsl(const GemmParams& p, bool pair) {
    const int ng = p.K / 1024;
    if (mid_built(pair, ng, 2) && mid_static_lds(ng, 2, pair) + mid_lds(p, pair) <= kMaxLds)
        return 2;
    return 0;
}

template <bool PAIR, bool KG8, int NG, int WSL, bool SPLIT = false>
hipError_t launch_cfg(const GemmParams& p, const dim3& grid, size_t lds, hipStream_t st) {
    hipLaunchKernelGGL((q4_mid_kernel<PAIR, KG8, NG, WSL, SPLIT>), grid, dim3(MTHREADS), lds, st,
                       p);
    return hipGetLastError();
}

hipError_t launch_sel(const GemmParams& p, bool pair, int wsl, const dim3& grid, size_t lds,
                      hipStream_t st) {
    const int ng = p.K / 1024;
    if (grid.y == 2) {   // K in two halves (one set)
        switch (ng / 2) {
            case 2: return launch_cfg<false, true, 2, 2, true>(p, grid, lds, st);
            case 4: return launch_cfg<false, true, 4, 2, true>(p, grid, lds, st);
            case 5: return launch_cfg<false, true, 5, 2, true>(p, grid, lds, st);
        }
        return hipErrorInvalidValue;
    }
    if (pair) {
        if (ng == 2) return launch_cfg<true, false, 2, 2>(p, grid, lds, st);
        if (ng == 3) return launch_cfg<true, false, 3, 2>(p, grid, lds, st);
        if (ng == 4) return launch_cfg<true, false, 4, 2>(p, grid, lds, st);
        return hipErrorInvalidValue;
    }
    switch (ng * 4 + wsl) {
        case 2 * 4 + 2: return launch_cfg<false, true, 2, 2>(p, grid, lds, st);
        case 3 * 4 + 2: return launch_cfg<false, true, 3, 2>(p, grid, lds, st);
        case 4 * 4 + 2: return launch_cfg<false, true, 4, 2>(p, grid, lds, st);
        case 8 * 4 + 2: return launch_cfg<false, true, 8, 2>(p, grid, lds, st);
        case 10 * 4 + 2: return launch_cfg<false, true, 10, 2>(p, grid, lds, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace

bool mid_plan(const GemmParams& p, bool a_bf16) {
    if (a_bf16 || p.M < 1 || p.M > BM || p.N < 1) return false;
    if (p.K <= 0 || p.K % 1024 != 0) return false;
    // whole 16-byte slab pieces per row group of 8 (the last block's slab
    // stops at a piece boundary: no copy reads past the arrays)
    if (p.gshift < 0 || p.gshift > 2 || p.groups % 8 != 0) return false;
    const bool pair = p.w1 != nullptr;
    if (pair && p.epilogue != kEpiSiluMul && p.epilogue != kEpiGeluMul) return false;
    if (!pair && p.epilogue != kEpiNone && p.epilogue != kEpiGeluTanh &&
        p.epilogue != kEpiResidual)
        return false;
    if (mid_wsl(p, pair) == 0) return false;
    // 16-byte loads and copies: X rows, W rows and the scale / bias slabs
    uintptr_t al = reinterpret_cast<uintptr_t>(p.a) | reinterpret_cast<uintptr_t>(p.w0) |
                   reinterpret_cast<uintptr_t>(p.s0) | reinterpret_cast<uintptr_t>(p.b0);
    if (pair)
        al |= reinterpret_cast<uintptr_t>(p.w1) | reinterpret_cast<uintptr_t>(p.s1) |
              reinterpret_cast<uintptr_t>(p.b1);
    return (al & 15) == 0;
}

// K in two halves across blocks for one weight set whose 32-row blocks would
// fill at most half of the CUs, where the half-K kernel is built (K = 4096,
// 8192, 10240).
int mid_splits(const GemmParams& p) {
    if (p.w1 != nullptr) return 1;
    const int nblocks = (p.N + 31) / 32, ng = p.K / 1024;
    if (2 * nblocks > kCUs || ng % 2 != 0) return 1;
    const int half = ng / 2;
    if (half != 2 && half != 4 && half != 5) return 1;
    // whole 16-byte slab pieces per row; the arrival flag's LDS beside the rest
    if ((p.groups / 2) % 8 != 0 ||
        mid_static_lds(ng, 2, false) + 256 + mid_lds(p, false, 2) > kMaxLds)
        return 1;
    return 2;
}

size_t mid_ws_bytes(const GemmParams& p, int splits) {
    return splits > 1 ? (size_t)splits * p.M * p.N * sizeof(float) : 0;
}

hipError_t launch_mid(const GemmParams& p, int splits, hipStream_t st) {
    const bool pair = p.w1 != nullptr;
    const unsigned nblocks = (unsigned)((p.N + 31) / 32);   // 32 output columns per block
    if (splits != 1 && (splits != 2 || pair || !p.ws || !p.tickets ||
                        nblocks > (unsigned)kTickets || mid_ws_bytes(p, splits) > 0x7fffffffu))
        return hipErrorInvalidValue;
    const dim3 grid(nblocks, (unsigned)splits);
    return launch_sel(p, pair, mid_wsl(p, pair), grid, mid_lds(p, pair, splits), st);
}

}  // namespace sltx
