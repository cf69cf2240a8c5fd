// q4_gemm.hip -- 4-bit dequant GEMM (prefill / DiT, M > 1) on CDNA4 MFMA.
//
// Y[M,N] = A[M,K] . dequant(W)[N,K]^T, fp32 accumulate, where
// dequant(W)[n,k] = s[n,k/g]*q[n,k] + b[n,k/g].  This is the computation
// swift-ltx routes through matmulQ4Fast / matmulQ4FastF32 (Ops.swift:312-381),
// whose quantized-B GEMM kernel lives in an external package.  The SILU_MUL
// epilogue fuses linear(gate), linear(up) and siluMul
// (LlamaModel.swift:275-277); the bias + GELU-tanh epilogue covers
// DiTLinear.applyF32in + geluApproximateF32 (DiTModel.swift:102-125, :953).
//
// Block: 512 threads = 8 waves in a 2 (M) x 4 (N) layout; block tile
// BM x 256 x 64 with BM = 64*WM (WM = 2 or 3), each wave computing
// (32*WM) x 64 with v_mfma_f32_32x32x16_{f16,bf16} (WM x 2 accumulator tiles).
//  * A tile (BM x 64, fp16 or bf16) is copied global -> LDS directly
//    (global_load_lds_dwordx4) into a 3-stage ring, two tiles ahead.
//  * W tile (256 rows x 64 nibbles = 32 B per row) is loaded one 16-byte
//    chunk per thread, dequantized in registers to fp16 (or bf16) with its
//    group's scale and bias, and written to LDS: dequantized once per block
//    and shared by both M-waves.  fp16: nibbles are spread to bytes, paired
//    with v_perm_b32, turned into 1024+q by mantissa insertion, reduced to q
//    exactly, then one fp16 FMA q*s+b (a single rounding).  bf16: q*s+b in
//    fp32, rounded once to bf16.
//  * LDS rows are 128 bytes with an XOR swizzle of the 16-byte columns (see
//    swz) that keeps the MFMA operand reads and the tile stores free of bank
//    conflicts.
//  * W goes through two staging register sets: tile k+2 is loaded while
//    tile k is multiplied, and tile k+1 (loaded one iteration earlier) is
//    dequantized into the other of two W stages between the k-steps of tile
//    k's MFMAs; one barrier per k-tile.
//  * Tile order is XCD-aware: the 8 XCDs receive workgroups round-robin, so
//    consecutive logical tiles (M fastest) are mapped to one XCD so that the
//    M-blocks sharing a weight column block share that XCD's L2.
//  * BM is chosen per launch so the tile count fills the 256 CUs in whole
//    rounds (M = 750: BM = 192 gives 4 x 64 = 256 tiles for gate/up).
#include <type_traits>

#include "q4_common.hpp"
#include "q4_launch.hpp"

namespace sltx {

constexpr int BN = 256, BK = 64;
constexpr int kThreads = 512;
constexpr int kCUs = 256;

// LDS layout of a 64-wide k-tile: 128-byte rows of eight 16-byte columns.
// Logical column c of row r sits at physical column c ^ (r & 7) ^ ((r >> 3) & 1).
// A ds_read_b128 is served 16 lanes at a time by 64 4-byte banks (256 B): the
// MFMA operand reads (16 consecutive rows, one logical column) and the tile
// stores then hit 16 distinct (row parity, column) slots, i.e. no bank
// conflicts; any 8 consecutive rows also land in 8 distinct columns.
__device__ __forceinline__ int swz(int row, int col16) {
    return row * 8 + (col16 ^ (row & 7) ^ ((row >> 3) & 1));
}

// One 32-bit word (8 nibbles, k order) -> 8 fp16 values s*q+b.  Nibbles are
// spread to bytes, paired with v_perm_b32, turned into 1024+q by mantissa
// insertion, reduced to q exactly, then one fp16 FMA q*s+b (one rounding).
__device__ __forceinline__ u32x4 dequant_word_f16(uint32_t w, f16x2 s2, f16x2 b2) {
    const f16x2 m1024 = {(f16)-1024.0f, (f16)-1024.0f};
    const uint32_t lo = w & 0x0F0F0F0Fu;          // bytes q6 q4 q2 q0
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;   // bytes q7 q5 q3 q1
    uint32_t pr[4];
    pr[0] = __builtin_amdgcn_perm(hi, lo, 0x0C040C00u) | kMagic1024x2;  // q0, q1
    pr[1] = __builtin_amdgcn_perm(hi, lo, 0x0C050C01u) | kMagic1024x2;  // q2, q3
    pr[2] = __builtin_amdgcn_perm(hi, lo, 0x0C060C02u) | kMagic1024x2;  // q4, q5
    pr[3] = __builtin_amdgcn_perm(hi, lo, 0x0C070C03u) | kMagic1024x2;  // q6, q7
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const f16x2 q = as_f16x2(pr[e]) + m1024;               // exact small integers
        o[e] = as_u32(__builtin_elementwise_fma(q, s2, b2));    // v_pk_fma_f16
    }
    return o;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
}

// One word -> 8 bf16 values bf16(s*q+b), q*s+b computed with one fp32 FMA.
__device__ __forceinline__ u32x4 dequant_word_bf16(uint32_t w, float s, float b) {
    const uint32_t lo = w & 0x0F0F0F0Fu;
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float q0 = (float)((lo >> (8 * e)) & 0xFFu);
        const float q1 = (float)((hi >> (8 * e)) & 0xFFu);
        o[e] = pack_bf16x2(fmaf(q0, s, b), fmaf(q1, s, b));
    }
    return o;
}

template <bool BF16>
__device__ __forceinline__ f32x16 mfma32(const u32x4 a, const u32x4 b, f32x16 c) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ void store_out(const GemmParams& p, size_t o, float v) {
    if (p.y_dtype == kF32)
        reinterpret_cast<float*>(p.y)[o] = v;
    else if (p.y_dtype == kBF16)
        reinterpret_cast<uint16_t*>(p.y)[o] = f2bf(v);
    else
        reinterpret_cast<uint16_t*>(p.y)[o] = f2h(v);
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt bits [3:0] and [15:14], expcnt [6:4] = 7, lgkmcnt [11:8] = 15).
#define SLTX_WAIT_VMCNT(n) \
    __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))

typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <int WM, bool BF16, bool SILU, bool KTAIL, bool SPLIT>
__global__ __launch_bounds__(kThreads, 1) void q4_gemm_kernel(GemmParams p) {
    constexpr int BM = 64 * WM;
    constexpr int NSA = WM == 2 ? 3 : 2;       // A stages (LDS budget)
    constexpr int A_STAGE = BM * BK / 8;       // 16-byte slots per A stage
    constexpr int W16_STAGE = BN * BK / 8;     // dequantized W, one k-tile
    constexpr int WP_STAGE = BN * 4;           // packed W, two k-tiles (64 B per row)
    constexpr int GPMAX = 4;                   // scale/bias groups per row per super-stage
    __shared__ u32x4 lds_a[NSA * A_STAGE];     // swizzled [row][col16]
    __shared__ u32x4 lds_w16[2 * W16_STAGE];   // swizzled [row][col16]
    __shared__ u32x4 lds_wp[2 * WP_STAGE];     // swizzled [row][piece]
    __shared__ uint16_t lds_sb[2][2][BN * GPMAX];   // [stage][scale|bias][row * GP + g]

    // ---- tile selection (XCD-aware) ----
    const int ntiles = p.tiles_m * p.tiles_n;
    int logical = blockIdx.x;
    if ((gridDim.x & 7) == 0) {
        const int per_xcd = gridDim.x >> 3;
        logical = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    }
    if (logical >= ntiles * (SPLIT ? p.splits : 1)) return;
    const int split = SPLIT ? logical / ntiles : 0;
    const int tile = SPLIT ? logical % ntiles : logical;
    const int tile_m = tile % p.tiles_m;
    const int tile_n = tile / p.tiles_m;
    // K range of this block: k-tiles [kb, kb + nk); Kl = its extent in k.
    const int nk_all = (p.K + BK - 1) / BK;
    const int kb = SPLIT ? split * p.split_tiles : 0;
    const int nk = SPLIT ? min(p.split_tiles, nk_all - kb) : nk_all;
    const int Kl = min(p.K - kb * BK, nk * BK);
    const int m0 = tile_m * BM;
    // SILU: a tile covers 128 output columns, as 128 gate rows + 128 up rows.
    const int n0 = tile_n * (SILU ? BN / 2 : BN);

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int GP = 4 >> p.gshift;   // scale/bias groups per 128 k (g = 32, 64, 128)

    // Virtual W row -> matrix row (and which matrix, for SILU).  Rows past N
    // are clamped to row 0: computed, never stored.
    auto wrow = [&](int v, const uint32_t*& W, const uint16_t*& S, const uint16_t*& B) {
        int n;
        if (SILU) {
            const int tn = (v >> 5) & 1;
            n = n0 + (v >> 6) * 32 + (v & 31);
            W = tn ? p.w1 : p.w0;
            S = tn ? p.s1 : p.s0;
            B = tn ? p.b1 : p.b0;
        } else {
            n = n0 + v;
            W = p.w0;
            S = p.s0;
            B = p.b0;
        }
        return n < p.N ? n : 0;
    };

    // ---- A: direct global -> LDS (global_load_lds_dwordx4) ----
    // Each wave fills WM 1-KB pieces of a stage: piece i covers slots
    // (wave + 8 i) * 64 .. +63, lane l landing in slot +l.  Slot s is physical
    // column s % 8 of row s / 8, i.e. logical column (s % 8) ^ xor(row): the
    // swizzle is applied on the global side.  Rows past M are clamped to M-1.
    const uint16_t* A = reinterpret_cast<const uint16_t*>(p.a);
    const uint16_t* a_src[WM];
    int a_col8[WM];
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        const int slot = (wave + 8 * i) * 64 + lane;
        const int row = slot >> 3;
        const int c16 = (slot & 7) ^ (row & 7) ^ ((row >> 3) & 1);
        const int m = m0 + row;
        a_col8[i] = c16 * 8;
        a_src[i] = A + (size_t)(m < p.M ? m : p.M - 1) * p.K + kb * BK + c16 * 8;
    }

    // ---- packed W: direct global -> LDS, two k-tiles (64 B per row) ----
    // Four lanes cover a row's 64 bytes, so each wave-wide copy reads 16 rows
    // of 64 contiguous bytes.  Slot s is row s / 4, physical piece s % 4 =
    // logical piece ^ ((row >> 2) & 3) (conflict-free reads below).
    const uint32_t* wp_src[2];
    int wp_piece[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int slot = (wave + 8 * i) * 64 + lane;
        const int row = slot >> 2;
        const int piece = (slot & 3) ^ ((row >> 2) & 3);
        const uint32_t* W;
        const uint16_t *S, *B;
        const int n = wrow(row, W, S, B);
        wp_piece[i] = piece;
        wp_src[i] = W + (size_t)n * (p.K / 8) + kb * (BK / 8) + piece * 4;
    }

    // ---- scales / biases: GP groups per row per super-stage ----
    // Threads 0-255 load scales, 256-511 biases; consecutive threads read
    // consecutive groups of a row.  Values land in registers and are written
    // to LDS one k-tile later.
    const int sb_arr = tid >> 8;
    const uint16_t* sb_src[GPMAX];
    int sb_dst[GPMAX];
#pragma unroll
    for (int u = 0; u < GPMAX; ++u) {
        const int v = (tid & 255) + 256 * u;
        const int row = v / GP, g = v % GP;
        const uint32_t* W;
        const uint16_t *S, *B;
        const int n = wrow(row < BN ? row : 0, W, S, B);
        sb_src[u] = (sb_arr ? B : S) + (size_t)n * p.groups + ((2 * kb) >> p.gshift) + g;
        sb_dst[u] = v;
    }

    // ---- dequant assignment: virtual row vr, half whalf (wave-uniform) ----
    const int vr = tid & 255, whalf = tid >> 8;

    const int nss = (nk + 1) / 2;   // super-stages

    auto load_a = [&](int kt) {   // WM vector-memory ops
        const int k0 = kt * BK;
        u32x4* stage = lds_a + (kt % NSA) * A_STAGE;
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            int off = k0;
            if (KTAIL && k0 + a_col8[i] >= Kl) off = Kl - 8 - a_col8[i];
            __builtin_amdgcn_global_load_lds((const void*)(a_src[i] + off),
                                             (lds_ptr_t)(stage + (wave + 8 * i) * 64), 16, 0, 0);
        }
    };
    auto zero_a_tail = [&](int kt) {   // after the copy for tile kt landed
        const int k0 = kt * BK;
        if (!KTAIL || k0 + BK <= Kl) return;
        u32x4* stage = lds_a + (kt % NSA) * A_STAGE;
        const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < WM; ++i)
            if (k0 + a_col8[i] >= Kl) stage[(wave + 8 * i) * 64 + lane] = z;
    };
    auto load_wp = [&](int ss) {   // 2 vector-memory ops
        u32x4* stage = lds_wp + (ss & 1) * WP_STAGE;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            int off = ss * 16;   // u32 words: 64 bytes per super-stage
            if (KTAIL && (ss * 128 + wp_piece[i] * 32) >= Kl) off = (Kl / 8) - 4 - wp_piece[i] * 4;
            __builtin_amdgcn_global_load_lds((const void*)(wp_src[i] + off),
                                             (lds_ptr_t)(stage + (wave + 8 * i) * 64), 16, 0, 0);
        }
    };
    uint32_t sbr[GPMAX];
    auto load_sb = [&](int ss) {   // GPMAX vector-memory ops (the first GP are used)
#pragma unroll
        for (int u = 0; u < GPMAX; ++u) {
            int g = ss * GP;
            const int groups_l = p.groups - ((2 * kb) >> p.gshift);
            if (KTAIL && g + (sb_dst[u] % GP) >= groups_l) g = groups_l - 1 - (sb_dst[u] % GP);
            sbr[u] = sb_src[u][g];   // unused slots read an in-bounds element
        }
    };
    auto store_sb = [&](int ss) {
#pragma unroll
        for (int u = 0; u < GPMAX; ++u)
            if (u < GP) lds_sb[ss & 1][sb_arr][sb_dst[u]] = (uint16_t)sbr[u];
    };
    // Dequantize word j of this thread's 32 nibbles of tile t (packed stage ->
    // W16 stage t & 1).
    u32x4 wpk;
    uint16_t dq_s, dq_b;
    auto fetch_dq = [&](int t) {
        const int tl = t & 1, ss = t >> 1;
        const int piece = tl * 2 + whalf;
        wpk = lds_wp[(ss & 1) * WP_STAGE + vr * 4 + (piece ^ ((vr >> 2) & 3))];
        const int gl = (tl * 2 + whalf) >> p.gshift;
        dq_s = lds_sb[ss & 1][0][vr * GP + gl];
        dq_b = lds_sb[ss & 1][1][vr * GP + gl];
        if (KTAIL && t * BK + whalf * 32 >= Kl) {
            dq_s = 0;
            dq_b = 0;
        }
    };
    auto store_w = [&](int t, int j) {
        u32x4 o;
        if constexpr (BF16) {
            o = dequant_word_bf16(wpk[j], h2f(dq_s), h2f(dq_b));
        } else {
            const f16 sh = __builtin_bit_cast(f16, dq_s), bh = __builtin_bit_cast(f16, dq_b);
            const f16x2 s2 = {sh, sh}, b2 = {bh, bh};
            o = dequant_word_f16(wpk[j], s2, b2);
        }
        lds_w16[(t & 1) * W16_STAGE + swz(vr, whalf * 4 + j)] = o;
    };

    f32x16 acc[WM][2];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    const int lrow = lane & 31, lk = lane >> 5;
    const int arow0 = wm * (WM * 32) + lrow;
    const int brow0 = wn * 64 + lrow;

    // Prologue: super-stages 0 and 1 (k-tiles 0-3) and the first A tiles in
    // flight; scales/biases of both super-stages to LDS; tile 0 dequantized.
    load_sb(0);
    load_wp(0);
    if (nss > 1) load_wp(1);
#pragma unroll
    for (int t = 0; t < NSA - 1; ++t)
        if (t < nk) load_a(t);
    store_sb(0);   // waits for this thread's scale/bias loads
    if (nss > 1) {
        load_sb(1);
        store_sb(1);
    }
    SLTX_WAIT_VMCNT(0);
    zero_a_tail(0);
    if (NSA > 2 && nk > 1) zero_a_tail(1);
    __syncthreads();
    fetch_dq(0);
#pragma unroll
    for (int j = 0; j < 4; ++j) store_w(0, j);
    __syncthreads();

    // k-tile kt: MFMAs on A stage kt % NSA and W16 stage kt & 1; tile kt+1 is
    // dequantized into the other W16 stage between the k-steps.  Loads issued
    // during kt: A tile kt+NSA-1; for odd kt = 2j+1 also packed W and the
    // scale/bias registers of super-stage j+2 (written to LDS during kt+1).
    // ODD is compile-time (the loop is unrolled by two) so that each step is
    // one branch-free block with a constant wait count.
    auto step = [&](auto odd_c, int kt) {
        constexpr bool ODD = decltype(odd_c)::value;
        const bool a_more = kt + NSA - 1 < nk;
        const bool dq_more = kt + 1 < nk;
        const int ss_ld = (kt + 3) >> 1;
        const bool w_more = ODD && ss_ld < nss;
        if (a_more) load_a(kt + NSA - 1);
        if (w_more) {
            load_wp(ss_ld);
            load_sb(ss_ld);
        }
        if (!ODD && kt >= 2 && (kt >> 1) + 1 < nss) store_sb((kt >> 1) + 1);
        if (dq_more) fetch_dq(kt + 1);
        const u32x4* sa = lds_a + (kt % NSA) * A_STAGE;
        const u32x4* sw = lds_w16 + (kt & 1) * W16_STAGE;
        // Operand fragments are double-buffered: k-step ks+1's LDS reads are
        // issued before k-step ks's MFMAs so their latency overlaps them.
        u32x4 af[2][WM], bf[2][2];
        auto ldfrag = [&](int ks, int b) {
            const int c16 = ks * 2 + lk;
#pragma unroll
            for (int t = 0; t < WM; ++t) af[b][t] = sa[swz(arow0 + t * 32, c16)];
#pragma unroll
            for (int j = 0; j < 2; ++j) bf[b][j] = sw[swz(brow0 + j * 32, c16)];
        };
        ldfrag(0, 0);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int b = ks & 1;
            if (ks + 1 < BK / 16) ldfrag(ks + 1, b ^ 1);
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = mfma32<BF16>(af[b][i], bf[b][j], acc[i][j]);
            if (dq_more) store_w(kt + 1, ks);
        }
        // Before the barrier, A tile kt+1 and the packed W / scales that the
        // next step dequantizes (super-stage (kt+2)/2) must have landed.
        // vmcnt retires in issue order; the count allows exactly the loads
        // that were issued after the last of those:
        //  NSA 2: A tile kt+1 was issued first in this step; after it only
        //         this step's W + scale/bias loads (odd steps).
        //  NSA 3: odd step: A tile kt+1 was issued in the previous (even)
        //         step, which issued nothing else; after it, this step's A and
        //         W + scale/bias loads.  Even step: the previous (odd) step
        //         issued W + scale/bias after its A, and those are needed next
        //         step, so only this step's A loads may remain.
        constexpr int NWSB = 2 + GPMAX;
        if constexpr (NSA == 2) {
            if (ODD && w_more) SLTX_WAIT_VMCNT(NWSB); else SLTX_WAIT_VMCNT(0);
        } else if constexpr (ODD) {
            if (a_more && w_more) SLTX_WAIT_VMCNT(WM + NWSB);
            else if (a_more) SLTX_WAIT_VMCNT(WM);
            else if (w_more) SLTX_WAIT_VMCNT(NWSB);
            else SLTX_WAIT_VMCNT(0);
        } else {
            if (a_more) SLTX_WAIT_VMCNT(WM); else SLTX_WAIT_VMCNT(0);
        }
        if (kt + 1 < nk) zero_a_tail(kt + 1);
        __syncthreads();
    };
    using T_ = std::true_type;
    using F_ = std::false_type;

    int kt = 0;
    for (; kt + 1 < nk; kt += 2) {
        step(F_{}, kt);
        step(T_{}, kt + 1);
    }
    if (kt < nk) step(F_{}, kt);

    // ---- epilogue ----
    // 32x32 accumulator layout: lane l, element v -> row 8*(v/4) + 4*(l/32) + v%4,
    // column l%32.
    const int col_l = lane & 31;
#pragma unroll
    for (int i = 0; i < WM; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int m = m0 + wm * (WM * 32) + i * 32 + 8 * (v >> 2) + 4 * lk + (v & 3);
            if (m >= p.M) continue;
            if constexpr (SPLIT) {
                // raw fp32 partial sums; the reduce kernel applies the epilogue
                const size_t nw = SILU ? 2 * (size_t)p.N : (size_t)p.N;
                float* wsr = p.ws + ((size_t)split * p.M + m) * nw;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int n = SILU ? n0 + wn * 32 + col_l : n0 + wn * 64 + j * 32 + col_l;
                    if (n >= p.N) continue;
                    wsr[SILU ? j * p.N + n : n] = acc[i][j][v];
                }
                continue;
            }
            if (SILU) {
                const int n = n0 + wn * 32 + col_l;
                if (n >= p.N) continue;
                store_out(p, (size_t)m * p.N + n, silu_mul_f32(acc[i][0][v], acc[i][1][v]));
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int n = n0 + wn * 64 + j * 32 + col_l;
                    if (n >= p.N) continue;
                    float out = acc[i][j][v];
                    if (p.bias) out += p.bias[n];
                    if (p.epilogue == kEpiGeluTanh) out = gelu_tanh_f32(out);
                    store_out(p, (size_t)m * p.N + n, out);
                }
            }
        }
    }
}

// Split-K reduction: out[m, n] = epilogue(sum over splits of the partials),
// summed in split order (deterministic).  SILU reduces gate and up
// separately before silu(gate) * up.
template <bool SILU>
__global__ __launch_bounds__(256) void q4_splitk_reduce_kernel(GemmParams p) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)p.M * p.N;
    if (idx >= total) return;
    const size_t m = idx / p.N, n = idx % p.N;
    const size_t nw = SILU ? 2 * (size_t)p.N : (size_t)p.N;
    const size_t stride = (size_t)p.M * nw;
    const float* src = p.ws + m * nw + n;
    float a = 0.0f, u = 0.0f;
    for (int s = 0; s < p.splits; ++s) {
        a += src[s * stride];
        if (SILU) u += src[s * stride + p.N];
    }
    float out;
    if (SILU) {
        out = silu_mul_f32(a, u);
    } else {
        out = a;
        if (p.bias) out += p.bias[n];
        if (p.epilogue == kEpiGeluTanh) out = gelu_tanh_f32(out);
    }
    store_out(p, idx, out);
}

// Launch plan: block-tile height WM (BM = 64*WM) and K splits.  Scores each
// option by useful work over the CU-rounds it occupies (tiles x splits over
// 256 CUs), prefers taller tiles (less dequantisation per MAC) and charges
// each split a little for the partial-sum round trip.  Splits cover an even
// number of k-tiles (the packed-weight stages move two k-tiles at a time).
struct GemmPlan {
    int wm, tiles_m, tiles_n, splits, split_tiles;
    size_t ws_bytes;
};

static GemmPlan plan_gemm(const GemmParams& p, bool allow_split) {
    const bool silu = p.epilogue == kEpiSiluMul;
    const int bn_out = silu ? BN / 2 : BN;
    const int tiles_n = (p.N + bn_out - 1) / bn_out;
    const int nk = (p.K + BK - 1) / BK;
    GemmPlan best = {2, 0, tiles_n, 1, nk, 0};
    double best_score = -1.0;
    for (int wm = 2; wm <= 3; ++wm) {
        const int bm = 64 * wm;
        const long tiles_m = (p.M + bm - 1) / bm;
        const long tiles = tiles_m * tiles_n;
        const int smax = allow_split ? 8 : 1;
        for (int s = 1; s <= smax; ++s) {
            if (s > 1 && nk < 8 * s) break;
            int chunk = (nk + s - 1) / s;
            chunk = s > 1 ? (chunk + 1) / 2 * 2 : chunk;
            const int s_eff = (nk + chunk - 1) / chunk;
            if (s > 1 && s_eff != s) continue;
            const long blocks = tiles * s_eff;
            const long rounds = (blocks + kCUs - 1) / kCUs;
            const double util = ((double)p.M * tiles_n * nk) /
                                ((double)rounds * kCUs * bm * chunk);
            const double score = util * (1.0 + 0.04 * (wm - 2)) * (s > 1 ? 1.0 - 0.02 * s : 1.0);
            if (score > best_score) {
                best_score = score;
                const size_t nw = silu ? 2 * (size_t)p.N : (size_t)p.N;
                best = {wm, (int)tiles_m, tiles_n, s_eff, chunk,
                        s_eff > 1 ? (size_t)s_eff * p.M * nw * sizeof(float) : 0};
            }
        }
    }
    return best;
}

size_t gemm_workspace_bytes(const GemmParams& p) { return plan_gemm(p, true).ws_bytes; }

template <int WM, bool BF16, bool SPLIT>
static void launch_wm(const GemmParams& p, bool silu, long grid, hipStream_t st) {
    // Packed W and scales move in 128-k super-stages: K % 128 != 0 needs the
    // tail handling (clamped sources, zeroed dequant past K).
    const bool ktail = p.K % (2 * BK) != 0;
    if (silu && ktail)
        hipLaunchKernelGGL((q4_gemm_kernel<WM, BF16, true, true, SPLIT>), dim3(grid), dim3(kThreads), 0, st, p);
    else if (silu)
        hipLaunchKernelGGL((q4_gemm_kernel<WM, BF16, true, false, SPLIT>), dim3(grid), dim3(kThreads), 0, st, p);
    else if (ktail)
        hipLaunchKernelGGL((q4_gemm_kernel<WM, BF16, false, true, SPLIT>), dim3(grid), dim3(kThreads), 0, st, p);
    else
        hipLaunchKernelGGL((q4_gemm_kernel<WM, BF16, false, false, SPLIT>), dim3(grid), dim3(kThreads), 0, st, p);
}

template <bool SPLIT>
static void launch_dtype(const GemmParams& p, bool a_bf16, bool silu, long grid, int wm,
                         hipStream_t st) {
    if (a_bf16) {
        if (wm == 2) launch_wm<2, true, SPLIT>(p, silu, grid, st);
        else launch_wm<3, true, SPLIT>(p, silu, grid, st);
    } else {
        if (wm == 2) launch_wm<2, false, SPLIT>(p, silu, grid, st);
        else launch_wm<3, false, SPLIT>(p, silu, grid, st);
    }
}

hipError_t launch_gemm(GemmParams p, bool a_bf16, hipStream_t st) {
    const bool silu = p.epilogue == kEpiSiluMul;
    GemmPlan plan = plan_gemm(p, p.ws != nullptr);
    p.tiles_m = plan.tiles_m;
    p.tiles_n = plan.tiles_n;
    p.splits = plan.splits;
    p.split_tiles = plan.split_tiles;
    const long ntiles = (long)p.tiles_m * p.tiles_n;
    if (ntiles <= 0) return hipSuccess;
    const long blocks = ntiles * p.splits;
    const long grid = (blocks + 7) / 8 * 8;
    if (grid > 0x7fffffffL) return hipErrorInvalidValue;
    if (p.splits > 1) {
        launch_dtype<true>(p, a_bf16, silu, grid, plan.wm, st);
        const size_t total = (size_t)p.M * p.N;
        const long rgrid = (long)((total + 255) / 256);
        if (silu)
            hipLaunchKernelGGL(q4_splitk_reduce_kernel<true>, dim3(rgrid), dim3(256), 0, st, p);
        else
            hipLaunchKernelGGL(q4_splitk_reduce_kernel<false>, dim3(rgrid), dim3(256), 0, st, p);
    } else {
        launch_dtype<false>(p, a_bf16, silu, grid, plan.wm, st);
    }
    return hipGetLastError();
}

}  // namespace sltx
