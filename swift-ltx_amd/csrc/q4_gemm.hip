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

template <int WM, bool BF16, bool SILU, bool KTAIL>
__global__ __launch_bounds__(kThreads, 1) void q4_gemm_kernel(GemmParams p) {
    constexpr int BM = 64 * WM;
    constexpr int A_STAGE = BM * BK / 8;    // 16-byte slots per A stage
    constexpr int W_STAGE = BN * BK / 8;
    __shared__ u32x4 lds_a[3 * A_STAGE];    // 3 stages, swizzled [row][col16]
    __shared__ u32x4 lds_w[2 * W_STAGE];    // 2 stages

    // ---- tile selection (XCD-aware) ----
    const int ntiles = p.tiles_m * p.tiles_n;
    int logical = blockIdx.x;
    if ((gridDim.x & 7) == 0) {
        const int per_xcd = gridDim.x >> 3;
        logical = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    }
    if (logical >= ntiles) return;
    const int tile_m = logical % p.tiles_m;
    const int tile_n = logical / p.tiles_m;
    const int m0 = tile_m * BM;
    // SILU: a tile covers 128 output columns, as 128 gate rows + 128 up rows.
    const int n0 = tile_n * (SILU ? BN / 2 : BN);

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;

    // ---- A: direct global -> LDS (global_load_lds_dwordx4) ----
    // Each wave fills WM 1-KB pieces of a stage: piece i covers slots
    // (wave + 8 i) * 64 .. +63, lane l landing in slot +l (the hardware puts
    // lane l's 16 bytes at the wave's base + 16 l).  Slot s is physical
    // column s % 8 of row s / 8, i.e. logical column (s % 8) ^ xor(row), so
    // the swizzle is applied on the global side.  Rows past M are clamped to
    // M-1 (computed, never stored).
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
        a_src[i] = A + (size_t)(m < p.M ? m : p.M - 1) * p.K + c16 * 8;
    }

    // ---- W: global -> registers -> dequantize -> LDS ----
    // Virtual row vr = tid % 256, half = tid / 256 (32 nibbles; the half is
    // wave-uniform).  Rows past N are clamped to row 0 (never stored).
    const int vr = tid & 255, whalf = tid >> 8;
    int wn_row;
    const uint32_t* Wsel;
    const uint16_t *Ssel, *Bsel;
    if (SILU) {
        const int wv = vr >> 6, tn = (vr >> 5) & 1;
        wn_row = n0 + wv * 32 + (vr & 31);
        Wsel = tn ? p.w1 : p.w0;
        Ssel = tn ? p.s1 : p.s0;
        Bsel = tn ? p.b1 : p.b0;
    } else {
        wn_row = n0 + vr;
        Wsel = p.w0;
        Ssel = p.s0;
        Bsel = p.b0;
    }
    const int wr = wn_row < p.N ? wn_row : 0;
    const uint32_t* w_ptr = Wsel + (size_t)wr * (p.K / 8) + whalf * 4;
    const uint16_t* s_ptr = Ssel + (size_t)wr * p.groups;
    const uint16_t* b_ptr = Bsel + (size_t)wr * p.groups;

    const int nk = (p.K + BK - 1) / BK;

    // Tile kt+2's loads are issued while tile kt is multiplied: A straight
    // into LDS stage (kt+2) % 3, W into one of two register sets.  A K tail
    // (K % 64 == 32: the last tile's upper 32 columns) clamps the A source in
    // bounds and zeroes those LDS slots once the copy has landed, and gives
    // the upper W half scale = bias = 0 (s*q + b = 0 whatever the codes).
    struct WRegs {
        u32x4 w;
        uint32_t s, b;
        bool zero;
    };

    auto load_a = [&](int kt) {   // WM vector-memory ops
        const int k0 = kt * BK;
        u32x4* stage = lds_a + (kt % 3) * A_STAGE;
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            int off = k0;
            if (KTAIL && k0 + a_col8[i] >= p.K) off = p.K - 8 - a_col8[i];
            __builtin_amdgcn_global_load_lds(
                (const void*)(a_src[i] + off),
                (lds_ptr_t)(stage + (wave + 8 * i) * 64), 16, 0, 0);
        }
    };
    auto zero_a_tail = [&](int kt) {   // after the copy for tile kt landed
        const int k0 = kt * BK;
        if (!KTAIL || k0 + BK <= p.K) return;
        u32x4* stage = lds_a + (kt % 3) * A_STAGE;
        const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < WM; ++i)
            if (k0 + a_col8[i] >= p.K) stage[(wave + 8 * i) * 64 + lane] = z;
    };
    auto load_w = [&](WRegs& r, int kt) {   // 3 vector-memory ops
        const int k0 = kt * BK;
        r.zero = KTAIL && k0 + whalf * 32 >= p.K;
        const int wz = r.zero ? 1 : 0;
        r.w = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(w_ptr + (k0 >> 3) - 4 * wz));
        const int gi = (2 * kt + whalf - wz) >> p.gshift;
        r.s = s_ptr[gi];
        r.b = b_ptr[gi];
    };
    // Dequantize word j of this thread's W chunk into W stage `stage`.
    auto store_w = [&](const WRegs& r, int stage, int j) {
        const uint16_t sb = (KTAIL && r.zero) ? (uint16_t)0 : (uint16_t)r.s;
        const uint16_t bb = (KTAIL && r.zero) ? (uint16_t)0 : (uint16_t)r.b;
        u32x4 o;
        if constexpr (BF16) {
            o = dequant_word_bf16(r.w[j], h2f(sb), h2f(bb));
        } else {
            const f16 sh = __builtin_bit_cast(f16, sb), bh = __builtin_bit_cast(f16, bb);
            const f16x2 s2 = {sh, sh}, b2 = {bh, bh};
            o = dequant_word_f16(r.w[j], s2, b2);
        }
        lds_w[stage * W_STAGE + swz(vr, whalf * 4 + j)] = o;
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

    // One k-tile: MFMAs on A stage kt % 3 and W stage kt % 2.  With LOAD, tile
    // kt+2 is loaded (A into LDS, W into `fre`); with STORE, tile kt+1's W
    // (in `nxt`) is dequantized into the other W stage between the k-steps.
    // LOAD and STORE are compile-time so each step is one branch-free block.
    auto step = [&](auto load_c, auto store_c, int kt, const WRegs& nxt, WRegs& fre) {
        constexpr bool LOAD = decltype(load_c)::value;
        constexpr bool STORE = decltype(store_c)::value;
        if constexpr (LOAD) {
            load_w(fre, kt + 2);
            load_a(kt + 2);
        }
        const u32x4* sa = lds_a + (kt % 3) * A_STAGE;
        const u32x4* sw = lds_w + (kt & 1) * W_STAGE;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int c16 = ks * 2 + lk;
            u32x4 af[WM], bf[2];
#pragma unroll
            for (int t = 0; t < WM; ++t) af[t] = sa[swz(arow0 + t * 32, c16)];
#pragma unroll
            for (int j = 0; j < 2; ++j) bf[j] = sw[swz(brow0 + j * 32, c16)];
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma32<BF16>(af[i], bf[j], acc[i][j]);
            if constexpr (STORE) store_w(nxt, (kt + 1) & 1, ks);
        }
        // Tile kt+1's A copy (issued one step earlier) must have landed before
        // the barrier; only this step's own loads may still be in flight.
        if constexpr (LOAD)
            SLTX_WAIT_VMCNT(WM + 3);
        else
            SLTX_WAIT_VMCNT(0);
        if constexpr (STORE) zero_a_tail(kt + 1);
        __syncthreads();
    };
    using T_ = std::true_type;
    using F_ = std::false_type;

    // Prologue: tiles 0 and 1 in flight, tile 0 made ready.
    WRegs ra, rb;
    load_w(ra, 0);
    load_a(0);
    if (nk > 1) {
        load_w(rb, 1);
        load_a(1);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) store_w(ra, 0, j);
    if (nk > 1)
        SLTX_WAIT_VMCNT(WM + 3);
    else
        SLTX_WAIT_VMCNT(0);
    zero_a_tail(0);
    __syncthreads();
    // Invariant at the top of each pass: tile kt is ready in LDS, rb holds
    // tile kt+1's W and its A copy is in flight.
    int kt = 0;
    for (; kt + 3 < nk; kt += 2) {
        step(T_{}, T_{}, kt, rb, ra);
        step(T_{}, T_{}, kt + 1, ra, rb);
    }
    const int rem = nk - kt;   // 1, 2 or 3 tiles left
    if (rem == 3) {
        step(T_{}, T_{}, kt, rb, ra);
        step(F_{}, T_{}, kt + 1, ra, rb);
        step(F_{}, F_{}, kt + 2, rb, ra);
    } else if (rem == 2) {
        step(F_{}, T_{}, kt, rb, ra);
        step(F_{}, F_{}, kt + 1, ra, rb);
    } else {
        step(F_{}, F_{}, kt, rb, ra);
    }

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

// Block-tile height: the WM (BM = 64*WM) whose tile count fills the CUs in
// the fewest rounds with the least padding, preferring taller tiles (less
// dequantisation per MAC) when close.
static int pick_wm(int M, int n_tiles) {
    int best = 2;
    double best_score = -1.0;
    for (int wm = 2; wm <= 3; ++wm) {
        const int bm = 64 * wm;
        const long tiles = (long)((M + bm - 1) / bm) * n_tiles;
        const long rounds = (tiles + kCUs - 1) / kCUs;
        const double util = (double)M * n_tiles / ((double)rounds * kCUs * bm);
        const double score = util * (1.0 + 0.04 * (wm - 2));
        if (score > best_score) {
            best_score = score;
            best = wm;
        }
    }
    return best;
}

template <int WM, bool BF16>
static void launch_wm(const GemmParams& p, bool silu, long grid, hipStream_t st) {
    const bool ktail = p.K % BK != 0;
    if (silu && ktail)
        hipLaunchKernelGGL((q4_gemm_kernel<WM, BF16, true, true>), dim3(grid), dim3(kThreads), 0, st, p);
    else if (silu)
        hipLaunchKernelGGL((q4_gemm_kernel<WM, BF16, true, false>), dim3(grid), dim3(kThreads), 0, st, p);
    else if (ktail)
        hipLaunchKernelGGL((q4_gemm_kernel<WM, BF16, false, true>), dim3(grid), dim3(kThreads), 0, st, p);
    else
        hipLaunchKernelGGL((q4_gemm_kernel<WM, BF16, false, false>), dim3(grid), dim3(kThreads), 0, st, p);
}

hipError_t launch_gemm(GemmParams p, bool a_bf16, hipStream_t st) {
    const bool silu = p.epilogue == kEpiSiluMul;
    const int bn_out = silu ? BN / 2 : BN;
    p.tiles_n = (p.N + bn_out - 1) / bn_out;
    const int wm = pick_wm(p.M, p.tiles_n);
    p.tiles_m = (p.M + 64 * wm - 1) / (64 * wm);
    const long ntiles = (long)p.tiles_m * p.tiles_n;
    if (ntiles <= 0) return hipSuccess;
    const long grid = (ntiles + 7) / 8 * 8;
    if (grid > 0x7fffffffL) return hipErrorInvalidValue;
    if (a_bf16) {
        if (wm == 2) launch_wm<2, true>(p, silu, grid, st);
        else launch_wm<3, true>(p, silu, grid, st);
    } else {
        if (wm == 2) launch_wm<2, false>(p, silu, grid, st);
        else launch_wm<3, false>(p, silu, grid, st);
    }
    return hipGetLastError();
}

}  // namespace sltx
