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
// Block: 512 threads = 8 waves, two per SIMD.  The block tile is BM x 256 x 64
// (BM = 64*WM activation rows, 256 weight rows); wave w owns weight rows
// 32w..32w+31 and all BM activation rows, i.e. BM/32 tiles of
// v_mfma_f32_32x32x16_{f16,bf16} along M.  No weight row is dequantized
// twice, and each dequantized B fragment feeds BM/32 MFMAs.  Two waves per
// SIMD let one wave's dequantization and LDS reads issue while the other's
// MFMAs occupy the matrix core (an MFMA blocks its own wave's issue for about
// half of its 32 cycles).
//  * The B operand never passes through LDS as fp16.  In a 32x32x16 MFMA lane
//    l supplies 8 consecutive k of column l%32.  Inside each 64-wide k-tile, k
//    is permuted so that k-step s of lane half h covers 8-nibble word 4h+s of
//    the row: over a k-tile a lane reads one aligned 16-byte piece of its row,
//    and each k-step's B fragment is exactly one packed word, dequantized in
//    registers just before use (v_perm_b32 byte pairing, mantissa insertion,
//    one v_pk_fma_f16 q*s+b per pair).  The A fragments follow the same
//    permutation by reading 16-byte column 4h+s of the A tile.
//  * Packed W (256 rows x 64 B per pair of k-tiles) and the per-group
//    (scale, bias) pairs are staged through LDS with coalesced loads (four
//    lanes per 64-byte row segment), so no lane gathers 16 bytes per row.
//  * A (BM x 64 fp16/bf16 per k-tile) is copied global -> LDS directly
//    (global_load_lds_dwordx4) into a 4-stage ring, three k-tiles ahead.
//  * LDS rows are 128 bytes with an XOR swizzle of the 16-byte columns (swz):
//    the A fragment reads (16 consecutive rows, one logical column) and the
//    copies are free of bank conflicts.
//  * SILU: a wave's 32 weight rows are the 16 gate and the 16 up rows of the
//    same 16 output columns, so silu(gate) * up is formed in the lane that
//    holds both (register epilogue below).
//  * One barrier per k-tile.  Everything the next k-tile's first k-step needs
//    (its A fragments, its packed words and scale/bias) is already visible
//    before that barrier, so it is read during the last k-step of the current
//    k-tile and the MFMA stream does not drain at k-tile boundaries.
//  * Tile order is XCD-aware: the 8 XCDs receive workgroups round-robin, so
//    consecutive logical tiles (M fastest) are mapped to one XCD and the
//    M-blocks sharing a weight column block share that XCD's L2.
//  * More tiles than CUs (the lm_head and DiT up shapes): one persistent
//    block per CU walks a tile list, the copy ring running on across tiles.
//  * Outputs are stored from registers (SiLU pairs, persistent launches) or
//    staged through LDS into whole row segments (single-round launches of one
//    weight set); see the epilogue.
//  * Shapes with too few output tiles to fill 256 CUs split K; partial sums
//    go to an fp32 workspace and a second kernel adds them in split order.
#include <type_traits>

#include "q4_common.hpp"
#include "q4_dequant.hpp"
#include "q4_epilogue.hpp"
#include "q4_launch.hpp"

namespace sltx {

constexpr int BN = 256, BK = 64;
constexpr int NW = 8;                  // waves per block (two per SIMD)
constexpr int kThreads = 64 * NW;
constexpr int NT = BN / 32 / NW;       // 32-row weight tiles (MFMA N-tiles) per wave
constexpr int NSA = 4;     // A stages in LDS
constexpr int GPMAX = 4;   // scale/bias groups per row per 128 k (group size 32)

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two fp32 values -> packed bf16 pair, round to nearest even (one
// v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// One word -> 8 bf16 values bf16(s*q+b), q*s+b computed with one fp32 FMA.
// nib_mask is 0x0F0F0F0F passed in at run time: with a compile-time mask the
// compiler knows each byte is below 16, narrows `(x >> 8k) & 0xFF` to a 4-bit
// field extract, and needs an extract plus a byte-0 conversion per value; with
// the mask unknown every value is one v_cvt_f32_ubyte{0..3}.  Measured per
// 64-wide k-tile of the bf16 loop: about 160 non-MFMA VALU ops before, 92 after.
__device__ __forceinline__ u32x4 dequant_word_bf16(uint32_t w, uint32_t nib_mask, float s, float b) {
    const uint32_t lo = w & nib_mask;          // bytes q6 q4 q2 q0
    const uint32_t hi = (w >> 4) & nib_mask;   // bytes q7 q5 q3 q1
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

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt bits [3:0] and [15:14], expcnt [6:4] = 7, lgkmcnt [11:8] = 15).
#define SLTX_WAIT_VMCNT(n) \
    __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Workgroup barrier for LDS hand-offs only.  __syncthreads() adds a
// workgroup release fence, which on gfx950 waits for every outstanding
// vector-memory op (vmcnt(0)), including the direct-to-LDS copies issued for
// k-tiles still three steps ahead.  Here each wave waits for its own LDS ops
// (lgkmcnt(0)); the copies a barrier must cover are waited for explicitly
// with SLTX_WAIT_VMCNT before it.  The memory clobber keeps the compiler from
// moving memory accesses across the barrier.
#define SLTX_LDS_BARRIER() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")

// Scale and bias of one (row, group), packed as fp16 bits scale | bias << 16.
struct SB {
    uint32_t v[NT];
};

// GEN = false: K % 128 == 0 and group size 64; every load is a direct-to-LDS
// copy with a fixed count per k-tile and exact wait counts.  GEN = true: any
// supported shape (K % 32 == 0, group 32/64/128): scale/bias staged through
// registers, clamped tails, zero-filled A past K, full waits.
// A32: fp32 activations (the generic path only), each cast to fp16 as
// half(clamp(x, -65504, 65504)) -- cast_f32_to_f16, Kernels.swift:816-822,
// which DiTLinear.applyF32in runs before matmulQ4FastF32
// (DiTModel.swift:104-110) -- while it is staged: a k-tile's A is loaded into
// registers three k-tiles ahead, then cast and written to its LDS stage at
// the end of the k-tile that loaded it.
// PERSIST: the fast path over more output tiles than one round of blocks.
// Each block walks a fixed list of tiles (see the tile selection below);
// the copy ring runs on across tile boundaries -- the last three k-tiles of
// a tile issue the next tile's first A tiles and packed-W / scale-bias
// super-stages -- and the register epilogue of one tile runs while those
// copies are in flight, so neither the next tile's first memory latency nor
// its stores stall the MFMA stream for long.
template <int WM, bool BF16, bool SILU, bool GEN, bool SPLIT, bool A32 = false, bool PERSIST = false>
__global__ __launch_bounds__(kThreads, 1) void q4_gemm_kernel(GemmParams p) {
    static_assert(!A32 || (GEN && !BF16 && !SILU), "fp32 activations: the generic fp16 path");
    static_assert(!PERSIST || (!GEN && !SPLIT && !A32), "persistent tiles: the fast unsplit path");
    constexpr int BM = 64 * WM;
    constexpr int TM = BM / 32;                // MFMA tiles along M per wave
    constexpr int A_STAGE = BM * BK / 8;       // 16-byte slots per A stage
    constexpr int NA = A_STAGE / kThreads;     // A copies per thread per k-tile
    constexpr int WP_STAGE = BN * 4;           // packed W of two k-tiles: 64 B per row
    constexpr int NWP = WP_STAGE / kThreads;   // packed-W copies per thread per super-stage
    constexpr int NPAIR = BN * GPMAX / kThreads;   // GEN: (row, group) pairs per thread per super-stage
    constexpr int NSB = BN * 2 / kThreads;         // fast path: scale/bias copies per thread per super-stage
    // Each stage is its own array: the compiler then knows that reads of one
    // stage do not alias a direct-to-LDS copy in flight into another, and
    // does not wait for that copy (stage indices are compile-time below).
    __shared__ u32x4 lds_a0[A_STAGE], lds_a1[A_STAGE], lds_a2[A_STAGE], lds_a3[A_STAGE];
    __shared__ u32x4 lds_wp0[WP_STAGE], lds_wp1[WP_STAGE];   // [row][piece ^ ((row >> 2) & 3)]
    // Scale/bias.  Fast path (group 64): per super-stage and row one dword of
    // the two groups' scales and one of their biases, [row][scales, biases],
    // copied direct to LDS.  Generic path: [row * GP + group] = scale | bias
    // << 16, staged through registers.
    __shared__ uint32_t lds_sb0[GEN ? BN * GPMAX : BN * 2], lds_sb1[GEN ? BN * GPMAX : BN * 2];
    static_assert(NSA == 4, "stage arrays");
    // A stage of k-tile t is t % 4, packed-W stage of super-stage ss is ss % 2.
    auto a_stage = [&](auto sc) -> u32x4* {
        constexpr int S = decltype(sc)::value & 3;
        if constexpr (S == 0) return lds_a0;
        else if constexpr (S == 1) return lds_a1;
        else if constexpr (S == 2) return lds_a2;
        else return lds_a3;
    };
    auto wp_stage = [&](auto sc) -> u32x4* {
        if constexpr ((decltype(sc)::value & 1) == 0) return lds_wp0;
        else return lds_wp1;
    };
    auto sb_stage = [&](auto sc) -> uint32_t* {
        if constexpr ((decltype(sc)::value & 1) == 0) return lds_sb0;
        else return lds_sb1;
    };

    // ---- tile selection (XCD-aware) ----
    // The 8 XCDs receive workgroups round-robin (block b on XCD b % 8).  One
    // tile per block: consecutive logical tiles (M fastest) go to one XCD.
    // PERSIST (grid a multiple of 8): XCD x owns logical tiles [x T8,
    // min((x + 1) T8, T)), T8 = ceil(T / 8), and its i-th block takes tiles
    // x T8 + i, + G / 8, + 2 G / 8, ... (G = grid): the blocks of one XCD
    // work on neighbouring tiles, which share weight columns, at any time.
    const int ntiles = p.tiles_m * p.tiles_n;
    int logical = blockIdx.x;
    int pstride = 0, pend = 0;
    if constexpr (PERSIST) {
        const int per_x = (ntiles + 7) >> 3;
        logical = (blockIdx.x & 7) * per_x + (blockIdx.x >> 3);
        pend = min(((int)(blockIdx.x & 7) + 1) * per_x, ntiles);
        pstride = gridDim.x >> 3;
        if (logical >= pend) return;
    } else {
        if ((gridDim.x & 7) == 0) {
            const int per_xcd = gridDim.x >> 3;
            logical = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
        }
        if (logical >= ntiles * (SPLIT ? p.splits : 1)) return;
    }
    const int split = SPLIT ? logical / ntiles : 0;
    const int tile = SPLIT ? logical % ntiles : logical;
    // K range of this block: k-tiles [kb, kb + nk); Kl = its extent in k.
    const int nk_all = (p.K + BK - 1) / BK;
    const int kb = SPLIT ? split * p.split_tiles : 0;
    const int nk = SPLIT ? min(p.split_tiles, nk_all - kb) : nk_all;
    const int Kl = min(p.K - kb * BK, nk * BK);
    const int nss = (nk + 1) / 2;   // super-stages (pairs of k-tiles)
    // SILU: a tile covers 128 output columns, as 128 gate rows + 128 up rows.
    // m0 / n0: the tile the copies are reading (PERSIST: the next one from
    // its first prefetch on); em0 / en0: the tile the accumulators hold.
    int m0 = (tile % p.tiles_m) * BM;
    int n0 = (tile / p.tiles_m) * (SILU ? BN / 2 : BN);
    int em0 = m0, en0 = n0;
    bool has_next = PERSIST && logical + pstride < pend;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wn = tid >> 6;
    const int lrow = lane & 31, h = lane >> 5;
    const int GP = 4 >> p.gshift;   // scale/bias groups per 128 k (g = 32, 64, 128)

    // Virtual W row -> matrix row (and which matrix, for SILU).  Wave wn owns
    // virtual rows 32wn..32wn+31 (one 32-row MFMA tile); with SILU its rows
    // 0-15 are the gate rows and 16-31 the up rows of the same 16 output
    // columns, n0 + 16wn .. +15, so that both halves of each output land in
    // one lane (see the epilogue).  Rows past N are clamped to row 0:
    // computed, never stored.
    auto wrow = [&](int v, const uint32_t*& W, const uint16_t*& S, const uint16_t*& B) {
        int n;
        if (SILU) {
            const int tn = (v >> 4) & 1;
            n = n0 + (v >> 5) * 16 + (v & 15);
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
    // Copy i of wave wn fills slots (wn + 4 i) * 64 .. +63, lane l landing in
    // slot +l.  Slot s is physical column s % 8 of row s / 8, i.e. logical
    // column (s % 8) ^ xor(row): the swizzle is applied on the global side.
    // Rows past M are clamped to M-1.
    const uint16_t* A = reinterpret_cast<const uint16_t*>(p.a);
    const uint16_t* a_src[NA];
    int a_col8[NA];
    auto set_a_src = [&]() {
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int slot = (wn + NW * i) * 64 + lane;
            const int row = slot >> 3;
            const int c16 = (slot & 7) ^ (row & 7) ^ ((row >> 3) & 1);
            const int m = m0 + row;
            a_col8[i] = c16 * 8;
            a_src[i] = A + (size_t)(m < p.M ? m : p.M - 1) * p.K + kb * BK + c16 * 8;
        }
    };
    set_a_src();

    // ---- packed W: direct global -> LDS, two k-tiles (64 B per row) ----
    // Four lanes cover a row's 64 bytes, so each wave-wide copy reads 16 rows
    // of 64 contiguous bytes.  Slot s is row s / 4, physical piece s % 4 =
    // logical piece ^ ((row >> 2) & 3) (conflict-free reads below).
    const uint32_t* wp_src[NWP];
    int wp_piece[NWP];
    auto set_wp_src = [&]() {
#pragma unroll
        for (int i = 0; i < NWP; ++i) {
            const int slot = (wn + NW * i) * 64 + lane;
            const int row = slot >> 2;
            const int piece = (slot & 3) ^ ((row >> 2) & 3);
            const uint32_t* W;
            const uint16_t *S, *B;
            const int n = wrow(row, W, S, B);
            wp_piece[i] = piece;
            wp_src[i] = W + (size_t)n * (p.K / 8) + kb * (BK / 8) + piece * 4;
        }
    };
    set_wp_src();

    // ---- scale / bias ----
    const int g_base = (2 * kb) >> p.gshift;
    // Fast path: copy i of wave wn fills dwords (wn + 4 i) * 64 + lane of the
    // stage, i.e. row slot / 2, scales (even slot) or biases (odd slot); the
    // source is the dword holding groups 2 ss and 2 ss + 1 of that row (4-byte
    // aligned: groups and g_base are even when K % 128 == 0 and splits cover
    // whole super-stages).
    const uint32_t* sbd_src[NSB];
    auto set_sbd_src = [&]() {
#pragma unroll
        for (int i = 0; i < NSB; ++i) {
            const int slot = (wn + NW * i) * 64 + lane;
            const uint32_t* W;
            const uint16_t *S, *B;
            const int n = wrow(slot >> 1, W, S, B);
            sbd_src[i] = reinterpret_cast<const uint32_t*>((slot & 1 ? B : S) + (size_t)n * p.groups + g_base);
        }
    };
    set_sbd_src();
    // Generic path: pair v = tid + 256 u is (row v / GP, group v % GP).
    // Consecutive threads read consecutive groups of a row.  Values land in
    // registers and are written to LDS one k-tile later; pairs past the tile
    // (v >= 256 GP) read row 0 and land in unused LDS slots.
    const uint16_t* s_src[NPAIR];
    const uint16_t* b_src[NPAIR];
    int sb_g[NPAIR];
#pragma unroll
    for (int u = 0; u < NPAIR; ++u) {
        const int v = tid + kThreads * u;
        const int row = v / GP, g = v % GP;
        const uint32_t* W;
        const uint16_t *S, *B;
        const int n = wrow(row < BN ? row : 0, W, S, B);
        s_src[u] = S + (size_t)n * p.groups + g_base + g;
        b_src[u] = B + (size_t)n * p.groups + g_base + g;
        sb_g[u] = g;
    }

    // load_a / zero_a_tail / fetch_w take the tile index t with its value mod
    // 4 as a compile-time constant TP; load_wp / store_sb take the super-stage
    // with its parity.
    // A32: this thread's eight fp32 values of each of its NA slots.
    f32x4 a32[A32 ? NA : 1][2];
    const float* const A32src = reinterpret_cast<const float*>(p.a);
    auto load_a = [&](auto tp, int t) {   // NA (A32: 2 NA) vector-memory ops (tiles past the end re-read the last)
        const int k0 = min(t, nk - 1) * BK;
        u32x4* stage = a_stage(tp);
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            int off = k0;
            if (GEN && k0 + a_col8[i] >= Kl) off = Kl - 8 - a_col8[i];
            if constexpr (A32) {
                // the slot's fp16 offset in A is also its fp32 element offset
                const f32x4* src = reinterpret_cast<const f32x4*>(
                    A32src + (a_src[i] - reinterpret_cast<const uint16_t*>(p.a)) + off);
                a32[i][0] = src[0];
                a32[i][1] = src[1];
            } else {
                __builtin_amdgcn_global_load_lds((const void*)(a_src[i] + off),
                                                 (lds_ptr_t)(stage + (wn + NW * i) * 64), 16, 0, 0);
            }
        }
    };
    // A32: tile t's slots from the registers load_a filled, cast with the
    // clamp, into stage tp (zeros past K).
    auto store_a32 = [&](auto tp, int t) {
        if constexpr (A32) {
            const int k0 = t * BK;
            u32x4* stage = a_stage(tp);
#pragma unroll
            for (int i = 0; i < NA; ++i) {
                u32x4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float lo = a32[i][e >> 1][2 * (e & 1)], hi = a32[i][e >> 1][2 * (e & 1) + 1];
                    o[e] = (uint32_t)f2h(fminf(fmaxf(lo, -65504.0f), 65504.0f)) |
                           ((uint32_t)f2h(fminf(fmaxf(hi, -65504.0f), 65504.0f)) << 16);
                }
                if (k0 + a_col8[i] >= Kl) o = u32x4{0u, 0u, 0u, 0u};
                stage[(wn + NW * i) * 64 + lane] = o;
            }
        }
    };
    auto zero_a_tail = [&](auto tp, int t) {   // GEN: after the copy of tile t landed
        const int k0 = t * BK;
        if (t >= nk || k0 + BK <= Kl) return;
        u32x4* stage = a_stage(tp);
        const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < NA; ++i)
            if (k0 + a_col8[i] >= Kl) stage[(wn + NW * i) * 64 + lane] = z;
    };
    auto load_wp = [&](auto sp, int ss) {   // NWP vector-memory ops
        const int sc = min(ss, nss - 1);
        u32x4* stage = wp_stage(sp);
#pragma unroll
        for (int i = 0; i < NWP; ++i) {
            int off = sc * 16;   // u32 words: 64 bytes per super-stage
            if (GEN && sc * 128 + wp_piece[i] * 32 >= Kl) off = (Kl / 8) - 4 - wp_piece[i] * 4;
            __builtin_amdgcn_global_load_lds((const void*)(wp_src[i] + off),
                                             (lds_ptr_t)(stage + (wn + NW * i) * 64), 16, 0, 0);
        }
    };
    auto load_sb_dma = [&](auto sp, int ss) {   // fast path: NSB vector-memory ops
        const int sc = min(ss, nss - 1);
        uint32_t* stage = sb_stage(sp);
#pragma unroll
        for (int i = 0; i < NSB; ++i)
            __builtin_amdgcn_global_load_lds((const void*)(sbd_src[i] + sc),
                                             (lds_ptr_t)(stage + (wn + NW * i) * 64), 4, 0, 0);
    };
    uint32_t s_reg[NPAIR], b_reg[NPAIR];
    auto load_sb = [&](int ss) {   // generic path: 2 NPAIR vector-memory ops
        const int sc = min(ss, nss - 1);
        const int groups_l = p.groups - g_base;
#pragma unroll
        for (int u = 0; u < NPAIR; ++u) {
            int g = sc * GP;
            if (GEN && g + sb_g[u] >= groups_l) g = groups_l - 1 - sb_g[u];
            s_reg[u] = s_src[u][g];
            b_reg[u] = b_src[u][g];
        }
    };
    auto store_sb = [&](auto sp) {
        uint32_t* stage = sb_stage(sp);
#pragma unroll
        for (int u = 0; u < NPAIR; ++u)
            stage[tid + kThreads * u] = (s_reg[u] & 0xFFFFu) | (b_reg[u] << 16);
    };

    // Packed words (16 bytes: this lane's four k-steps) and scale|bias of
    // tile t for both of the wave's 32-row MFMA tiles.
    auto fetch_w = [&](auto tp, int t, u32x4 (&wk)[NT], SB& sb) {
        constexpr int TP = decltype(tp)::value & 3;
        constexpr int TL = TP & 1, SP = (TP >> 1) & 1;   // tile within / parity of super-stage
        const u32x4* ws = wp_stage(std::integral_constant<int, SP>{});
        const int piece = TL * 2 + h;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int vr = wn * 32 * NT + j * 32 + lrow;
            wk[j] = ws[vr * 4 + (piece ^ ((vr >> 2) & 3))];
            uint32_t v;
            if constexpr (GEN) {
                v = sb_stage(std::integral_constant<int, SP>{})[vr * GP + (piece >> p.gshift)];
            } else {
                // group TL of the super-stage: half TL of the scale and bias dwords
                const uint2 d = reinterpret_cast<const uint2*>(sb_stage(std::integral_constant<int, SP>{}))[vr];
                v = __builtin_amdgcn_perm(d.y, d.x, TL ? 0x07060302u : 0x05040100u);
            }
            if (GEN && t * BK + h * 32 >= Kl) v = 0;   // k past K: w = 0
            sb.v[j] = v;
        }
    };
    // B fragment of k-step ks for MFMA tile j.
    auto dequant = [&](const u32x4 (&wk)[NT], const SB& sb, int ks, u32x4 (&dst)[NT]) {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const uint32_t v = sb.v[j];
            if constexpr (BF16) {
                dst[j] = dequant_word_bf16(wk[j][ks], p.nib_mask, h2f((uint16_t)(v & 0xFFFFu)),
                                           h2f((uint16_t)(v >> 16)));
            } else {
                const f16x2 s2 = as_f16x2(__builtin_amdgcn_perm(v, v, 0x01000100u));
                const f16x2 b2 = as_f16x2(__builtin_amdgcn_perm(v, v, 0x03020302u));
                dst[j] = dequant_word_f16(wk[j][ks], s2, b2);
            }
        }
    };
    auto read_a = [&](const u32x4* sa, int ks, u32x4 (&dst)[TM]) {
        const int c16 = 4 * h + ks;
#pragma unroll
        for (int i = 0; i < TM; ++i) dst[i] = sa[swz(i * 32 + lrow, c16)];
    };

    // TRANS: the packed-weight fragment is the MFMA's A operand, so the
    // accumulators hold D^T (weight rows along the lane's 16 values) -- the
    // layout the register epilogue stores from.  Otherwise (the LDS-staged
    // epilogue) the activation fragment is A, as measured 1.3% faster on the
    // bf16 DiT down loop (the dequantized fragment is then read as the B
    // operand).
    constexpr bool TRANS = PERSIST || SILU;
    f32x16 acc[TM][NT];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;

    // Prologue: A tiles 0..2 and packed W / scale-bias of super-stages 0 and
    // 1 in flight.  k-tile 0 needs A tiles 0 and 1 and super-stage 0 before
    // it starts; A tile 2 and super-stage 1 (issued last) may still land
    // during it (the wait at the end of k-tile 0 covers them).  Generic path:
    // scale/bias of super-stage 0 to LDS, super-stage 1's stay in registers
    // and are written at the end of k-tile 0.
    if constexpr (A32) {
        // one tile of A registers: tiles 0, 1, 2 one after another
        load_wp(I0{}, 0);
        load_wp(I1{}, 1);
        load_sb(0);
        load_a(I0{}, 0);
        SLTX_WAIT_VMCNT(0);
        store_sb(I0{});
        store_a32(I0{}, 0);
        load_sb(1);
        load_a(I1{}, 1);
        SLTX_WAIT_VMCNT(0);
        store_a32(I1{}, 1);
        load_a(I2{}, 2);
        SLTX_WAIT_VMCNT(0);
        store_a32(I2{}, 2);
    } else if constexpr (GEN) {
        load_a(I0{}, 0);
        load_a(I1{}, 1);
        load_a(I2{}, 2);
        load_wp(I0{}, 0);
        load_wp(I1{}, 1);
        load_sb(0);
        SLTX_WAIT_VMCNT(0);
        store_sb(I0{});
        load_sb(1);
        SLTX_WAIT_VMCNT(0);
        zero_a_tail(I0{}, 0);
        zero_a_tail(I1{}, 1);
        zero_a_tail(I2{}, 2);
    } else {
        load_a(I0{}, 0);
        load_a(I1{}, 1);
        load_wp(I0{}, 0);
        load_sb_dma(I0{}, 0);
        load_a(I2{}, 2);
        load_wp(I1{}, 1);
        load_sb_dma(I1{}, 1);
        SLTX_WAIT_VMCNT(NA + NWP + NSB);
    }
    SLTX_LDS_BARRIER();

    u32x4 wk_c[NT], wk_n[NT];
    SB sb_c, sb_n;
    u32x4 af[2][TM], bq[2][NT];
    fetch_w(I0{}, 0, wk_c, sb_c);
    read_a(a_stage(I0{}), 0, af[0]);
    dequant(wk_c, sb_c, 0, bq[0]);

    // k-tile kt (TP = kt % 4, compile-time): MFMAs on A stage TP with B
    // dequantized from tile kt's packed words.  Issued during kt: A tile kt+3;
    // for odd kt = 2j+1 the packed W and scale/bias registers of super-stage
    // j+2 (the latter written to LDS at the end of k-tile kt+1).  The operands
    // of tile kt+1's first k-step are formed during the last k-step.  Each
    // tile is one branch-free block with a constant wait count.
    auto step = [&](auto tp, int kt) {
        constexpr int TP = decltype(tp)::value;
        constexpr bool ODD = TP & 1;
        using N1 = std::integral_constant<int, (TP + 1) & 3>;
        using N3 = std::integral_constant<int, (TP + 3) & 3>;
        int ta = kt + NSA - 1, tw = (kt + 3) >> 1;   // A tile and super-stage to copy
        if constexpr (PERSIST) {
            if (has_next) {
                // from k-tile nk - 3 on, the copies read the next tile
                if (kt == nk - (NSA - 1)) {
                    const int nt = logical + pstride;
                    m0 = (nt % p.tiles_m) * BM;
                    n0 = (nt / p.tiles_m) * (SILU ? BN / 2 : BN);
                    set_a_src();
                    set_wp_src();
                    set_sbd_src();
                }
                if (ta >= nk) ta -= nk;
                if (tw >= nss) tw -= nss;
            }
        }
        load_a(N3{}, ta);
        if constexpr (ODD) {
            // super-stage (kt+3)/2: parity ((TP+3) >> 1) & 1
            load_wp(std::integral_constant<int, ((TP + 3) >> 1) & 1>{}, tw);
            if constexpr (GEN) load_sb(tw);
            else load_sb_dma(std::integral_constant<int, ((TP + 3) >> 1) & 1>{}, tw);
        }
        const u32x4* sa = a_stage(tp);
        const u32x4* sa_n = a_stage(N1{});
        __builtin_amdgcn_sched_barrier(0);
        // Each k-step: this step's MFMAs (operands read / dequantized during
        // the previous step) with the next step's A fragment reads and B
        // dequantization interleaved.  The first MFMA goes before any new LDS
        // read: the compiler's wait for its operands then covers only reads
        // issued a full k-step earlier (it cannot count LDS reads separately
        // while direct-to-LDS copies are in flight, so every LDS wait it
        // emits waits for all of them).  The scheduling-group barriers fix
        // that order: 1 MFMA, half the step's reads, 1 MFMA, the other half,
        // then MFMAs with up to six VALU ops each, so the dequantization
        // finishes early in the step (measured 1-3% faster than one read per
        // MFMA with three VALU ops, and than all reads after the first MFMA;
        // the bf16 shapes and split down gain most).  Step 0
        // also reads tile kt+1's packed words and scale/bias (used from step 3
        // on).
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int b = ks & 1;
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < NT; ++j)
                    acc[i][j] = TRANS ? mfma32<BF16>(bq[b][j], af[b][i], acc[i][j])
                                      : mfma32<BF16>(af[b][i], bq[b][j], acc[i][j]);
            if (ks + 1 < BK / 16) {
                read_a(sa, ks + 1, af[b ^ 1]);
                dequant(wk_c, sb_c, ks + 1, bq[b ^ 1]);
            } else {
                read_a(sa_n, 0, af[b ^ 1]);
                dequant(wk_n, sb_n, 0, bq[b ^ 1]);
            }
            if (ks == 0) fetch_w(N1{}, kt + 1, wk_n, sb_n);
            constexpr int NR0 = TM + 2 * NT;   // LDS reads in step 0
            static_assert(NT * TM >= 2, "two MFMAs per step to spread the reads over");
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // MFMA
            if (ks == 0) __builtin_amdgcn_sched_group_barrier(0x100, (NR0 + 1) / 2, 0);   // DS reads
            else __builtin_amdgcn_sched_group_barrier(0x100, (TM + 1) / 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);       // VALU
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // MFMA
            if (ks == 0) __builtin_amdgcn_sched_group_barrier(0x100, NR0 / 2, 0);   // DS reads
            else __builtin_amdgcn_sched_group_barrier(0x100, TM / 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);       // VALU
#pragma unroll
            for (int q = 2; q < NT * TM; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);   // VALU
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // even kt: scale/bias of super-stage (kt+2)/2 (parity ((TP+2) >> 1) & 1)
        if constexpr (GEN && !ODD) store_sb(std::integral_constant<int, ((TP + 2) >> 1) & 1>{});
        // Before the barrier, A tile kt+2 and the packed W / scale-bias of
        // tile kt+2 must have landed (they are read during k-tile kt+1).
        // vmcnt retires in issue order.  Even kt issued only A tile kt+3;
        // odd kt issued A tile kt+3 and super-stage (kt+3)/2 after A tile
        // kt+2 (issued at kt-1, which issued nothing else).
        if constexpr (A32) {
            // tile kt+3 (loaded at the start of this k-tile) into its stage,
            // which k-tile kt-1 read before the last barrier
            SLTX_WAIT_VMCNT(0);
            store_a32(N3{}, kt + NSA - 1);
        } else if constexpr (GEN) {
            SLTX_WAIT_VMCNT(0);
            zero_a_tail(std::integral_constant<int, (TP + 2) & 3>{}, kt + 2);
        } else if constexpr (ODD) {
            SLTX_WAIT_VMCNT(NA + NWP + NSB);
        } else {
            SLTX_WAIT_VMCNT(NA);
        }
        SLTX_LDS_BARRIER();
#pragma unroll
        for (int j = 0; j < NT; ++j) wk_c[j] = wk_n[j];
        sb_c = sb_n;
    };

    // ---- epilogue, from registers (TRANS) ----
    // The MFMAs compute D^T = W_tile . A_tile^T, so lane l holds, for activation row em0 + 32 i + l % 32,
    // the wave's weight rows 8 g + 4 h + r (r = 0..3, h = l / 32) in
    // acc[i][0][4 g + r]: four consecutive output columns per g.  One
    // v_permlane32_swap per value gives each lane eight consecutive columns
    // (groups g and g + 1 of lanes l and l + 32): lane l < 32 columns 0-7 of
    // the pair, lane l + 32 columns 8-15, stored as one 16-byte vector.  With
    // SILU, g = 0, 1 are gate rows and g + 2 the up rows of the same columns,
    // so silu(gate) * up is formed before the swap.  No LDS and no barrier:
    // a persistent block goes on to the next tile's k-tiles (copied during
    // the last three of this one) while the stores drain.
    static_assert(NT == 1, "one 32-row MFMA tile of W rows per wave");
    auto swap8 = [&](const float (&lo)[4], const float (&hi)[4], float (&o)[8]) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, lo[r]),
                                                             __builtin_bit_cast(uint32_t, hi[r]),
                                                             false, false);
            o[r] = __builtin_bit_cast(float, (uint32_t)sw[0]);
            o[4 + r] = __builtin_bit_cast(float, (uint32_t)sw[1]);
        }
    };
    auto group = [&](const f32x16& t, int g, float (&o)[4]) {
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = t[4 * g + r];
    };
    auto epilogue = [&]() {
        const bool vec = out_vec_ok(p);
        const int cw = en0 + (SILU ? 16 : 32) * wn + 8 * h;   // this lane's first column
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int m = em0 + i * 32 + lrow;   // lanes l and l + 32 share a row
            float x[8];
            if constexpr (SPLIT) {
                // raw fp32 partial sums; the reduce kernel applies the epilogue
                const size_t nw = SILU ? 2 * (size_t)p.N : (size_t)p.N;
                float* wsr = p.ws + ((size_t)split * p.M + (m < p.M ? m : 0)) * nw;
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    float lo[4], hi[4];
                    group(acc[i][0], 2 * q, lo);
                    group(acc[i][0], 2 * q + 1, hi);
                    swap8(lo, hi, x);
                    // SILU: q = 1 is up, whose partials follow gate's
                    if (m < p.M) store_f32x8(SILU && q ? wsr + p.N : wsr, cw + (SILU ? 0 : 16 * q), p.N, x);
                }
            } else if constexpr (SILU) {
                const bool gelu = p.epilogue == kEpiGeluMul;
                float lo[4], hi[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    lo[r] = glu_f32(gelu, acc[i][0][r], acc[i][0][8 + r]);
                    hi[r] = glu_f32(gelu, acc[i][0][4 + r], acc[i][0][12 + r]);
                }
                swap8(lo, hi, x);
                if (m < p.M) store_out8(p, (size_t)m * p.N, cw, x, vec);
            } else {
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    float lo[4], hi[4];
                    group(acc[i][0], 2 * q, lo);
                    group(acc[i][0], 2 * q + 1, hi);
                    swap8(lo, hi, x);
                    if (m < p.M) epi_store8(p, (size_t)m * p.N, cw + 16 * q, x, vec);
                }
            }
        }
    };

    // One launch of a single round, one weight set (no SiLU pair): each
    // 32-row accumulator tile (D, activation rows along the lane's 16 values,
    // row 8 (v / 4) + 4 h + v % 4, column l % 32) is staged through LDS (the
    // A stages, idle once the last copy into them has landed) as two fp32
    // [32][128] buffers, output columns 0-127 and 128-255, so that all 512
    // threads store whole 256-byte row segments: 16-byte pieces at 8 (t % 16)
    // of row t / 16.  Measured against the register epilogue at DiT down
    // (M = 6144, 25 MB of output at once): 2 us faster; the register stores
    // put 32 rows in each store instruction.
    auto staged_epilogue = [&]() {
        static_assert(32 * 128 * 4 <= A_STAGE * 16, "a 32 x 128 fp32 tile fits one A stage");
        SLTX_WAIT_VMCNT(0);
        SLTX_LDS_BARRIER();
        float* const eb0 = reinterpret_cast<float*>(lds_a0);
        float* const eb1 = reinterpret_cast<float*>(lds_a1);
        float* const wdst = (wn >> 2) ? eb1 : eb0;
        const int wcol = (wn & 3) * 32 + lrow;
        const int er = tid >> 4, ec = (tid & 15) * 8;
        const bool vec = out_vec_ok(p);
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int v = 0; v < 16; ++v) wdst[(8 * (v >> 2) + 4 * h + (v & 3)) * 128 + wcol] = acc[i][0][v];
            SLTX_LDS_BARRIER();
            const int m = em0 + i * 32 + er;
            if (m < p.M) {
                float x0[8], x1[8];
                const f32x4* r0 = reinterpret_cast<const f32x4*>(eb0 + er * 128 + ec);
                const f32x4* r1 = reinterpret_cast<const f32x4*>(eb1 + er * 128 + ec);
                const f32x4 a0 = r0[0], a1 = r0[1], b0 = r1[0], b1 = r1[1];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x0[e] = a0[e];
                    x0[4 + e] = a1[e];
                    x1[e] = b0[e];
                    x1[4 + e] = b1[e];
                }
                if constexpr (SPLIT) {
                    // raw fp32 partial sums; the reduce kernel applies the epilogue
                    float* wsr = p.ws + ((size_t)split * p.M + m) * (size_t)p.N;
                    store_f32x8(wsr, en0 + ec, p.N, x0);
                    store_f32x8(wsr, en0 + 128 + ec, p.N, x1);
                } else {
                    epi_store8(p, (size_t)m * p.N, en0 + ec, x0, vec);
                    epi_store8(p, (size_t)m * p.N, en0 + 128 + ec, x1, vec);
                }
            }
            SLTX_LDS_BARRIER();
        }
    };

    for (;;) {
        int kt = 0;
        for (; kt + 3 < nk; kt += 4) {
            step(I0{}, kt);
            step(I1{}, kt + 1);
            step(I2{}, kt + 2);
            step(I3{}, kt + 3);
        }
        if constexpr (!PERSIST) {   // PERSIST: nk % 4 == 0
            if (kt < nk) step(I0{}, kt);
            if (kt + 1 < nk) step(I1{}, kt + 1);
            if (kt + 2 < nk) step(I2{}, kt + 2);
        }
        if constexpr (PERSIST || SILU) {
            // the block's last copies (clamped re-reads of the last k-tile)
            // land before it ends and its LDS is released; the stores need
            // no wait
            if (!has_next) SLTX_WAIT_VMCNT(0);
            epilogue();
        } else {
            static_assert(!TRANS, "the staged epilogue reads D, not D^T");
            staged_epilogue();
        }
        if (!has_next) break;
        // the next tile: its copies are in flight, its first k-step's operands
        // were formed during the last k-step
        logical += pstride;
        em0 = m0;
        en0 = n0;
        has_next = logical + pstride < pend;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][0][v] = 0.0f;
    }
}


// Split-K reduction: out[m, n] = epilogue(sum over splits of the partials),
// summed in split order (deterministic).  SILU reduces gate and up
// separately before silu(gate) * up.  S > 0 is the split count, known at
// compile time: every split's loads are issued before the first add, so the
// pass pays one memory latency instead of one per split (the adds keep the
// split order, so the sums are the same bit for bit).  S == 0: any count.
template <bool SILU, int S>
__global__ __launch_bounds__(256) void q4_splitk_reduce_kernel(GemmParams p) {
    // each thread: 8 consecutive outputs of one row
    const int nb8 = (p.N + 7) / 8;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)p.M * nb8) return;
    const size_t m = idx / nb8;
    const int n0 = (int)(idx % nb8) * 8;
    const size_t nw = SILU ? 2 * (size_t)p.N : (size_t)p.N;
    const size_t stride = (size_t)p.M * nw;
    const float* src = p.ws + m * nw;
    const bool vin = (p.N & 7) == 0;   // 16-byte aligned workspace rows and no tail
    float a[8], u[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = u[e] = 0.0f;
    if constexpr (S > 0) {
        f32x4 q[S][2], r[SILU ? S : 1][2];
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const f32x4* g = reinterpret_cast<const f32x4*>(src + s * stride + n0);
            q[s][0] = g[0];
            q[s][1] = g[1];
            if (SILU) {
                const f32x4* h = reinterpret_cast<const f32x4*>(src + s * stride + p.N + n0);
                r[s][0] = h[0];
                r[s][1] = h[1];
            }
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                a[e] += q[s][0][e];
                a[4 + e] += q[s][1][e];
                if (SILU) {
                    u[e] += r[s][0][e];
                    u[4 + e] += r[s][1][e];
                }
            }
        }
    } else {
    for (int s = 0; s < p.splits; ++s, src += stride) {
        if (vin) {
            const f32x4* q = reinterpret_cast<const f32x4*>(src + n0);
            const f32x4 q0 = q[0], q1 = q[1];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                a[e] += q0[e];
                a[4 + e] += q1[e];
            }
            if (SILU) {
                const f32x4* r = reinterpret_cast<const f32x4*>(src + p.N + n0);
                const f32x4 r0 = r[0], r1 = r[1];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    u[e] += r0[e];
                    u[4 + e] += r1[e];
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if (n0 + e < p.N) {
                    a[e] += src[n0 + e];
                    if (SILU) u[e] += src[p.N + n0 + e];
                }
            }
        }
    }
    }
    const bool vec = out_vec_ok(p);
    if (SILU) {
        const bool gelu = p.epilogue == kEpiGeluMul;
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = glu_f32(gelu, a[e], u[e]);
        store_out8(p, m * p.N, n0, a, vec);
    } else {
        epi_store8(p, m * p.N, n0, a, vec);
    }
}

// Split-K reduction fused with the residual add and the RMSNorm of each
// output row (one block of 256 threads per row, N % 8 == 0):
//   o = half(sum over splits, in split order)        the projection (linear)
//   t = float(residual) + float(o);  r = half(t)     elemAdd / residualRmsNorm
//   rms = rsqrt(mean(q^2) + eps), q = t (sum_rounded == 0, residualRmsNorm,
//         Kernels.swift:238-290) or q = float(r) (sum_rounded == 1: elemAdd then
//         rmsNorm of the stored fp16 stream, Kernels.swift:40-86, 121-128)
//   out = half(float(r) * rms * w)
// The partial sums follow q4_splitk_reduce_kernel and the row sum of squares
// follows rms_norm_vec_kernel (thread t: pieces t, t + 256, ... of 8 values;
// wave trees, then the four waves in order), so the results equal the unfused
// GEMM + reduce + norm sequence bit for bit.  S > 0 is the split count,
// known at compile time: a piece's loads of every split are issued before its
// first add (same order of adds).
template <int VPT, int S>
__global__ __launch_bounds__(256) void q4_splitk_residual_rms_norm_kernel(
    GemmParams p, const float* w, float eps, uint16_t* res_out, uint16_t* out, int sum_rounded) {
    __shared__ float red[4];
    const int nv = p.N / 8;
    const size_t m = blockIdx.x;
    const size_t stride = (size_t)p.M * p.N;
    const f16x8* R = reinterpret_cast<const f16x8*>(p.residual + m * p.N);
    f16x8 r[VPT];
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
        const int v = threadIdx.x + 256 * u;
        if (v >= nv) continue;
        float a[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = 0.0f;
        const float* q = p.ws + m * p.N + (size_t)v * 8;
        if constexpr (S > 0) {
            f32x4 qs[S][2];
#pragma unroll
            for (int s = 0; s < S; ++s) {
                qs[s][0] = reinterpret_cast<const f32x4*>(q + s * stride)[0];
                qs[s][1] = reinterpret_cast<const f32x4*>(q + s * stride)[1];
            }
#pragma unroll
            for (int s = 0; s < S; ++s) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    a[e] += qs[s][0][e];
                    a[4 + e] += qs[s][1][e];
                }
            }
        } else {
            for (int s = 0; s < p.splits; ++s, q += stride) {
                const f32x4 q0 = reinterpret_cast<const f32x4*>(q)[0];
                const f32x4 q1 = reinterpret_cast<const f32x4*>(q)[1];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    a[e] += q0[e];
                    a[4 + e] += q1[e];
                }
            }
        }
        const f16x8 h = R[v];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float t = (float)h[e] + h2f(f2h(a[e]));
            r[u][e] = (f16)t;
            const float sq = sum_rounded ? (float)r[u][e] : t;
            ss += sq * sq;
        }
        reinterpret_cast<f16x8*>(res_out + m * p.N)[v] = r[u];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float rms = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)p.N + eps);
    const f32x4* W = reinterpret_cast<const f32x4*>(w);
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
        const int v = threadIdx.x + 256 * u;
        if (v >= nv) continue;
        const f32x4 w0 = W[2 * v], w1 = W[2 * v + 1];
        f16x8 o8;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            o8[e] = (f16)((float)r[u][e] * rms * w0[e]);
            o8[4 + e] = (f16)((float)r[u][4 + e] * rms * w1[e]);
        }
        reinterpret_cast<f16x8*>(out + m * p.N)[v] = o8;
    }
}

// Launch plan: block-tile height WM (BM = 64*WM) and K splits, chosen by
// estimated time on 256 CUs: rounds of blocks x (k-tiles per block x the
// measured time of one k-tile -- 1.37 us at BM = 192, 0.95 us at BM = 128,
// a 256-row W tile -- plus ~8 us of prologue and epilogue, which every round
// repeats) + ~2 us per launch, plus, when split, writing the fp32 partials
// (~6 TB/s) and the reduce pass reading them back (~4 TB/s, its own launch).
// Measured at M = 750 (lm_head, N = 128256): 664 us at BM = 192 vs 730 us at
// BM = 128; DiT up (M = 6144, bf16): 318 vs 356 us.  Splits cover an even
// number of k-tiles (packed weights move two k-tiles at a time).
struct GemmPlan {
    int wm, tiles_m, tiles_n, splits, split_tiles;
    size_t ws_bytes;
};

// partials: the output goes through the fp32 workspace at every split count
// (including one), because a row-wise pass follows (the fused residual +
// RMSNorm), so the unsplit plan pays the partial traffic too.
static GemmPlan plan_gemm(const GemmParams& p, bool allow_split, bool partials = false) {
    const bool silu = p.epilogue == kEpiSiluMul || p.epilogue == kEpiGeluMul;
    const int bn_out = silu ? BN / 2 : BN;
    const int tiles_n = (p.N + bn_out - 1) / bn_out;
    const int nk = (p.K + BK - 1) / BK;
    const size_t nw = silu ? 2 * (size_t)p.N : (size_t)p.N;
    GemmPlan best = {2, 0, tiles_n, 1, nk, 0};
    double best_us = 1e30;
    // fp32 activations hold a k-tile of A in registers: the 192-row tile
    // would spill, so they take the 128-row tile only
    for (int wm = 2; wm <= (p.a_f32 ? 2 : 3); ++wm) {
        const int bm = 64 * wm;
        const long tiles_m = (p.M + bm - 1) / bm;
        const long tiles = tiles_m * tiles_n;
        const double kt_us = wm == 3 ? 1.37 : 0.95;
        const int smax = allow_split ? 8 : 1;
        for (int s = 1; s <= smax; ++s) {
            if (s > 1 && nk < 8 * s) break;
            int chunk = (nk + s - 1) / s;
            chunk = s > 1 ? (chunk + 1) / 2 * 2 : chunk;
            const int s_eff = (nk + chunk - 1) / chunk;
            if (s > 1 && s_eff != s) continue;
            const long blocks = tiles * s_eff;
            const long rounds = (blocks + kCUs - 1) / kCUs;
            double us = (double)rounds * (chunk * kt_us + 8.0) + 2.0;
            const bool ws = s_eff > 1 || partials;
            if (ws) {
                const double part = (double)s_eff * p.M * nw * 4.0;
                us += part / 6.0e6 + 3.0 + (part + (double)p.M * p.N * 2.0) / 4.0e6;
            }
            if (us < best_us) {
                best_us = us;
                best = {wm, (int)tiles_m, tiles_n, s_eff, chunk,
                        ws ? (size_t)s_eff * p.M * nw * sizeof(float) : 0};
            }
        }
    }
    return best;
}

size_t gemm_workspace_bytes(const GemmParams& p) { return plan_gemm(p, true).ws_bytes; }
size_t gemm_partials_workspace_bytes(const GemmParams& p) { return plan_gemm(p, true, true).ws_bytes; }

template <int WM, bool BF16, bool SPLIT>
static void launch_wm(const GemmParams& p, bool silu, long grid, hipStream_t st) {
    if constexpr (WM == 2) {
        if (p.a_f32) {
            hipLaunchKernelGGL((q4_gemm_kernel<2, false, false, true, SPLIT, true>), dim3(grid),
                               dim3(kThreads), 0, st, p);
            return;
        }
    }
    // The fixed-count kernel needs whole 128-k super-stages and group size 64
    // (scales and biases move as dword pairs of groups, so their arrays must
    // also be 4-byte aligned; 2-byte aligned ones take the generic kernel,
    // which reads them as 16-bit values).
    const uintptr_t sb_addr = reinterpret_cast<uintptr_t>(p.s0) | reinterpret_cast<uintptr_t>(p.b0) |
                              reinterpret_cast<uintptr_t>(p.s1) | reinterpret_cast<uintptr_t>(p.b1);
    const bool gen = p.K % (2 * BK) != 0 || p.gshift != 1 || (sb_addr & 3) != 0;
    // More tiles than one block per CU: one persistent block per CU walks
    // them (the ring's stage parity restarts with each tile: K % 256 == 0).
    if constexpr (!SPLIT) {
        if (!gen && p.K % (4 * BK) == 0 && (long)p.tiles_m * p.tiles_n > kCUs) {
            const dim3 pg(kCUs);
            if (silu)
                hipLaunchKernelGGL((q4_gemm_kernel<WM, BF16, true, false, false, false, true>), pg,
                                   dim3(kThreads), 0, st, p);
            else
                hipLaunchKernelGGL((q4_gemm_kernel<WM, BF16, false, false, false, false, true>), pg,
                                   dim3(kThreads), 0, st, p);
            return;
        }
    }
    if (silu && gen)
        hipLaunchKernelGGL((q4_gemm_kernel<WM, BF16, true, true, SPLIT>), dim3(grid), dim3(kThreads), 0, st, p);
    else if (silu)
        hipLaunchKernelGGL((q4_gemm_kernel<WM, BF16, true, false, SPLIT>), dim3(grid), dim3(kThreads), 0, st, p);
    else if (gen)
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

template <bool SILU>
void launch_reduce_s(const GemmParams& p, dim3 g, hipStream_t st) {
    // the loads-first form needs whole 16-byte rows (N % 8 == 0)
    const int s = (p.N & 7) == 0 ? p.splits : 0;
    switch (s) {
    case 2: hipLaunchKernelGGL((q4_splitk_reduce_kernel<SILU, 2>), g, dim3(256), 0, st, p); break;
    case 3: hipLaunchKernelGGL((q4_splitk_reduce_kernel<SILU, 3>), g, dim3(256), 0, st, p); break;
    case 4: hipLaunchKernelGGL((q4_splitk_reduce_kernel<SILU, 4>), g, dim3(256), 0, st, p); break;
    case 5: hipLaunchKernelGGL((q4_splitk_reduce_kernel<SILU, 5>), g, dim3(256), 0, st, p); break;
    case 6: hipLaunchKernelGGL((q4_splitk_reduce_kernel<SILU, 6>), g, dim3(256), 0, st, p); break;
    case 7: hipLaunchKernelGGL((q4_splitk_reduce_kernel<SILU, 7>), g, dim3(256), 0, st, p); break;
    case 8: hipLaunchKernelGGL((q4_splitk_reduce_kernel<SILU, 8>), g, dim3(256), 0, st, p); break;
    default: hipLaunchKernelGGL((q4_splitk_reduce_kernel<SILU, 0>), g, dim3(256), 0, st, p); break;
    }
}

hipError_t launch_splitk_reduce(const GemmParams& p, hipStream_t st) {
    const bool silu = p.epilogue == kEpiSiluMul || p.epilogue == kEpiGeluMul;
    const size_t total = (size_t)p.M * ((p.N + 7) / 8);
    const dim3 rgrid((unsigned)((total + 255) / 256));
    if (silu)
        launch_reduce_s<true>(p, rgrid, st);
    else
        launch_reduce_s<false>(p, rgrid, st);
    return hipGetLastError();
}

hipError_t launch_gemm(GemmParams p, bool a_bf16, hipStream_t st) {
    const bool silu = p.epilogue == kEpiSiluMul || p.epilogue == kEpiGeluMul;
    GemmPlan plan = plan_gemm(p, p.ws != nullptr);
    p.nib_mask = 0x0F0F0F0Fu;
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
        (void)launch_splitk_reduce(p, st);
    } else {
        launch_dtype<false>(p, a_bf16, silu, grid, plan.wm, st);
    }
    return hipGetLastError();
}

template <int VPT>
void launch_rrn_s(const GemmParams& p, const float* norm_w, float eps, uint16_t* res_out,
                  uint16_t* norm_out, int sr, hipStream_t st) {
    const dim3 g(p.M), t(256);
    switch (p.splits) {
    case 1: hipLaunchKernelGGL((q4_splitk_residual_rms_norm_kernel<VPT, 1>), g, t, 0, st, p, norm_w, eps, res_out, norm_out, sr); break;
    case 2: hipLaunchKernelGGL((q4_splitk_residual_rms_norm_kernel<VPT, 2>), g, t, 0, st, p, norm_w, eps, res_out, norm_out, sr); break;
    case 3: hipLaunchKernelGGL((q4_splitk_residual_rms_norm_kernel<VPT, 3>), g, t, 0, st, p, norm_w, eps, res_out, norm_out, sr); break;
    case 4: hipLaunchKernelGGL((q4_splitk_residual_rms_norm_kernel<VPT, 4>), g, t, 0, st, p, norm_w, eps, res_out, norm_out, sr); break;
    default: hipLaunchKernelGGL((q4_splitk_residual_rms_norm_kernel<VPT, 0>), g, t, 0, st, p, norm_w, eps, res_out, norm_out, sr); break;
    }
}

// GEMM into fp32 partials (one or more K splits; p.ws holds
// gemm_partials_workspace_bytes(p)), then the fused reduce + residual +
// RMSNorm pass.  Requires N % 8 == 0, N <= 16384 and 16-byte aligned rows.
hipError_t launch_gemm_residual_rms_norm(GemmParams p, bool a_bf16, const float* norm_w, float eps,
                                         uint16_t* res_out, uint16_t* norm_out, bool sum_rounded,
                                         hipStream_t st) {
    if (p.M <= 0 || p.N <= 0) return hipSuccess;
    if (p.N % 8 != 0 || p.N / 8 > 8 * 256 || !p.ws || !p.residual) return hipErrorInvalidValue;
    if ((long)p.M * 256 > 0xffffffffL) return hipErrorInvalidValue;   // one 256-thread block per row
    const GemmPlan plan = plan_gemm(p, true, true);
    p.nib_mask = 0x0F0F0F0Fu;
    p.tiles_m = plan.tiles_m;
    p.tiles_n = plan.tiles_n;
    p.splits = plan.splits;
    p.split_tiles = plan.split_tiles;
    const long blocks = (long)p.tiles_m * p.tiles_n * p.splits;
    const long grid = (blocks + 7) / 8 * 8;
    if (grid > 0x7fffffffL) return hipErrorInvalidValue;
    launch_dtype<true>(p, a_bf16, false, grid, plan.wm, st);
    const int vpt = (p.N / 8 + 255) / 256;
    const int sr = sum_rounded ? 1 : 0;
    if (vpt == 1)
        launch_rrn_s<1>(p, norm_w, eps, res_out, norm_out, sr, st);
    else if (vpt == 2)
        launch_rrn_s<2>(p, norm_w, eps, res_out, norm_out, sr, st);
    else if (vpt <= 4)
        launch_rrn_s<4>(p, norm_w, eps, res_out, norm_out, sr, st);
    else
        launch_rrn_s<8>(p, norm_w, eps, res_out, norm_out, sr, st);
    return hipGetLastError();
}

}  // namespace sltx
