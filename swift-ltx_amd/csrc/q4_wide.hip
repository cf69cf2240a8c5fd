// q4_wide.hip -- 4-bit dequant matmul for 32 < M <= 256 activation rows
// (T5 encoder layers at S <= 256, T5Encoder.swift:72-78 and :140-205; short
// prompts) on CDNA4 MFMA.
//
// Same product as q4_gemm.hip, Y[M,N] = X[M,K] . dequant(W)[N,K]^T with fp32
// accumulation (matmulQ4Fast, Ops.swift:312-381).  Between the mid-M weight
// stream (M <= 32) and the large-M GEMM (128- or 192-row tiles of 256 weight
// rows), the GEMM's tiles are too few to fill 256 CUs and its split-K fp32
// partials cost more HBM traffic than the weights (M = 128, gate/up: 33 MB of
// partials against 28 MB of weights).  Here a block owns few weight rows and
// all of its K range instead:
//  * Block: 64 weight rows -- two 32-row MFMA N-tiles of one set, or the
//    gate and up tiles of 32 output columns for the gated epilogues -- by
//    BM = 32 TM activation rows (TM = 2..4; more rows take more blocks along
//    M).  The 8 waves split K: in each round of 128 k, wave g takes the
//    16-k MFMA step g, so every wave holds all TM x 2 accumulator tiles of the
//    block (v_mfma_f32_32x32x16_f16), each packed word is dequantized once
//    per block and feeds TM MFMAs, and each A fragment feeds two.
//  * A round's X (BM rows x 256 bytes) and packed W (64 rows x 64 bytes) are
//    copied global -> LDS directly (global_load_lds, 16-byte pieces; W by the
//    first four waves, one piece per lane) into a ring of 3 (TM = 4) or 4
//    stages, issued a ring's depth ahead.  Each wave issues the same number
//    of copies every round (rounds past the last re-read it), so one exact
//    s_waitcnt vmcnt and one LDS-only barrier per round hand a stage over.  Each stage is its own array, and the loop is
//    unrolled by the ring depth so that stage indices are compile-time: the
//    compiler then knows that reads of one stage do not alias copies in
//    flight into another.
//  * The block's scales and biases (64 rows x its K range's groups, at most
//    64 groups) are read once into an LDS slab as scale | bias << 16 words.
//  * After the last round the 8 waves' tiles are summed in LDS in a fixed
//    order (one 32-row tile at a time) and the epilogue (gated SiLU /
//    GELU-tanh, bias, GELU-tanh, residual add) runs on the fp32 sums.  With a
//    K split across blocks each block stores its sums to the fp32 workspace
//    and counts its arrival on its output tile's counter; the last block to
//    arrive adds the splits in split order and runs the epilogue (no reduce
//    pass).
#include <type_traits>
#include <utility>

#include "q4_common.hpp"
#include "q4_dequant.hpp"
#include "q4_epilogue.hpp"
#include "q4_launch.hpp"
#include "q4_split.hpp"

namespace sltx {

namespace {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int NWV = 8;              // waves, one K-group each
constexpr int WT = 64 * NWV;        // threads per block
constexpr int WBN = 64;             // weight rows per block (two MFMA N-tiles)
constexpr int RK = NWV * 16;        // k per round: one 16-k MFMA step per wave
constexpr int XCH = RK * 2 / 16;    // 16-byte pieces of an X row per round (16)
constexpr int WRD = RK / 8;         // packed words of a weight row per round (16)
constexpr int WDW = WBN * WRD;      // dwords of a W stage (1024)
constexpr int WPC = WDW / 4;        // 16-byte W pieces per round (256)
constexpr int WCW = WPC / 64;       // waves that copy them, one piece per lane (4)
constexpr int SLAB_G = 64;          // scale / bias groups a block holds
// Ring stages by tile height (a stage is BM x 256 bytes of X + 4 KB of W).
// Measured over the Llama and T5 shapes at M = 33..256: at TM = 4 three
// stages run 0.1-0.5 us faster than four; at TM = 2 six or seven stages
// (which the LDS would hold) run 0.5-1.7 us slower than four, three about
// even.  The loop is not waiting on copy latency (every extra stage only
// lengthens the prologue, which waits for the slab loads issued behind the
// first rounds' copies).
template <int TM>
constexpr int wide_nsx() { return TM == 4 ? 3 : 4; }

#define WIDE_LDS_BARRIER() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")

// f(integral_constant<int, i>) for i = 0 .. N - 1, unrolled
template <typename F, int... I>
__device__ __forceinline__ void static_for_seq(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_seq(f, std::make_integer_sequence<int, N>{});
}

struct WideArgs {
    int mrows;    // activation rows of this launch's M-blocks (the last may hold fewer)
    int kblk;     // k per split
};

// LDS reads the compiler does not see as memory operations.  Its wait-count
// pass cannot tell reads of one ring stage from copies in flight into
// another once the loop's back-edge merges its state, and would drain every
// copy in flight (vmcnt(0)) before the first read of each unrolled
// iteration; the stage a round reads has been waited for by that round's
// own vmcnt and barrier.  The results must pass through lds_wait() before
// use.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(lds_ptr_t)(p);
}
__device__ __forceinline__ u32x4 ds_read16(uint32_t a) {
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(a) : "memory");
    return v;
}
__device__ __forceinline__ uint32_t ds_read4(uint32_t a) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(a) : "memory");
    return v;
}

__device__ __forceinline__ f32x16 mfma32_f16(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// X piece (row, c) of a stage sits at row * XCH + (c ^ (row & 15)): the 16
// rows a quarter-wave reads at one logical piece hit 16 distinct pieces.
__device__ __forceinline__ int xpos(int row, int c) { return row * XCH + (c ^ (row & 15)); }
// W word (row, w) of a stage: the row's four 16-byte pieces, piece p at
// position p ^ ((row >> 2) & 3).  The 32 rows a half-wave reads at one
// logical word meet at most two to a bank.  (Copied as single words, which
// allow a conflict-free layout, the copies took 16 instead of 4 wave-wide
// copy instructions per round, and the route up to 0.7 us more per launch.)
__device__ __forceinline__ int wpos(int row, int w) {
    return row * WRD + ((((w >> 2) ^ (row >> 2)) & 3) << 2) + (w & 3);
}
// Slab entry (group gi, row) at gi * 64 + (row ^ (gi & 63)): conflict-free
// both for the fill (consecutive groups of a row) and for the reads (the
// rows of one group).
__device__ __forceinline__ int spos(int gi, int row) { return gi * WBN + (row ^ (gi & 63)); }

// The last block of an output tile: the S splits' partial sums of the rows
// and columns this thread summed (32 i + ml, n .. n + NV - 1) -- its own
// split's from registers (own0 / own1), the others' loaded, every load
// issued before the first add -- added in split order from zero as the
// split-K reduce pass adds them, then the epilogue.
template <int S, int TM, bool PAIR, int NV>
__device__ __forceinline__ void wide_fixup(const GemmParams& p, int m0, int mrows, int ml, int n,
                                           int split, const float (&own0)[TM][NV],
                                           const float (&own1)[TM][NV]) {
    const size_t nw = PAIR ? 2 * (size_t)p.N : (size_t)p.N;
    const __amdgpu_buffer_rsrc_t rs = ws_rsrc(p.ws);
    // slot o holds split o + (o >= split)
    float g[TM][S - 1][NV], u[PAIR ? TM : 1][PAIR ? S - 1 : 1][NV];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int m = min(m0 + 32 * i + ml, p.M - 1);
#pragma unroll
        for (int o = 0; o < S - 1; ++o) {
            const int j = o + (o >= split ? 1 : 0);
            const size_t r = ((size_t)j * p.M + m) * nw;
            load_f32v_sc1<NV>(rs, r, n, p.N, g[i][o]);
            if constexpr (PAIR) load_f32v_sc1<NV>(rs, r + p.N, n, p.N, u[i][o]);
        }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int brow = 32 * i + ml;
        const int m = m0 + brow;
        if (brow >= mrows || m >= p.M) continue;
        float a[NV], b[NV];
#pragma unroll
        for (int e = 0; e < NV; ++e) a[e] = b[e] = 0.0f;
#pragma unroll
        for (int j = 0; j < S; ++j)
#pragma unroll
            for (int e = 0; e < NV; ++e) {
                const int lo = j > 0 ? j - 1 : 0, hi = j < S - 1 ? j : S - 2;
                a[e] += j == split ? own0[i][e] : (j < split ? g[i][hi][e] : g[i][lo][e]);
                if constexpr (PAIR)
                    b[e] += j == split ? own1[i][e] : (j < split ? u[i][hi][e] : u[i][lo][e]);
            }
        if constexpr (PAIR) {
            const bool gelu = p.epilogue == kEpiGeluMul;
#pragma unroll
            for (int e = 0; e < NV; ++e) a[e] = glu_f32(gelu, a[e], b[e]);
            store_outv<NV>(p, (size_t)m * p.N, n, a);
        } else {
            epi_storev<NV>(p, (size_t)m * p.N, n, a);
        }
    }
}

template <int TM, bool PAIR, bool SPLIT>
__global__ __launch_bounds__(WT, 1) void q4_wide_kernel(GemmParams p, WideArgs wa) {
    constexpr int BM = 32 * TM;
    constexpr int XS = BM * XCH;        // 16-byte pieces of an X stage
    constexpr int NXC = XS / WT;        // X copies per thread per round
    static_assert(NXC * WT == XS && WCW * 64 == WPC && WCW <= NWV, "whole copies");
    // vector-memory ops per thread per round: NXC, plus one W piece in the
    // first WCW waves
    constexpr int CPR_W = NXC + 1, CPR_X = NXC;
    constexpr int NSX = wide_nsx<TM>(); // ring stages
    static_assert(NSX == 3 || NSX == 4, "ring depth");
    static_assert(XS * 16 >= 2 * 8 * 1024, "two waves' 32-row tiles fit one X stage");
    // One array per stage (stage indices are compile-time, so the compiler
    // sees that reads of one stage do not alias copies into another).  The
    // fourth X array exists at NSX = 3 too: the K-groups' sums are staged in
    // all four.
    __shared__ u32x4 xs0[XS], xs1[XS], xs2[XS], xs3[XS];
    __shared__ uint32_t ws0[WDW], ws1[WDW], ws2[WDW], ws3[NSX > 3 ? WDW : 1];
    __shared__ uint32_t slab[SLAB_G * WBN];
    auto xstage = [&](auto sc) -> u32x4* {
        constexpr int S = decltype(sc)::value % NSX;
        if constexpr (S == 0) return xs0;
        else if constexpr (S == 1) return xs1;
        else if constexpr (S == 2) return xs2;
        else return xs3;
    };
    auto wstage = [&](auto sc) -> uint32_t* {
        constexpr int S = decltype(sc)::value % NSX;
        if constexpr (S == 0) return ws0;
        else if constexpr (S == 1) return ws1;
        else if constexpr (S == 2) return ws2;
        else return ws3;
    };

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = blockIdx.x * (PAIR ? 32 : WBN);
    const int m0 = blockIdx.y * wa.mrows;
    const int split = SPLIT ? (int)blockIdx.z : 0;
    const int kb = split * wa.kblk;
    const int nr = wa.kblk / RK;        // rounds
    const int K = p.K;

    // Weight row of block row `row` (0..63): the matrix and its row index;
    // rows past N read row 0 (computed, never stored).
    auto wrow = [&](int row, const uint32_t*& W, const uint16_t*& S, const uint16_t*& B) {
        int n;
        if (PAIR) {
            const bool up = row >= 32;
            n = n0 + (row & 31);
            W = up ? p.w1 : p.w0;
            S = up ? p.s1 : p.s0;
            B = up ? p.b1 : p.b0;
        } else {
            n = n0 + row;
            W = p.w0;
            S = p.s0;
            B = p.b0;
        }
        return n < p.N ? n : 0;
    };

    // ---- copy sources ----
    // X copy i of thread t fills piece s = t + WT i of the stage: row s / XCH,
    // physical piece s % XCH = logical piece ^ (row & 15); rows past M read
    // row M - 1 (computed, never stored).
    const uint16_t* A = reinterpret_cast<const uint16_t*>(p.a);
    const uint16_t* x_src[NXC];
#pragma unroll
    for (int i = 0; i < NXC; ++i) {
        const int s = tid + WT * i;
        const int row = s / XCH;
        const int c = (s % XCH) ^ (row & 15);
        const int m = min(m0 + row, p.M - 1);
        x_src[i] = A + (size_t)m * K + kb + c * 8;
    }
    // W: thread t < WPC fills piece t of the stage: row t / 4, physical piece
    // t % 4 = logical piece ^ ((row >> 2) & 3).
    const bool w_copier = wave < WCW;
    const uint32_t* w_src;
    {
        const int t = w_copier ? tid : 0;
        const int row = t >> 2;
        const int lp = (t & 3) ^ ((row >> 2) & 3);
        const uint32_t* W;
        const uint16_t *S, *B;
        const int n = wrow(row, W, S, B);
        w_src = W + (size_t)n * (K / 8) + kb / 8 + lp * 4;
    }
    // Round q (clamped to the last round: copies past the end re-read it into
    // a stage no later round reads).
    auto issue = [&](auto sc, int q) {   // CPR_W or CPR_X vector-memory ops
        const int qc = min(q, nr - 1);
        u32x4* xd = xstage(sc);
        uint32_t* wd = wstage(sc);
#pragma unroll
        for (int i = 0; i < NXC; ++i)
            __builtin_amdgcn_global_load_lds((const void*)(x_src[i] + (size_t)qc * RK),
                                             (lds_ptr_t)(xd + (tid & ~63) + WT * i), 16, 0, 0);
        if (w_copier)
            __builtin_amdgcn_global_load_lds((const void*)(w_src + (size_t)qc * WRD),
                                             (lds_ptr_t)(wd + 4 * (tid & ~63)), 16, 0, 0);
    };

    // rounds 0 .. NSX - 2 into their stages
    static_for<NSX - 1>([&](auto sc) { issue(sc, decltype(sc)::value); });

    // ---- scale / bias slab: the block's rows over its K range ----
    // Every load is issued before the first is used (one memory latency for
    // the whole slab, behind the ring's first copies).
    const int glog2 = 5 + p.gshift;
    const int gbase = kb >> glog2;
    const int ng = wa.kblk >> glog2;    // groups of this block (<= SLAB_G)
    constexpr int NSE = (WBN * SLAB_G + WT - 1) / WT;   // slab entries per thread (at most)
    uint32_t sv[NSE], bv[NSE];
#pragma unroll
    for (int u = 0; u < NSE; ++u) {
        const int e = tid + WT * u;
        const int row = e / ng, gi = e % ng;
        const uint32_t* W;
        const uint16_t *S, *B;
        const int n = wrow(e < WBN * ng ? row : 0, W, S, B);
        const size_t o = (size_t)n * p.groups + gbase + (e < WBN * ng ? gi : 0);
        sv[u] = S[o];
        bv[u] = B[o];
    }
#pragma unroll
    for (int u = 0; u < NSE; ++u) {
        const int e = tid + WT * u;
        if (e < WBN * ng) slab[spos(e % ng, e / ng)] = sv[u] | (bv[u] << 16);
    }

    const int r = lane & 31, h = lane >> 5;
    const int c = 2 * wave + h;         // this lane's X piece and W word in a round
    f32x16 acc[TM][2];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    // Round q's operands from stage q % NSX: reads() issues the LDS reads (A
    // fragments, packed words, scale|bias words), settle() waits for them
    // (one lgkmcnt(0) that every value passes through) and dequantizes the B
    // fragments.
    u32x4 a[TM], b[2];       // operands of the round whose MFMAs run next
    u32x4 an[TM];            // raw operands of the round after it
    uint32_t wn[2], sn[2];
    auto reads = [&](auto sc, int q) {
        const uint32_t xb = lds_addr(xstage(sc)), wb = lds_addr(wstage(sc)), sb = lds_addr(slab);
#pragma unroll
        for (int i = 0; i < TM; ++i) an[i] = ds_read16(xb + 16 * xpos(32 * i + r, c));
        const int gi = ((TM >= 3 ? min(q, nr - 1) : q) * RK + 16 * wave + 8 * h) >> glog2;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int row = 32 * j + r;
            wn[j] = ds_read4(wb + 4 * wpos(row, c));
            sn[j] = ds_read4(sb + 4 * spos(gi, row));
        }
    };
    auto settle = [&]() {
        if constexpr (TM == 2)
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(an[0]), "+v"(an[1]), "+v"(wn[0]), "+v"(wn[1]),
                         "+v"(sn[0]), "+v"(sn[1]));
        else if constexpr (TM == 3)
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(an[0]), "+v"(an[1]), "+v"(an[2]), "+v"(wn[0]),
                         "+v"(wn[1]), "+v"(sn[0]), "+v"(sn[1]));
        else
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(an[0]), "+v"(an[1]), "+v"(an[2]), "+v"(an[3]),
                         "+v"(wn[0]), "+v"(wn[1]), "+v"(sn[0]), "+v"(sn[1]));
#pragma unroll
        for (int i = 0; i < TM; ++i) a[i] = an[i];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const f16x2 s2 = as_f16x2(__builtin_amdgcn_perm(sn[j], sn[j], 0x01000100u));
            const f16x2 b2 = as_f16x2(__builtin_amdgcn_perm(sn[j], sn[j], 0x03020302u));
            b[j] = dequant_word_f16(wn[j], s2, b2);
        }
        // At TM >= 3 this use keeps the dequantization ahead of the next
        // round's barrier; the compiler otherwise sinks it past the barrier
        // and the copies, in front of the next round's first MFMA.
        if constexpr (TM >= 3) asm volatile("" ::"v"(b[0]), "v"(b[1]));
    };
    // Every wave's copies of the next round to read have landed: this
    // thread's were issued before NSX - 2 later rounds' (which may still be
    // in flight), then the barrier.  (A separate W ring eight rounds deep,
    // its first eight rounds issued with the prologue, measured 0.3-1 us
    // slower on every shape: the prologue then waits for all of them.)
    auto ready = [&]() {
        if (w_copier)
            __builtin_amdgcn_s_waitcnt(vmcnt_only((NSX - 2) * CPR_W));
        else
            __builtin_amdgcn_s_waitcnt(vmcnt_only((NSX - 2) * CPR_X));
        WIDE_LDS_BARRIER();
    };
    // Round q (operands in a, b): round q + 1's stage is waited for, the
    // stage round q read is refilled with round q + NSX, round q + 1's LDS
    // reads are issued, then round q's MFMAs run while they return, and
    // round q + 1's B fragments are dequantized behind the MFMAs.  In the
    // unrolled body at TM >= 3 (`always`) even a last round does all of
    // this: its copies re-read the last round, its reads fetch a stage no
    // round uses (scale groups clamped to the block's), and the round has no
    // branch, so the dequantization is scheduled between the MFMAs.  With
    // the use in settle() this measured 0.5-0.8 us faster per launch at
    // M = 128 on every wide shape, and 0.1 us slower at TM = 2.
    auto round = [&](auto sc, int q, auto always) {
        constexpr int S = decltype(sc)::value % NSX;
        const bool more = (TM >= 3 && decltype(always)::value) || q + 1 < nr;
        if (more) {
            ready();
            issue(std::integral_constant<int, S>{}, q + NSX);
            reads(std::integral_constant<int, (S + 1) % NSX>{}, q + 1);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = mfma32_f16(a[i], b[j], acc[i][j]);
        if (more) settle();
    };

    ready();
    reads(std::integral_constant<int, 0>{}, 0);
    settle();
    issue(std::integral_constant<int, NSX - 1>{}, NSX - 1);
    int q = 0;
    for (; q + NSX - 1 < nr; q += NSX)
        static_for<NSX>([&](auto sc) { round(sc, q + decltype(sc)::value, std::true_type{}); });
    static_for<NSX - 1>([&](auto sc) {
        if (q + decltype(sc)::value < nr) round(sc, q + decltype(sc)::value, std::false_type{});
    });

    // ---- the K-groups' sums, G 32-row tiles at a time ----
    // Wave w's two tiles of row tile i go to X stage w / 2 at float
    // (i % G) * 4096 + (w % 2) * 2048, as [tile][element v][lane]: G = 2 where
    // a stage holds two waves' tiles twice (TM = 4), which halves the
    // barriers, else 1.  D[m][col] of a 32 x 32 tile is element
    // 4 (m / 8) + m % 4 of lane col + 32 ((m / 4) % 2).  Every thread then
    // sums 4 columns (one set) or 2 gate and 2 up columns (pair) of one row
    // over the 8 waves, in wave order.
    constexpr int G = XS * 16 >= 2 * 2 * 8 * 1024 ? 2 : 1;
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    WIDE_LDS_BARRIER();
    auto buf = [&](int w, int d) -> float* {
        u32x4* st = (w >> 1) == 0 ? xs0 : (w >> 1) == 1 ? xs1 : (w >> 1) == 2 ? xs2 : xs3;
        return reinterpret_cast<float*>(st) + d * 4096 + (w & 1) * 2048;
    };
    constexpr int NV = PAIR ? 2 : 4;     // columns a thread sums
    const size_t nw = PAIR ? 2 * (size_t)p.N : (size_t)p.N;
    const int ml = tid >> 4, cq = tid & 15;
    const int l0 = 32 * ((ml >> 2) & 1), v = 4 * (ml >> 3) + (ml & 3);
    // one set: tile cq / 8, columns 4 (cq % 8) ..; pair: columns 2 cq ..
    const int j0 = PAIR ? 0 : cq >> 3;
    const int c0 = PAIR ? 2 * cq : 4 * (cq & 7);
    const int n = n0 + 32 * j0 + c0;
    // this split's sums, kept for the fix-up should this block be the last
    float own0[TM][NV], own1[TM][NV];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int e = 0; e < NV; ++e) own0[i][e] = own1[i][e] = 0.0f;
#pragma unroll
    for (int i0 = 0; i0 < TM; i0 += G) {
        if (i0 > 0) WIDE_LDS_BARRIER();
#pragma unroll
        for (int d = 0; d < G && i0 + d < TM; ++d) {
            float* const mine = buf(wave, d);
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) mine[j * 1024 + e * 64 + lane] = acc[i0 + d][j][e];
        }
        WIDE_LDS_BARRIER();
#pragma unroll
        for (int d = 0; d < G && i0 + d < TM; ++d) {
            const int i = i0 + d;
            const int brow = 32 * i + ml;
            const int m = m0 + brow;
            if (brow >= wa.mrows || m >= p.M) continue;
            float x0[NV], x1[NV];
#pragma unroll
            for (int e = 0; e < NV; ++e) x0[e] = x1[e] = 0.0f;
#pragma unroll
            for (int w = 0; w < NWV; ++w) {
                const float* bw = buf(w, d) + v * 64 + l0 + c0;
                if constexpr (PAIR) {
                    const float2 g = *reinterpret_cast<const float2*>(bw);
                    const float2 u = *reinterpret_cast<const float2*>(bw + 1024);
                    x0[0] += g.x;
                    x0[1] += g.y;
                    x1[0] += u.x;
                    x1[1] += u.y;
                } else {
                    const f32x4 g = *reinterpret_cast<const f32x4*>(bw + j0 * 1024);
#pragma unroll
                    for (int e = 0; e < 4; ++e) x0[e] += g[e];
                }
            }
            if constexpr (SPLIT) {
                const __amdgpu_buffer_rsrc_t rs = ws_rsrc(p.ws);
                const size_t r = ((size_t)split * p.M + m) * nw;
                store_f32v_sc1<NV>(rs, r, n, p.N, x0);
                if constexpr (PAIR) store_f32v_sc1<NV>(rs, r + p.N, n, p.N, x1);
#pragma unroll
                for (int e = 0; e < NV; ++e) {
                    own0[i][e] = x0[e];
                    own1[i][e] = x1[e];
                }
            } else if constexpr (PAIR) {
                const bool gelu = p.epilogue == kEpiGeluMul;
#pragma unroll
                for (int e = 0; e < NV; ++e) x0[e] = glu_f32(gelu, x0[e], x1[e]);
                store_outv<NV>(p, (size_t)m * p.N, n, x0);
            } else {
                epi_storev<NV>(p, (size_t)m * p.N, n, x0);
            }
        }
    }
    if constexpr (SPLIT) {
        // the last of the tile's blocks (q4_split.hpp) adds the splits
        if (!split_arrive_last(p.tickets + blockIdx.y * gridDim.x + blockIdx.x, gridDim.z)) return;
        if (gridDim.z == 2) wide_fixup<2, TM, PAIR, NV>(p, m0, wa.mrows, ml, n, split, own0, own1);
        else if (gridDim.z == 3) wide_fixup<3, TM, PAIR, NV>(p, m0, wa.mrows, ml, n, split, own0, own1);
        else if (gridDim.z == 4) wide_fixup<4, TM, PAIR, NV>(p, m0, wa.mrows, ml, n, split, own0, own1);
        else wide_fixup<8, TM, PAIR, NV>(p, m0, wa.mrows, ml, n, split, own0, own1);
    }
}

template <int TM, bool PAIR>
hipError_t launch_tm(const GemmParams& p, const WideArgs& wa, const dim3& grid, bool split,
                     hipStream_t st) {
    if (split)
        hipLaunchKernelGGL((q4_wide_kernel<TM, PAIR, true>), grid, dim3(WT), 0, st, p, wa);
    else
        hipLaunchKernelGGL((q4_wide_kernel<TM, PAIR, false>), grid, dim3(WT), 0, st, p, wa);
    return hipGetLastError();
}

}  // namespace

// Plan: M-blocks of at most 128 rows (balanced), TM = the 32-row tiles of
// one; K split across blocks when the blocks would not fill the GPU (and
// until a block's K range holds at most 64 scale groups), in whole rounds.
bool wide_plan(const GemmParams& p, bool a_bf16, WidePlan* out) {
    if (a_bf16 || p.M <= 32 || p.M > 256 || p.N < 1) return false;
    if (p.K <= 0 || p.K % RK != 0 || p.gshift < 0 || p.gshift > 2) return false;
    const bool pair = p.w1 != nullptr;
    if (pair && p.epilogue != kEpiSiluMul && p.epilogue != kEpiGeluMul) return false;
    if (!pair && p.epilogue != kEpiNone && p.epilogue != kEpiGeluTanh &&
        p.epilogue != kEpiResidual)
        return false;
    // 16-byte X pieces: 16-byte aligned X (K % 8 == 0 keeps every row so);
    // packed W moves as dwords
    if ((reinterpret_cast<uintptr_t>(p.a) & 15) != 0) return false;
    WidePlan pl;
    pl.mblocks = (p.M + 127) / 128;
    pl.mrows = (p.M + pl.mblocks - 1) / pl.mblocks;
    pl.tm = (pl.mrows + 31) / 32;
    if (pl.tm < 2) pl.tm = 2;
    pl.nblocks = (p.N + (pair ? 31 : WBN - 1)) / (pair ? 32 : WBN);
    // Two M-blocks of up to 128 rows that fill 160-255 CUs where three
    // fit one round: three, of up to 86 rows (Llama q|k|v, 80 blocks per
    // M-block: 14.7 / 17.2 / 17.4 against 17.0 / 19.9 / 20.3 us at M = 160 /
    // 200 / 256).
    if (pl.mblocks == 2 && pl.nblocks * 2 >= 160 && pl.nblocks * 3 <= kCUs) {
        pl.mblocks = 3;
        pl.mrows = (p.M + 2) / 3;
        pl.tm = (pl.mrows + 31) / 32;
    }
    const int g = 32 << p.gshift;
    const int rounds = p.K / RK;
    const long blocks = (long)pl.nblocks * pl.mblocks;
    int s = 1;   // 1, 2, 3, 4 or 8 (the fix-up's instantiations)
    while (s < 8 && rounds % (2 * s) == 0 &&
           ((long)p.K / s / g > SLAB_G || (blocks * s < 160 && rounds / (2 * s) >= 4)))
        s *= 2;
    // Two splits that leave a quarter of the CUs idle, where three fit one
    // round: three (Llama q|k|v, 80 blocks: 240 instead of 160; 11.2 / 11.8
    // / 15.9 against 12.2 / 12.6 / 17.0 us at M = 33 / 64 / 128).
    if (s < 3 && blocks * s < 192 && blocks * 3 <= kCUs && rounds % 3 == 0 && rounds / 3 >= 4 &&
        (long)p.K / 3 / g <= SLAB_G)
        s = 3;
    if ((long)p.K / s / g > SLAB_G) return false;
    // One block per CU: a grid of more than one round of 256 blocks repeats
    // the whole per-block time.  Measured against the GEMM (us, weights
    // rotated over >= 1.5 GB): one round wins on every Llama and T5 shape
    // (e.g. gate/up + SiLU at M = 128: 24.9 against 33.5, T5 wo 26.2 against
    // 30.8); two rounds lose at M >= 100 (gate/up at M = 200: 45.7 against
    // 41.3, the T5 GeGLU pair's 320 blocks at M = 128: 55.3 against 42.4)
    // and still win at M <= 64 (that pair at M = 64: 34.8 against 37.3).
    const long grid = blocks * s;
    if (grid > kCUs && !(p.M <= 64 && grid <= 2 * kCUs)) return false;
    pl.splits = s;
    pl.kblk = p.K / s;
    pl.ws_bytes = s > 1 ? (size_t)s * p.M * (pair ? 2 : 1) * p.N * sizeof(float) : 0;
    *out = pl;
    return true;
}

hipError_t launch_wide(GemmParams p, const WidePlan& pl, hipStream_t st) {
    const bool pair = p.w1 != nullptr;
    // split launches: a counter per output tile, and partial-sum offsets that
    // fit the 32-bit byte offsets of the workspace's buffer accesses
    if (pl.splits > 1 && (!p.ws || !p.tickets || pl.nblocks * pl.mblocks > kTickets ||
                          pl.ws_bytes > 0x7fffffffu))
        return hipErrorInvalidValue;
    p.splits = pl.splits;
    const WideArgs wa = {pl.mrows, pl.kblk};
    const dim3 grid((unsigned)pl.nblocks, (unsigned)pl.mblocks, (unsigned)pl.splits);
    const bool split = pl.splits > 1;
    hipError_t e;
    if (pair) {
        if (pl.tm == 2) e = launch_tm<2, true>(p, wa, grid, split, st);
        else if (pl.tm == 3) e = launch_tm<3, true>(p, wa, grid, split, st);
        else e = launch_tm<4, true>(p, wa, grid, split, st);
    } else {
        if (pl.tm == 2) e = launch_tm<2, false>(p, wa, grid, split, st);
        else if (pl.tm == 3) e = launch_tm<3, false>(p, wa, grid, split, st);
        else e = launch_tm<4, false>(p, wa, grid, split, st);
    }
    return e;
}

}  // namespace sltx
