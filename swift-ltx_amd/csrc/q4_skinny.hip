// q4_skinny.hip -- 4-bit dequant matmul for small M (1..32 activation rows:
// short prompts, the T5 encoder's S <= 128 layers, batched decode) on CDNA4
// MFMA, as a weight stream.
//
// Same product as q4_gemm.hip, Y[M,N] = X[M,K] . dequant(W)[N,K]^T with fp32
// accumulation (matmulQ4Fast, Ops.swift:312-381).  At small M each weight
// byte feeds only M multiply-adds, so the kernel is bound by the weight
// stream, like the GEMV: the block tile of the large-M GEMM (128 or 192
// activation rows, LDS-staged weights) would pad M and re-stage weights for
// nothing.  Here:
//  * A block owns 16 * RT weight rows (of each weight set: gate and up for
//    the gated epilogues) and all K; its W waves split K into equal slices of
//    128 * STEPS.  In wave w, lane l covers row l % 16 of each 16-row tile
//    and, in each 128-wide k-step, the 32 k at offset 32 * (l / 16): one
//    16-byte load of packed words per step.  Two steps are loaded together
//    as 8 rows x 128 contiguous bytes per wave-wide load and swapped into
//    that layout with one DPP move per word.  Every load of a wave is issued
//    before the first MFMA, in the order of use.
//  * The block's scales and biases (one contiguous slab per array) are
//    copied to LDS with direct 16-byte global -> LDS loads, issued first.
//  * The wave's slice of X (all M rows, 16 per MFMA tile) stays in
//    registers for the whole kernel.  With one 16-row tile and M * K * 2
//    bytes that fit (XL), the block first copies the M real rows to LDS
//    (rows padded by 16 bytes: the 16 rows of a fragment read hit distinct
//    banks), before its weight loads, and each wave reads its fragments from
//    there, with zeros for rows past M: every 16-byte load through the
//    vector memory path costs that path 16 cycles whatever its lanes hold,
//    so fragments loaded from memory for all 16 rows (zeros past M) cost
//    the CU more load issue than its weights at small M.  Otherwise the
//    fragments are read through a buffer resource of M * K fp16, so that
//    rows past M read as zeros without a branch.
//  * Each word is dequantized in registers without leaving fp16: its
//    nibbles are spread to bytes (q0 q2 q4 q6 and q1 q3 q5 q7), and
//    v_cvt_scalef32_pk_f16_fp8 turns two bytes into two fp16 at a time: read
//    as fp8 e4m3, a byte b < 16 is b * 2^-9 exactly (the subnormals and the
//    first binade share one spacing), and the instruction's scale, of which
//    only the exponent counts, is 2^9.  One v_pk_fma_f16 per pair then gives
//    s * q + b with the GEMM's single rounding.  The k order inside a word
//    is 0,2,1,3,4,6,5,7; X is permuted alike when it is loaded, once per
//    wave.  Four MFMAs per 16-byte load accumulate into the tile's
//    accumulators directly.
//  * The partial tiles of the W waves are summed through LDS once, then the
//    epilogue (gated SiLU / GELU-tanh pair, bias, GELU-tanh, residual add)
//    runs on the fp32 sums.
#include "q4_common.hpp"
#include "q4_dequant.hpp"
#include "q4_launch.hpp"

namespace sltx {

namespace {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 16-byte pieces of one array's scale / bias slab (rows x groups fp16), and
// the pieces reserved per slab in LDS (whole waves of 64).
__host__ __device__ constexpr int slab_pieces(int rows, int groups) { return rows * groups / 8; }
__host__ __device__ constexpr int slab_alloc(int rows, int groups) {
    return (slab_pieces(rows, groups) + 63) / 64 * 64;
}

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// W waves, MT tiles of 16 activation rows, STEPS 128-wide k-steps per wave,
// PAIR: two weight sets (gate, up) and a gated epilogue, RT tiles of 16
// weight rows per block.  OCC: blocks per CU the register budget is sized for.
template <int W, int MT, int STEPS, bool PAIR, int RT, int OCC, bool XL>
__global__ __launch_bounds__(64 * W, OCC) void q4_skinny_kernel(GemmParams p) {
    constexpr int NS = PAIR ? 2 : 1;
    constexpr int ROWS = 16 * RT;
    static_assert(!XL || MT == 1, "LDS X holds one 16-row tile");
    __shared__ f32x4 red[W][RT][NS][MT][64];
    // [2 * NS slabs][ROWS][groups] fp16, then (XL) X rows [M][K + 8] fp16
    extern __shared__ u32x4 sb_lds[];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, kq = lane >> 4;
    const int n0 = blockIdx.x * ROWS;
    const int K = p.K, groups = p.groups;
    const int kw0 = wave * (128 * STEPS) + 32 * kq;   // this lane's first k

    // ---- scales and biases -> LDS (slab a: s0, b0[, s1, b1]) ----
    const int pieces = slab_pieces(ROWS, groups), alloc = slab_alloc(ROWS, groups);
    const int valid = min(ROWS, p.N - n0) * groups * 2;   // slab bytes inside the arrays
    constexpr int RA = (RT * STEPS + 7) / 8;              // rounds per slab (groups <= K/32)
#pragma unroll
    for (int a = 0; a < 2 * NS; ++a) {
        const uint16_t* arr = a == 0 ? p.s0 : a == 1 ? p.b0 : a == 2 ? p.s1 : p.b1;
        const char* src = reinterpret_cast<const char*>(arr + (size_t)n0 * groups);
#pragma unroll
        for (int r = 0; r < RA; ++r) {
            const int c0 = r * 64 * W + 64 * wave;   // wave-uniform
            if (c0 < pieces) {
                int off = (c0 + lane) * 16;
                if (off >= valid) off = 0;          // a spare copy of piece 0
                __builtin_amdgcn_global_load_lds((const void*)(src + off),
                                                 (lds_ptr_t)(sb_lds + a * alloc + c0), 16, 0, 0);
            }
        }
    }
    // ---- XL: X rows [0, M) -> LDS, 1 KB (one wave-wide copy) at a time ----
    const int xrow16 = K / 8 + 1;   // LDS row stride in 16-byte units (one of padding)
    u32x4* const xl = sb_lds + 2 * NS * alloc;
    if constexpr (XL) {
        const int per_row = K / 512;   // 1 KB chunks per row (K % 1024 == 0)
        for (int c = wave; c < p.M * per_row; c += W) {   // wave-uniform
            const int m = c / per_row, j = c - m * per_row;
            const char* src = reinterpret_cast<const char*>(p.a) + (size_t)m * K * 2 +
                              j * 1024 + lane * 16;
            __builtin_amdgcn_global_load_lds((const void*)src,
                                             (lds_ptr_t)(xl + m * xrow16 + j * 64), 16, 0, 0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- the wave's slice of X: fragment r of step t is x[k .. k+7] with
    // k = kw0 + 128 t + 8 r, the k of word r of the lane's packed load ----
    u32x4 xa[MT][STEPS][4];
    if constexpr (!XL) {
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<void*>(p.a), (short)0, p.M * K * 2, 0x00020000);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int xrow = ((mt * 16 + r16) * K + kw0) * 2;
#pragma unroll
            for (int t = 0; t < STEPS; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    xa[mt][t][r] = __builtin_bit_cast(
                        u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, xrow + 256 * t + 16 * r, 0, 0));
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- packed words, step by step ----
    // Steps t, t+1 of a tile and set are loaded as 2 x 8 rows x 128 bytes
    // (whole lines: load h, lane l reads row (l & 7) | 8h, piece
    // 4 * bit3(l) + l / 16 of the 128-byte run) and swapped into the MFMA
    // layout before use: a load of the layout itself is 16 rows x 64 bytes,
    // every request half a line, and streams ~15% slower.  An odd last step
    // keeps that layout.
    u32x4 wq[STEPS][RT][NS];
    const int prow = lane & 7, ppiece = 4 * ((lane >> 3) & 1) + (lane >> 4);
#pragma unroll
    for (int t = 0; t < STEPS; t += 2) {
        if (t + 1 < STEPS) {
#pragma unroll
            for (int i = 0; i < RT; ++i)
#pragma unroll
                for (int s = 0; s < NS; ++s)
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const int row = min(n0 + 16 * i + (prow | (h << 3)), p.N - 1);
                        const uint32_t* wr = (s ? p.w1 : p.w0) + (size_t)row * (K / 8) +
                                             (wave * 128 * STEPS + 128 * t) / 8 + ppiece * 4;
                        wq[t + h][i][s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr));
                    }
        } else {
#pragma unroll
            for (int i = 0; i < RT; ++i)
#pragma unroll
                for (int s = 0; s < NS; ++s) {
                    const int row = min(n0 + 16 * i + r16, p.N - 1);
                    const uint32_t* wr = (s ? p.w1 : p.w0) + (size_t)row * (K / 8) + kw0 / 8;
                    wq[t][i][s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + 16 * t));
                }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // The slabs are complete once at most the X and weight loads issued after
    // them are outstanding (every wave issues all of those).  Both waits are
    // builtins: with a wait in inline assembly the compiler loses its count
    // of the loads in flight and waits for all of them at the next use.  The
    // barrier is assembly with a memory clobber, so that no LDS read moves
    // above it.
    __builtin_amdgcn_s_waitcnt(vmcnt_only((XL ? 0 : MT * STEPS * 4) + STEPS * RT * NS));
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (XL) {   // rows past M read row 0 and are replaced by zeros
        const bool live = r16 < p.M;
        const u32x4* xr = xl + (live ? r16 : 0) * xrow16 + kw0 / 8;
        const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int t = 0; t < STEPS; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const u32x4 v = xr[16 * t + r];
                xa[0][t][r] = live ? v : zero;
            }
    }

#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < STEPS; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) xa[mt][t][r] = permute_x(xa[mt][t][r]);

    const uint16_t* sbl = reinterpret_cast<const uint16_t*>(sb_lds);
    const int gshift = 5 + p.gshift;   // log2(group size)
    f32x4 acc[RT][NS][MT];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[i][s][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
        if ((t & 1) == 0 && t + 1 < STEPS) {
            // lane l of the pair's load h holds row (l & 7) | 8h, piece
            // 4 * bit3(l) + l / 16: lanes whose bit 3 is h already hold their
            // step-h data; the others take it from lane l ^ 8 of the other
            // load (a row rotation by 8 inside each 16-lane row, written
            // only to the banks of 4 lanes that need it)
#pragma unroll
            for (int i = 0; i < RT; ++i)
#pragma unroll
                for (int s = 0; s < NS; ++s)
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const int r0 = (int)wq[t][i][s][c], r1 = (int)wq[t + 1][i][s][c];
                        wq[t][i][s][c] = (uint32_t)__builtin_amdgcn_update_dpp(r0, r1, 0x128, 0xF, 0xC, false);
                        wq[t + 1][i][s][c] = (uint32_t)__builtin_amdgcn_update_dpp(r1, r0, 0x128, 0xF, 0x3, false);
                    }
        }
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                // the lane's 32 k lie in one group (group sizes 32, 64, 128)
                const int gi = (kw0 + 128 * t) >> gshift;
                const uint16_t* srow = sbl + (size_t)(2 * s) * alloc * 8 + (16 * i + r16) * groups;
                const uint32_t sv = srow[gi], bv = srow[alloc * 8 + gi];
                const f16x2 s2 = as_f16x2(sv | (sv << 16));
                const f16x2 b2 = as_f16x2(bv | (bv << 16));
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const u32x4 b = dequant_word(wq[t][i][s][r], s2, b2);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        acc[i][s][mt] = mfma16(xa[mt][t][r], b, acc[i][s][mt]);
                }
            }
    }

#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) red[wave][i][s][mt][lane] = acc[i][s][mt];
    __syncthreads();

    // one output per thread: D[m][n] of a 16x16 tile sits in lane
    // 16 * (m / 4) + n, element m % 4
    for (int o = threadIdx.x; o < RT * MT * 256; o += 64 * W) {
        const int i = o / (MT * 256), mt = (o >> 8) % MT, ml = (o >> 4) & 15, nl = o & 15;
        const int m = mt * 16 + ml, n = n0 + 16 * i + nl;
        if (m >= p.M || n >= p.N) continue;
        const int src = 16 * (ml >> 2) + nl, e = ml & 3;
        float v[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            float a = 0.0f;
#pragma unroll
            for (int w = 0; w < W; ++w) a += red[w][i][s][mt][src][e];
            v[s] = a;
        }
        float out;
        if constexpr (PAIR) {
            out = glu_f32(p.epilogue == kEpiGeluMul, v[0], v[NS - 1]);
        } else {
            out = v[0];
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

// Registers of a configuration, roughly: X fragments, the packed words in
// flight, accumulators, and about 40 for the rest.
constexpr int skinny_vgprs(int mt, int steps, int ns, int rt) {
    return 16 * mt * steps + 4 * rt * ns * steps + 4 * rt * ns * mt + 40;
}
constexpr int kSkinnyMaxVgprs = 224;   // of the 256 one block of 8 waves may use

// Dynamic LDS of a launch: the scale / bias slabs, then (XL) X's rows.
size_t skinny_lds(const GemmParams& p, int rt, bool pair, bool xl) {
    return (size_t)(pair ? 4 : 2) * slab_alloc(16 * rt, p.groups) * 16 +
           (xl ? (size_t)p.M * (p.K / 8 + 1) * 16 : 0);
}

// Blocks per CU a configuration is compiled for: two when a wave fits in
// 128 VGPRs.
constexpr int skinny_occ(int w, int mt, int steps, int ns, int rt) {
    return (w == 8 && skinny_vgprs(mt, steps, ns, rt) <= 120) ? 2 : 1;
}

template <int W, int MT, int STEPS, bool PAIR, int RT, bool XL>
hipError_t launch_cfg(const GemmParams& p, hipStream_t st) {
    constexpr int OCC = skinny_occ(W, MT, STEPS, PAIR ? 2 : 1, RT);
    const dim3 grid((unsigned)((p.N + 16 * RT - 1) / (16 * RT))), block(64 * W);
    const size_t lds = skinny_lds(p, RT, PAIR, XL);
    hipLaunchKernelGGL((q4_skinny_kernel<W, MT, STEPS, PAIR, RT, OCC, XL>), grid, block, lds, st, p);
    return hipGetLastError();
}

template <int W, int MT, int STEPS, bool PAIR, int RT>
hipError_t launch_xl(const GemmParams& p, bool xl, hipStream_t st) {
    if constexpr (MT == 1) {
        if (xl) return launch_cfg<W, MT, STEPS, PAIR, RT, true>(p, st);
    }
    return launch_cfg<W, MT, STEPS, PAIR, RT, false>(p, st);
}

template <int W, int MT, int STEPS>
hipError_t launch_steps(const GemmParams& p, const SkinnyPlan& pl, hipStream_t st) {
    const bool pair = p.w1 != nullptr;
    if (pl.RT == 2) {
        if constexpr (W == 8 && skinny_vgprs(MT, STEPS, 2, 2) <= kSkinnyMaxVgprs)
            return pair ? launch_xl<W, MT, STEPS, true, 2>(p, pl.XL, st)
                        : launch_xl<W, MT, STEPS, false, 2>(p, pl.XL, st);
        return hipErrorInvalidValue;
    }
    if (pair) {
        // a gated pair of 5 steps does not fit the 128 VGPRs of 16 waves
        if constexpr (W == 16 && STEPS == 5) return hipErrorInvalidValue;
        else return launch_xl<W, MT, STEPS, true, 1>(p, pl.XL, st);
    }
    return launch_xl<W, MT, STEPS, false, 1>(p, pl.XL, st);
}

}  // namespace

bool skinny_plan(const GemmParams& p, bool a_bf16, SkinnyPlan* out) {
    if (a_bf16 || p.M < 1 || p.M > 32 || p.N < 1 || p.K <= 0) return false;
    if (p.gshift < 0 || p.gshift > 2) return false;
    if ((long)p.M * p.K * 2 > 0x7fffffffL) return false;   // X buffer offsets are 32-bit
    const bool pair = p.w1 != nullptr;
    if (pair && p.epilogue != kEpiSiluMul && p.epilogue != kEpiGeluMul) return false;
    if (!pair && p.epilogue != kEpiNone && p.epilogue != kEpiGeluTanh &&
        p.epilogue != kEpiResidual)
        return false;
    const int mt = p.M <= 16 ? 1 : 2;
    SkinnyPlan pl{0, mt, 0, 1, 1, false};
    // 8 waves of 1..6 steps (1..4 with 32 activation rows), else 16 waves of
    // 1..5 steps (1..4 for a gated pair; 16 activation rows)
    if (p.K % 1024 == 0 && p.K / 1024 <= (mt == 1 ? 6 : 4)) {
        pl.W = 8;
        pl.STEPS = p.K / 1024;
    } else if (mt == 1 && p.K % 2048 == 0 && p.K / 2048 <= (pair ? 4 : 5)) {
        // (a gated pair of 5 steps does not fit the 128 VGPRs of 16 waves)
        pl.W = 16;
        pl.STEPS = p.K / 2048;
    } else {
        return false;
    }
    // Two row tiles per block (the X slice serves twice the weight rows), with
    // 8 waves and at least one block per CU: when the two-tile block still
    // fits two per CU, or above 8 activation rows.  Measured: the vocabulary
    // head at M = 2 takes 43.8 us with two tiles (two blocks per CU) against
    // 53.5 us with one; the gate/up pair at M = 8 (two tiles: one block per
    // CU) 10.6 against 10.1 us, at M = 16 11.2 against 12.4 us.
    const int ns = pair ? 2 : 1;
    // (launch_steps instantiates two tiles where a gated pair of them fits
    // the register budget; every two-tile block that fits two per CU does)
    if (pl.W == 8 && (p.N + 31) / 32 >= kCUs &&
        (skinny_occ(8, mt, pl.STEPS, ns, 2) == 2 ||
         (p.M > 8 && skinny_vgprs(mt, pl.STEPS, 2, 2) <= kSkinnyMaxVgprs)))
        pl.RT = 2;
    pl.OCC = skinny_occ(pl.W, mt, pl.STEPS, ns, pl.RT);
    // X in LDS: one 16-row tile whose rows fit beside the slabs, so that a
    // block still gets its share of the CU's LDS
    pl.XL = mt == 1 && skinny_lds(p, pl.RT, pair, true) <= (size_t)(pl.RT == 2 ? 128 : 64) * 1024;
    // scales and biases are staged with 16-byte loads
    const uintptr_t sb = reinterpret_cast<uintptr_t>(p.s0) | reinterpret_cast<uintptr_t>(p.b0) |
                         (pair ? reinterpret_cast<uintptr_t>(p.s1) | reinterpret_cast<uintptr_t>(p.b1)
                               : 0);
    if ((sb & 15) != 0) return false;
    *out = pl;
    return true;
}

hipError_t launch_skinny(const GemmParams& p, const SkinnyPlan& pl, hipStream_t st) {
    if (pl.W == 8 && pl.MT == 1) {
        switch (pl.STEPS) {
            case 1: return launch_steps<8, 1, 1>(p, pl, st);
            case 2: return launch_steps<8, 1, 2>(p, pl, st);
            case 3: return launch_steps<8, 1, 3>(p, pl, st);
            case 4: return launch_steps<8, 1, 4>(p, pl, st);
            case 5: return launch_steps<8, 1, 5>(p, pl, st);
            case 6: return launch_steps<8, 1, 6>(p, pl, st);
        }
    } else if (pl.W == 8 && pl.MT == 2) {
        switch (pl.STEPS) {
            case 1: return launch_steps<8, 2, 1>(p, pl, st);
            case 2: return launch_steps<8, 2, 2>(p, pl, st);
            case 3: return launch_steps<8, 2, 3>(p, pl, st);
            case 4: return launch_steps<8, 2, 4>(p, pl, st);
        }
    } else if (pl.W == 16 && pl.MT == 1) {
        switch (pl.STEPS) {
            case 1: return launch_steps<16, 1, 1>(p, pl, st);
            case 2: return launch_steps<16, 1, 2>(p, pl, st);
            case 3: return launch_steps<16, 1, 3>(p, pl, st);
            case 4: return launch_steps<16, 1, 4>(p, pl, st);
            case 5: return launch_steps<16, 1, 5>(p, pl, st);
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace sltx
