// q4_gemv.hip -- 4-bit dequant GEMV (decode, M == 1) for gfx950.
//
// Computes y[n] = sum_k x[k] * (s[n,k/g] * q[n,k] + b[n,k/g]) with fp32
// accumulation and an fp16 store: the semantics of swift-ltx's matmul_q4
// (Kernels.swift:444-620) at M == 1, dispatched by matmulQ4 (Ops.swift:285-305).
// The SWIGLU variant computes silu(x.Wg^T) * (x.Wu^T) in one pass, replacing
// linear(gate) + linear(up) + siluMul (LlamaModel.swift:327-329, Kernels.swift:90-98).
//
// Work decomposition (HBM-bound; every weight byte is read exactly once):
//   * A row of K nibbles is K/32 "chunks" of 32 nibbles = one 16-byte load.
//   * L lanes share a row: lane kl reads chunks kl, kl+L, ... (CPL of them), so a
//     wave-wide load covers 64/L rows with contiguous 16*L-byte segments.
//   * Each lane always sees the same chunk positions, so the x values it needs
//     are prepared once per block (in LDS) and held in registers for all of
//     its rows.  Each wave owns T row-iterations of 64/L rows.
//
// Dequant + dot (per 32-bit word of 8 nibbles q0..q7 for x0..x7):
//   p0 = (w      & 0x000F000F) | 0x6400_6400  -> fp16 pair (1024+q0,    1024+q4)
//   p1 = (w      & 0x00F000F0) | 0x6400_6400  -> fp16 pair (1024+16q1,  1024+16q5)
//   p2 = (w>>8   & 0x000F000F) | 0x6400_6400  -> fp16 pair (1024+q2,    1024+q6)
//   p3 = (w>>8   & 0x00F000F0) | 0x6400_6400  -> fp16 pair (1024+16q3,  1024+16q7)
// dotted (v_dot2_f32_f16, fp32 accumulate) with the x pairs (x0,x4),
// (x1/16,x5/16), (x2,x6), (x3/16,x7/16).  This gives sum(q*x) + 1024*sum(xs),
// where xs are the x values as scaled.  The second term ("corr") depends on x
// only and is subtracted by starting the accumulator at -corr.  Per chunk:
//   acc += s_g * (sum q*x)  +  b_g * (sum x)
// which is the reference's own bias factoring (Kernels.swift:594-600).
#include "q4_common.hpp"
#include "q4_gemv_ops.hpp"
#include "q4_launch.hpp"

namespace sltx {


// Prepared x for one chunk of 32 values: 16 fp16 pairs in dot order, plus
// (-corr, sum).  Stored planar in LDS: xs[j][chunk] holds pairs 4j..4j+3.
constexpr int kGemvMaxWaves = 16;   // waves per block: 4 .. 16, chosen per launch

template <int NCH, int MR>
struct GemvLds {
    u32x4 xs[MR][4][NCH];       // per x row
    float2 xc[MR][NCH];
    float red[kGemvMaxWaves];   // per-wave partial sums of squares (RMS-norm prologue)
};

// One row-iteration's operands for one lane: CPL weight chunks per weight
// set and their group scale/bias bit patterns (kept as 32-bit registers so
// the loads are not merged with a wait in between).
template <int CPL, int NW, int MR>
struct GemvStage {
    u32x4 w[NW][CPL];
    uint32_t s[NW][CPL];
    uint32_t b[NW][CPL];
    uint32_t res[MR];   // residual of the row, per x row (residual epilogue only)
    float bias;         // bias of the row (two x rows only)
};

// Row index is clamped into [0, N) so every load is unconditional (a
// predicated load would be compiled into a branch with a wait inside it);
// clamped rows are computed and discarded.
template <int L, int CPL, int NW, int MR>
__device__ __forceinline__ void gemv_load(GemvStage<CPL, NW, MR>& st, const GemvParams& p, int r,
                                          int kl) {
    constexpr int NCH = L * CPL;
    const int rr = r < p.N ? r : p.N - 1;
#pragma unroll
    for (int m = 0; m < NW; ++m) {
        const u32x4* W = reinterpret_cast<const u32x4*>(m == 0 ? p.w0 : p.w1);
        const uint16_t* S = m == 0 ? p.s0 : p.s1;
        const uint16_t* B = m == 0 ? p.b0 : p.b1;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = kl + i * L;
            st.w[m][i] = __builtin_nontemporal_load(&W[(size_t)rr * NCH + c]);
            const size_t gi = (size_t)rr * p.groups + (c >> p.gshift);
            st.s[m][i] = S[gi];
            st.b[m][i] = B[gi];
        }
    }
    // fetched with the weights so the epilogue does not wait a memory latency
    if constexpr (MR == 1) {
        if (p.residual) st.res[0] = p.residual[rr];
    } else {
        if (p.residual) {
#pragma unroll
            for (int mr = 0; mr < MR; ++mr) st.res[mr] = p.residual[(size_t)mr * p.N + rr];
        }
        if (p.bias) st.bias = p.bias[rr];
    }
}

template <int L, int CPL, int NW, int MR>
__device__ __forceinline__ void gemv_compute_store(const GemvStage<CPL, NW, MR>& st,
                                                   const u32x4 (&xq)[MR][CPL][4],
                                                   const float2 (&xc)[MR][CPL],
                                                   const GemvParams& p, int r, int kl) {
    if constexpr (MR == 1) {
        float acc[NW];
#pragma unroll
        for (int m = 0; m < NW; ++m) {
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const float d = chunk_dot(st.w[m][i], xq[0][i], xc[0][i].x);
                a = fmaf(h2f((uint16_t)st.s[m][i]), d, a);
                a = fmaf(h2f((uint16_t)st.b[m][i]), xc[0][i].y, a);
            }
            acc[m] = row_reduce<L>(a);
        }
        if (kl == 0 && r < p.N) {
            const float out = NW == 2 ? glu_f32(p.gelu, acc[0], acc[NW - 1]) : acc[0];
            p.y[r] = p.residual ? residual_add_f16((uint16_t)st.res[0], out) : f2h(out);
        }
    } else {
        // two x rows: each weight word dequantized once for both
        float acc[NW][2];
#pragma unroll
        for (int m = 0; m < NW; ++m) {
            float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                float d0, d1;
                chunk_dot_x2(st.w[m][i], xq[0][i], xq[1][i], xc[0][i].x, xc[1][i].x, d0, d1);
                const float sc = h2f((uint16_t)st.s[m][i]), bc = h2f((uint16_t)st.b[m][i]);
                a0 = fmaf(sc, d0, a0);
                a0 = fmaf(bc, xc[0][i].y, a0);
                a1 = fmaf(sc, d1, a1);
                a1 = fmaf(bc, xc[1][i].y, a1);
            }
            acc[m][0] = row_reduce<L>(a0);
            acc[m][1] = row_reduce<L>(a1);
        }
        if (kl == 0 && r < p.N) {
#pragma unroll
            for (int mr = 0; mr < 2; ++mr) {
                // y [2, N] in y_dtype, + bias and GELU-tanh (one weight set)
                float out = NW == 2 ? glu_f32(p.gelu, acc[0][mr], acc[NW - 1][mr]) : acc[0][mr];
                const size_t o = (size_t)mr * p.N + r;
                if (p.bias) out += st.bias;
                if (p.gelu_tanh) out = gelu_tanh_f32(out);
                if (p.residual)
                    p.y[o] = residual_add_f16((uint16_t)st.res[mr], out);
                else if (p.y_dtype == kF32)
                    reinterpret_cast<float*>(p.y)[o] = out;
                else
                    p.y[o] = p.y_dtype == kBF16 ? f2bf(out) : f2h(out);
            }
        }
    }
}

// Each wave owns T consecutive row-iterations (T * 64/L rows), processed with
// a two-stage register pipeline: the loads of iteration t+1 are in flight
// while iteration t is computed.
// MULTI: T >= 2 row-iterations per wave (compile-time, so the one-iteration
// kernel carries no loop).  PRO (GemvPro): the input is x, rms_norm(x) or
// rms_norm(x + xb); each block recomputes the norm of its own copy of the
// input vector (K values) while its first weight loads are in flight.
// Largest block (in waves) of one instantiation: a block of w waves leaves a
// wave 2048 / w VGPRs (4 waves per SIMD at w = 16).  The two-weight-set and
// pipelined (MULTI) kernels hold two to four times the weight registers, and
// more than 4 chunks per lane doubles them again; each cap keeps its kernel
// free of spills.
template <int CPL, bool SWIGLU, bool MULTI, int MR = 1>
constexpr int gemv_max_waves() {
    return ((SWIGLU || MULTI || MR > 1) ? 8 : 16) / (CPL > 4 ? 2 : 1);
}

// Blocks of 4 to gemv_max_waves() waves (blockDim.x / 64, chosen per launch).
template <int L, int CPL, bool SWIGLU, bool MULTI, int PRO, int MR>
__global__ __launch_bounds__((64 * gemv_max_waves<CPL, SWIGLU, MULTI, MR>())) void q4_gemv_kernel(GemvParams p, int T) {
    constexpr int RPI = 64 / L;        // rows per wave-wide instruction
    constexpr int NCH = L * CPL;       // chunks per row (K / 32)
    constexpr int NW = SWIGLU ? 2 : 1; // weight sets
    static_assert(MR == 1 || (PRO == kProNone && !MULTI), "two x rows: no prologue, one iteration");
    __shared__ GemvLds<NCH, MR> lds;

    const int NTH = blockDim.x;        // 256 .. 1024 threads
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int kl = lane % L;
    const int sub = lane / L;
    const int row0 = (blockIdx.x * (NTH >> 6) + wave) * (RPI * T) + sub;

    // x loads first: vmcnt retires in issue order, so x issued after the
    // weights would make the x preparation wait for the HBM latency too.
    // The vector is prepared in units of G consecutive 8-value words of one
    // chunk; unit ui = threadIdx.x + NTH * u.  Vectors of up to 512 words take
    // one word per thread (G = 1): the serial conversion work per thread stays
    // short, and the four words of a chunk sit in one lane quad, which sums
    // their (corr, sum).  Longer vectors take a whole chunk per thread (G = 4),
    // which keeps the unrolled preparation code (one copy per unit a thread
    // may own) short.  Measured at K = 3072: q|k|v with rms_norm 4.32 -> 4.00
    // us, gate/up with residual + rms_norm 8.48 -> 8.03 us; at K = 8192 one
    // word per thread made the down launch slower (4.55 -> 4.88 us).
    constexpr int NWD = 4 * NCH;                // words in the input vector
    constexpr int G = NWD <= 512 ? 1 : 4;       // words per unit
    constexpr int NU = NWD / G;                 // units
    constexpr int XPU = (NU + 255) / 256;       // units per thread (at most)
    static_assert(G == 4 || NWD % 64 == 0, "one-word units: every lane of a preparing wave is valid");
    constexpr bool NORM = PRO != kProNone, RES = PRO == kProResidualRms;
    const int wave_base = __builtin_amdgcn_readfirstlane((int)(threadIdx.x & ~63u));
    // Waves whose units all lie past the vector skip the preparation
    // (wave-uniform branch); redundant loads would only delay the weight
    // loads queued behind them.  Lanes past the vector in a preparing wave
    // (G = 4 only) load the last unit and store nothing.
    auto has_units = [&](int u) { return wave_base + NTH * u < NU; };
    f16x8 xr[MR][XPU][G];
    f16x8 xb[RES ? XPU : 1][G];
    f32x4 nw[NORM ? XPU : 1][2 * G];
#pragma unroll
    for (int u = 0; u < XPU; ++u) {
        if (!has_units(u)) continue;
        const int ui = threadIdx.x + NTH * u;
        const int uc = ui < NU ? ui : NU - 1;
#pragma unroll
        for (int g = 0; g < G; ++g) {
#pragma unroll
            for (int mr = 0; mr < MR; ++mr)
                xr[mr][u][g] = reinterpret_cast<const f16x8*>(p.x)[mr * NWD + uc * G + g];
            if constexpr (RES) xb[u][g] = reinterpret_cast<const f16x8*>(p.xb)[uc * G + g];
        }
        if constexpr (NORM) {
#pragma unroll
            for (int q = 0; q < 2 * G; ++q) nw[u][q] = reinterpret_cast<const f32x4*>(p.norm_w)[uc * 2 * G + q];
        }
    }
    __builtin_amdgcn_sched_barrier(0);   // keep every x load ahead of the weight loads

    // The first stage's weight loads are issued before the x preparation and
    // stay in flight across the barrier below; the second stage follows after
    // it (measured: issuing both at once is slower for the 28 MB gate/up
    // launch, and keeps twice the registers live during the x preparation).
    GemvStage<CPL, NW, MR> sa, sb;
    gemv_load<L, CPL, NW, MR>(sa, p, row0, kl);
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (NORM) {
        // rms_norm (Kernels.swift:40-86) / residual_rms_norm (Kernels.swift:238-290):
        // v = x (or a + b, whose fp16 rounding is the residual stream); the
        // sum of squares uses the unrounded v; out = half(r * rms * w) with r
        // the (rounded) input and rms = rsqrt(mean(v^2) + eps).
        float ss = 0.0f;
#pragma unroll
        for (int u = 0; u < XPU; ++u) {
            if (!has_units(u)) continue;
            const int ui = threadIdx.x + NTH * u;
            if (ui >= NU) continue;
#pragma unroll
            for (int g = 0; g < G; ++g) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    float v = (float)xr[0][u][g][e];
                    if constexpr (RES) {
                        v += (float)xb[u][g][e];
                        xr[0][u][g][e] = (f16)v;
                    }
                    ss += v * v;
                }
                if constexpr (RES) {
                    if (blockIdx.x == 0) reinterpret_cast<f16x8*>(p.res_out)[ui * G + g] = xr[0][u][g];
                }
            }
        }
        ss = row_reduce<64>(ss);
        if ((threadIdx.x & 63) == 0) lds.red[threadIdx.x >> 6] = ss;
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        // the block sum of the wave partials: lane l of each 16-lane row reads
        // the partial of wave l % 16 (zero past the last wave), one LDS read
        // per lane and a fixed DPP tree, instead of a serial loop of
        // dependent LDS reads
        const int nwv = NTH >> 6, wl = threadIdx.x & 15;
        const float part = lds.red[wl < nwv ? wl : nwv - 1];
        const float ssum = row_reduce<16>(wl < nwv ? part : 0.0f);
        const float rms = rsqrtf(ssum / (float)p.K + p.eps);
#pragma unroll
        for (int u = 0; u < XPU; ++u) {
            if (!has_units(u)) continue;
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    xr[0][u][g][e] = (f16)((float)xr[0][u][g][e] * rms * nw[u][2 * g + (e >> 2)][e & 3]);
        }
    }

    // Prepare x once per block while the weight loads are in flight.
#pragma unroll
    for (int u = 0; u < XPU; ++u) {
        if (!has_units(u)) continue;
        const int ui = threadIdx.x + NTH * u;
        const bool ok = ui < NU;
        const int c = (ui * G) >> 2, j0 = (ui * G) & 3;
#pragma unroll
        for (int mr = 0; mr < MR; ++mr) {
            float corr = 0.0f, sum = 0.0f;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                uint32_t pr[4];
                pair_word(xr[mr][u][g], pr, corr, sum);
                u32x4 v = {pr[0], pr[1], pr[2], pr[3]};
                if (ok) lds.xs[mr][j0 + g][c] = v;
            }
            if constexpr (G == 1) {
                corr = dpp_add<0x4E>(dpp_add<0xB1>(corr));
                sum = dpp_add<0x4E>(dpp_add<0xB1>(sum));
            }
            if (ok && j0 == 0) lds.xc[mr][c] = make_float2(-corr, sum);
        }
    }
    // LDS-only barrier: __syncthreads() would also wait for every
    // outstanding weight load (its release fence waits on vmcnt(0)).
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    u32x4 xq[MR][CPL][4];
    float2 xc[MR][CPL];
#pragma unroll
    for (int mr = 0; mr < MR; ++mr)
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = kl + i * L;
#pragma unroll
            for (int j = 0; j < 4; ++j) xq[mr][i][j] = lds.xs[mr][j][c];
            xc[mr][i] = lds.xc[mr][c];
        }
    // Keep these LDS reads here, before the first wait for weights: left to
    // itself the compiler sinks each one to its use (fewer VGPRs, 36 instead of
    // 99 for gate/up), which puts an LDS round trip per chunk after the data
    // arrive.  Measured: gate/up 6.74-6.79 -> 6.67 us, q|k|v + rms_norm
    // 3.82-3.86 -> 3.73 us.
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (MULTI) {
        for (int t = 0; t < T; t += 2) {
            if (t + 1 < T) gemv_load<L, CPL, NW, MR>(sb, p, row0 + (t + 1) * RPI, kl);
            gemv_compute_store<L, CPL, NW, MR>(sa, xq, xc, p, row0 + t * RPI, kl);
            if (t + 2 < T) gemv_load<L, CPL, NW, MR>(sa, p, row0 + (t + 2) * RPI, kl);
            if (t + 1 < T)
                gemv_compute_store<L, CPL, NW, MR>(sb, xq, xc, p, row0 + (t + 1) * RPI, kl);
        }
    } else {
        gemv_compute_store<L, CPL, NW, MR>(sa, xq, xc, p, row0, kl);
    }
}

// Generic fallback for K that no (L, CPL) specialisation covers (K % 32 == 0,
// any size): one wave per row.  x is prepared in LDS kGenSeg chunks at a time
// and each lane visits its chunks (lane, lane + 64, ...) in increasing order
// across the segments, so any K fits in a fixed 36 KB.
constexpr int kGenSeg = 512;   // a multiple of 64

template <bool SWIGLU>
__global__ __launch_bounds__(256) void q4_gemv_generic_kernel(GemvParams p) {
    __shared__ u32x4 xs[4][kGenSeg];
    __shared__ float2 xcv[kGenSeg];
    __shared__ float red[4];
    const int nch = p.K / 32;
    // Input element i: x, or the (rounded) residual x + xb; rms_norm applied
    // when the prologue asks for it (same formulas as the specialized kernel).
    auto in_val = [&](int i) {
        float v = h2f(p.x[i]);
        if (p.pro == kProResidualRms) v = h2f(f2h(v + h2f(p.xb[i])));
        return v;
    };
    float rms = 0.0f;
    if (p.pro != kProNone) {
        float ss = 0.0f;
        for (int i = threadIdx.x; i < p.K; i += blockDim.x) {
            float v = h2f(p.x[i]);
            if (p.pro == kProResidualRms) {
                v += h2f(p.xb[i]);
                if (blockIdx.x == 0) p.res_out[i] = f2h(v);
            }
            ss += v * v;
        }
        ss = row_reduce<64>(ss);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        rms = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)p.K + p.eps);
    }
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    const bool row_ok = r < p.N;   // wave-uniform; every wave still takes the barriers
    constexpr int NW = SWIGLU ? 2 : 1;
    float a[NW];
#pragma unroll
    for (int m = 0; m < NW; ++m) a[m] = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += kGenSeg) {
        const int cn = min(kGenSeg, nch - c0);
        if (c0 > 0) __syncthreads();   // the previous segment has been read
        for (int cl = threadIdx.x; cl < cn; cl += blockDim.x) {
            const int c = c0 + cl;
            const f16x8* xp = reinterpret_cast<const f16x8*>(p.x + (size_t)c * 32);
            float corr = 0.0f, sum = 0.0f;
            for (int j = 0; j < 4; ++j) {
                uint32_t pr[4];
                f16x8 xv = xp[j];
                if (p.pro != kProNone)
                    for (int e = 0; e < 8; ++e) {
                        const int i = c * 32 + j * 8 + e;
                        xv[e] = (f16)(in_val(i) * rms * p.norm_w[i]);
                    }
                pair_word(xv, pr, corr, sum);
                u32x4 v = {pr[0], pr[1], pr[2], pr[3]};
                xs[j][cl] = v;
            }
            xcv[cl] = make_float2(-corr, sum);
        }
        __syncthreads();
        if (row_ok) {
#pragma unroll
            for (int m = 0; m < NW; ++m) {
                const u32x4* W = reinterpret_cast<const u32x4*>(m == 0 ? p.w0 : p.w1);
                const uint16_t* S = m == 0 ? p.s0 : p.s1;
                const uint16_t* B = m == 0 ? p.b0 : p.b1;
                for (int cl = lane; cl < cn; cl += 64) {
                    const int c = c0 + cl;
                    u32x4 xq[4];
                    for (int j = 0; j < 4; ++j) xq[j] = xs[j][cl];
                    const float2 xc = xcv[cl];
                    const float d = chunk_dot(W[(size_t)r * nch + c], xq, xc.x);
                    const size_t gi = (size_t)r * p.groups + (c >> p.gshift);
                    a[m] = fmaf(h2f(S[gi]), d, a[m]);
                    a[m] = fmaf(h2f(B[gi]), xc.y, a[m]);
                }
            }
        }
    }
    if (!row_ok) return;
    float acc[NW];
#pragma unroll
    for (int m = 0; m < NW; ++m) acc[m] = row_reduce<64>(a[m]);
    if (lane == 0) {
        float out = SWIGLU ? glu_f32(p.gelu, acc[0], acc[NW - 1]) : acc[0];
        p.y[r] = p.residual ? residual_add_f16(p.residual[r], out) : f2h(out);
    }
}

// ----------------------------------------------------------------- dispatch --

// Waves per block: about one block per CU, 4 to max_w waves.  The input
// vector is prepared once per block, so fewer, larger blocks prepare fewer
// copies of it; balanced blocks keep every CU's share equal.  Measured on the
// decode-layer launches (us, vs 4-wave blocks): down 4.55 vs 4.79 (12 waves),
// q|k|v 3.78 vs 4.00 (10), q|k|v with the rms_norm prologue 4.31 vs 5.68
// (10), gate/up 7.03 vs 7.29 (8), gate/up with residual + rms_norm 8.47 vs
// 9.03 (8).
static int gemv_block_waves(long waves, int max_w) {
    long w = (waves + kCUs - 1) / kCUs;
    return (int)(w < 4 ? 4 : w > max_w ? max_w : w);
}

template <int L, int CPL, bool SWIGLU>
static hipError_t launch_lc(const GemvParams& p, hipStream_t st) {
    constexpr int RPI = 64 / L;
    // Row-iterations per wave: one (every block resident at once, all weight
    // loads in flight from the start) until single-iteration waves would
    // exceed ~4096, then up to 8 to amortise the per-block x preparation on
    // tall matrices (the vocabulary head).  A norm prologue makes that
    // preparation dearer, so those launches switch to two iterations from
    // ~2048 waves.  Measured: plain gate/up (4096 iterations) 7.67 us at
    // T = 2 vs 7.27 us at T = 1, the fused-norm decode layer 22.5 us at T = 2
    // vs 23.4 us at T = 1; the 128256-row head is fastest at T = 8.
    const long iters = (p.N + RPI - 1) / RPI;
    long T = iters / (p.pro != kProNone ? 2048 : 4096);
    if (T < 1) T = 1;
    if (T > 8) T = 8;
    const long waves = (iters + T - 1) / T;
    // Prologues instantiated: rms_norm for the plain GEMV (q|k|v after
    // input_layernorm), residual + rms_norm for the fused gate/up.
    constexpr int PRO_N = SWIGLU ? kProResidualRms : kProRms;
    const bool norm = p.pro != kProNone;
    const int wpb = gemv_block_waves(waves, T > 1 ? gemv_max_waves<CPL, SWIGLU, true>()
                                                   : gemv_max_waves<CPL, SWIGLU, false>());
    const dim3 grid((unsigned)((waves + wpb - 1) / wpb)), block(64 * wpb);
    if (p.rows == 2) {   // two x rows: one weight set, one iteration, no prologue (gemv2_ok)
        if constexpr (CPL <= 4 && !SWIGLU) {
            if (T > 1 || norm) return hipErrorInvalidValue;
            const int wpb2 = gemv_block_waves(waves, gemv_max_waves<CPL, SWIGLU, false, 2>());
            hipLaunchKernelGGL((q4_gemv_kernel<L, CPL, SWIGLU, false, kProNone, 2>),
                               dim3((unsigned)((waves + wpb2 - 1) / wpb2)), dim3(64 * wpb2), 0,
                               st, p, 1);
            return hipGetLastError();
        }
        return hipErrorInvalidValue;
    }
    if (T > 1 && norm)
        hipLaunchKernelGGL((q4_gemv_kernel<L, CPL, SWIGLU, true, PRO_N, 1>), grid, block, 0, st, p, (int)T);
    else if (T > 1)
        hipLaunchKernelGGL((q4_gemv_kernel<L, CPL, SWIGLU, true, kProNone, 1>), grid, block, 0, st, p, (int)T);
    else if (norm)
        hipLaunchKernelGGL((q4_gemv_kernel<L, CPL, SWIGLU, false, PRO_N, 1>), grid, block, 0, st, p, 1);
    else
        hipLaunchKernelGGL((q4_gemv_kernel<L, CPL, SWIGLU, false, kProNone, 1>), grid, block, 0, st, p, 1);
    return hipGetLastError();
}

template <int L, bool SWIGLU>
static hipError_t launch_l(const GemvParams& p, int cpl, hipStream_t st) {
    switch (cpl) {
        case 1: return launch_lc<L, 1, SWIGLU>(p, st);
        case 2: return launch_lc<L, 2, SWIGLU>(p, st);
        case 3: return launch_lc<L, 3, SWIGLU>(p, st);
        case 4: return launch_lc<L, 4, SWIGLU>(p, st);
        case 5: return launch_lc<L, 5, SWIGLU>(p, st);
        case 6: return launch_lc<L, 6, SWIGLU>(p, st);
        case 7: return launch_lc<L, 7, SWIGLU>(p, st);
        case 8: return launch_lc<L, 8, SWIGLU>(p, st);
    }
    return hipErrorInvalidValue;
}

// Pick the widest L (lanes per row) that divides the chunk count with at most
// 8 chunks per lane.  Returns 0 when no specialisation applies.
int gemv_pick_lanes(int K, int* cpl_out) {
    const int nch = K / 32;
    const int lanes[3] = {64, 32, 16};
    for (int i = 0; i < 3; ++i) {
        const int L = lanes[i];
        if (nch % L == 0 && nch / L >= 1 && nch / L <= 8) {
            *cpl_out = nch / L;
            return L;
        }
    }
    return 0;
}

// Two x rows (p.rows == 2) of one weight set run where a specialised
// (L, CPL) kernel covers K with at most 4 chunks per lane (both rows' x pairs
// stay in registers) in one row-iteration per wave, with no prologue.
bool gemv2_ok(int N, int K) {
    int cpl = 0;
    const int L = gemv_pick_lanes(K, &cpl);
    return L != 0 && cpl <= 4 && (N + 64 / L - 1) / (64 / L) < 8192;
}

hipError_t launch_gemv(const GemvParams& p, bool swiglu, hipStream_t st) {
    if (p.pro != kProNone && p.pro != (swiglu ? kProResidualRms : kProRms)) return hipErrorInvalidValue;
    if (p.rows == 2 && (swiglu || p.pro != kProNone || !gemv2_ok(p.N, p.K)))
        return hipErrorInvalidValue;
    int cpl = 0;
    const int L = gemv_pick_lanes(p.K, &cpl);
    if (L == 64) return swiglu ? launch_l<64, true>(p, cpl, st) : launch_l<64, false>(p, cpl, st);
    if (L == 32) return swiglu ? launch_l<32, true>(p, cpl, st) : launch_l<32, false>(p, cpl, st);
    if (L == 16) return swiglu ? launch_l<16, true>(p, cpl, st) : launch_l<16, false>(p, cpl, st);
    const int grid = (p.N + 3) / 4;
    if (swiglu)
        hipLaunchKernelGGL(q4_gemv_generic_kernel<true>, dim3(grid), dim3(256), 0, st, p);
    else
        hipLaunchKernelGGL(q4_gemv_generic_kernel<false>, dim3(grid), dim3(256), 0, st, p);
    return hipGetLastError();
}

}  // namespace sltx
