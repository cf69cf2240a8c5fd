// q4_decode.hip -- one Llama decode layer's projections after attention, in
// a single launch (gfx950).
//
// The reference encodes a token's ~200 dispatches into one Metal command
// buffer with a memory barrier between dependent ones (MetalContext.swift:
// 109-134; transformerBlock, LlamaModel.swift:284-332).  Here the four
// dependent GEMVs of a layer that follow attention, and the next layer's
// input norm + q|k|v, run as phases of one kernel:
//   O  o = half(attn . Wo^T)                                 LlamaModel.swift:324-325
//   G  h1 = half(h + o); n = rms_norm(h1) with the sum of     :326 (residualRmsNorm,
//      squares over the unrounded h + o;                          Kernels.swift:238-290)
//      act = half(silu(n . Wg^T) * (n . Wu^T))                :327-329 (silu_mul, :90-98)
//   D  d = half(act . Wd^T); h2 = half(h1 + d) -> h_out       :330-331
//   Q  (next layer) q|k|v = half(rms_norm(h2) . Wqkv^T)       :288-292, rms_norm :40-86
// with the numerics of the separate entry points (fp32 accumulation, the
// reference's fp16 rounding points).
//
// Structure.  One block per CU (all resident at once: the grid is the CU
// count and the launcher checks the occupancy), 7 compute waves and one sync
// wave.  Each phase's rows are spread over all compute waves.  A phase's
// weight loads are issued as soon as the previous phase's rows are stored,
// behind the first poll of that exchange, so the exchange overlaps them.
// A phase's outputs are exchanged through device memory as 32-bit words
// (fp16 value | 16-bit tag << 16) stored with agent-scope (sc1) stores.  The
// sync wave, which has no weight loads in flight (vmcnt retires in issue
// order, so a poll behind them would wait for them), polls the whole vector
// with sc1 buffer loads until every word carries this launch's tag, and
// copies the values to LDS for the block.  No fence or atomic counter is
// involved: a value and its tag arrive together.  Tags are 3 * epoch +
// phase + 1 with the epoch (mod 21845) kept in the workspace and advanced by
// block 0 once it has consumed the last exchange (by then every block has
// read the epoch), so a stale word from an earlier launch never matches.
// Every wait is bounded (spin_limit polls); a wait that runs out adds one to
// the workspace's fault counter and the kernel finishes normally.
#include "q4_common.hpp"
#include "q4_gemv_ops.hpp"
#include "q4_launch.hpp"

namespace sltx {
namespace {

// 7 compute waves + the sync wave = 2 waves per SIMD, which leaves each wave
// 256 VGPRs: room for the weights of two phases in flight without spilling
// (a spilled load result must be waited for, and loads return in order).
constexpr int kCW = 7;                      // compute waves per block
constexpr int kThreads = 64 * (kCW + 1);    // + one sync wave
constexpr int kSc1 = 16;                    // buffer cache policy: sc1 (agent-coherent)
constexpr int kRsrcWord3 = 0x00020000;      // raw buffer resource, 32-bit data
constexpr uint32_t kEpochs = 21845;         // 3 * 21845 = 65535 tags

// Lanes per row and chunks per lane for rows of K nibbles (the GEMV's rule:
// the widest of 64, 32, 16 lanes that divides K / 32 with at most 8 chunks).
template <int K>
struct Lanes {
    static constexpr int nch = K / 32;
    static constexpr int L = (nch % 64 == 0 && nch / 64 <= 8) ? 64
                             : (nch % 32 == 0 && nch / 32 <= 8) ? 32 : 16;
    static constexpr int CPL = nch / L;
    static constexpr int RPI = 64 / L;   // rows per wave-wide load
    static_assert(nch % L == 0 && CPL >= 1 && CPL <= 8, "unsupported K");
};

struct Mat {
    const uint32_t* w;
    const uint16_t* s;
    const uint16_t* b;
};

// T row-iterations of prefetched operands for one lane: the weight chunks,
// and 8 bytes of the iteration's scales and biases.  The scales of the RPI
// rows of an iteration are contiguous (rows are), as are their biases; lane l
// loads halves 4l .. 4l+3 of [scales | biases] of those rows, one load per
// iteration instead of two 16-bit loads per chunk (which would also exceed
// the 63 loads the wait counter can track), and the values are shared through
// LDS when the iteration is computed.
template <int CPL, int NW, int T>
struct Pref {
    u32x4 w[T][NW][CPL];
    uint2 sb[T][NW];
};

template <int H, int F>
struct DlLds {
    static constexpr int NCH = (F > H ? F : H) / 32;
    u32x4 xs[4][NCH];              // prepared x, chunk-planar (the GEMV's layout)
    float2 xc[NCH];                // (-corr, sum) per chunk
    u32x4 tagged[(F > H ? F : H) / 4];   // the exchanged vector (o, act or d), tagged words
    uint16_t hres[H];              // residual stream in, then h1
    float nw0[H];                  // post-attention norm weight
    float nw1[H];                  // next layer's input norm weight
    float red[kCW + 1];
    uint2 sb[kCW][64];             // per-wave scale / bias staging
};

// Orders issue only: every wave of the block has issued what precedes it.
__device__ __forceinline__ void issue_barrier() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ void lds_barrier() {
    // LDS-only: __syncthreads() would also wait for every weight load in flight
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Loads of row-iterations TB .. TE-1 of T (iteration it = gw + t * GW covers
// rows it * RPI .. +RPI-1), iterations clamped to the last one so every load
// is unconditional and in bounds (clamped iterations are computed and
// discarded; N % RPI == 0).
template <int K, int NW, int T, int TB = 0, int TE = T>
__device__ __forceinline__ void pref_load(Pref<Lanes<K>::CPL, NW, T>& st, const Mat* m, int N,
                                          int groups, int gshift, int gw, int GW, int lane) {
    using LC = Lanes<K>;
    const int kl = lane % LC::L, sub = lane / LC::L;
    const int sbh = LC::RPI * groups;   // scale (and bias) halves of one iteration
#pragma unroll
    for (int t = TB; t < TE; ++t) {
        // clamp the iteration (not the row): its RPI rows stay consecutive and
        // inside [0, N), so the scale / bias load below stays in bounds
        const int it = min(gw + t * GW, N / LC::RPI - 1);
        const int r0 = it * LC::RPI;                 // the iteration's first row
        const int rr = r0 + sub;
        const int l = lane < sbh / 2 ? lane : 0;     // lanes past [scales | biases] repeat lane 0
        const int hoff = 4 * l < sbh ? r0 * groups + 4 * l : r0 * groups + 4 * l - sbh;
#pragma unroll
        for (int q = 0; q < NW; ++q) {
            const u32x4* W = reinterpret_cast<const u32x4*>(m[q].w);
#pragma unroll
            for (int i = 0; i < LC::CPL; ++i) {
                // 32-bit element offsets (every matrix here is far below 4 GB)
                const int c = kl + i * LC::L;
                st.w[t][q][i] = __builtin_nontemporal_load(&W[(uint32_t)(rr * LC::nch + c)]);
            }
            const uint16_t* src = 4 * l < sbh ? m[q].s : m[q].b;
            st.sb[t][q] = *reinterpret_cast<const uint2*>(src + (uint32_t)hoff);
        }
    }
}

// The prepared x a lane needs for its chunks (kl, kl + L, ...), read from LDS
// once per phase and held in registers for every row-iteration and weight
// set (re-reading it per iteration would make the phase LDS-bound).
template <int K>
struct XFrag {
    u32x4 q[Lanes<K>::CPL][4];
    float2 c[Lanes<K>::CPL];
};

template <int K, int NCH>
__device__ __forceinline__ void load_xfrag(XFrag<K>& x, const u32x4 (&xs)[4][NCH], const float2* xc,
                                           int lane) {
    using LC = Lanes<K>;
    const int kl = lane % LC::L;
#pragma unroll
    for (int i = 0; i < LC::CPL; ++i) {
        const int c = kl + i * LC::L;
#pragma unroll
        for (int j = 0; j < 4; ++j) x.q[i][j] = xs[j][c];
        x.c[i] = xc[c];
    }
}

// Dot products of prefetched row-iterations TB .. TE-1 with the prepared x;
// epi(row, acc) runs in lane 0 of each row for rows that exist.  The
// iteration's scales and biases go through the wave's staging area.
template <int K, int NW, int T, int TB, int TE, class Epi>
__device__ __forceinline__ void pref_compute(const Pref<Lanes<K>::CPL, NW, T>& st, const XFrag<K>& x,
                                             uint2* sbw, int N, int groups, int gshift, int gw,
                                             int GW, int lane, Epi epi) {
    using LC = Lanes<K>;
    const int kl = lane % LC::L, sub = lane / LC::L;
    const uint16_t* sb16 = reinterpret_cast<const uint16_t*>(sbw);
    const int sbh = LC::RPI * groups;
#pragma unroll
    for (int t = TB; t < TE; ++t) {
        const int row = (gw + t * GW) * LC::RPI + sub;
        float acc[NW];
#pragma unroll
        for (int q = 0; q < NW; ++q) {
            sbw[lane] = st.sb[t][q];   // wave-local: LDS ops of one wave complete in order
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < LC::CPL; ++i) {
                const int c = kl + i * LC::L;
                const int gi = sub * groups + (c >> gshift);
                const float d = chunk_dot(st.w[t][q][i], x.q[i], x.c[i].x);
                a = fmaf(h2f(sb16[gi]), d, a);
                a = fmaf(h2f(sb16[sbh + gi]), x.c[i].y, a);
            }
            acc[q] = row_reduce<LC::L>(a);
        }
        if (kl == 0 && row < N) epi(row, acc);
    }
}

// Prepares the K-value input (8-value word wi = tid + kThreads * u given by
// word(wi)) into xs / xc.  K / 8 is a multiple of 64, so a wave is either
// wholly inside the vector or skips the unit; the four words of a chunk sit
// in one lane quad, which sums the chunk's (corr, sum) by DPP.
template <int K, int NCH, class Word>
__device__ __forceinline__ void prep_x(u32x4 (&xs)[4][NCH], float2* xc, int tid, Word word) {
    constexpr int NWD = K / 8;
    static_assert(NWD % 64 == 0, "K must be a multiple of 512");
    constexpr int U = (NWD + kThreads - 1) / kThreads;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if ((tid & ~63) + kThreads * u >= NWD) continue;   // wave-uniform
        const int wi = tid + kThreads * u;
        uint32_t pr[4];
        float corr = 0.0f, sum = 0.0f;
        pair_word(word(wi, u), pr, corr, sum);
        const int c = wi >> 2, j = wi & 3;
        xs[j][c] = u32x4{pr[0], pr[1], pr[2], pr[3]};
        corr = dpp_add<0x4E>(dpp_add<0xB1>(corr));
        sum = dpp_add<0x4E>(dpp_add<0xB1>(sum));
        if (j == 0) xc[c] = make_float2(-corr, sum);
    }
}

// Sum of v over the block, identical (same order) in every block.
__device__ __forceinline__ float block_sum(float v, float* red, int tid) {
    v = row_reduce<64>(v);
    if ((tid & 63) == 0) red[tid >> 6] = v;
    lds_barrier();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w <= kCW; ++w) s += red[w];
    return s;
}

__device__ __forceinline__ void put_word(uint32_t* dst, float v, uint32_t tag) {
    __hip_atomic_store(dst, (uint32_t)f2h(v) | (tag << 16), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Sync wave: copies the NW tagged words of buf into LDS with direct-to-LDS
// sc1 buffer loads (all in flight at once, no data registers, one address
// register).  poll_issue only enqueues the copies; poll_finish waits for them
// and re-polls until every word carries `tag` (false if spin_limit polls ran
// out).  The split lets the compute waves queue the next phase's weight loads
// behind the first poll: a CU returns vector loads in order, so the poll then
// costs no more than waiting for those weights would.
template <int NW>
__device__ __forceinline__ void poll_issue(const uint32_t* buf, u32x4* dst, int lane) {
    static_assert(NW % 256 == 0, "exchanged vectors are multiples of 256 words");
    const auto rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(buf), (short)0,
                                                        NW * 4, kRsrcWord3);
#pragma unroll
    for (int i = 0; i < NW / 256; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr_t)(dst + 64 * i), 16, lane * 16,
                                                 i * 1024, 0, kSc1);
}

template <int NW>
__device__ __forceinline__ bool poll_finish(const uint32_t* buf, uint32_t tag, u32x4* dst, int lane,
                                            int spin_limit) {
    for (int n = 0; n < spin_limit; ++n) {
        // vmcnt(0) only (gfx9 encoding: expcnt and lgkmcnt left at their maxima)
        __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8));
        bool ok = true;
#pragma unroll
        for (int i = 0; i < NW / 256; ++i) {
            const u32x4 v = dst[lane + 64 * i];
            ok = ok && (v.x >> 16) == tag && (v.y >> 16) == tag && (v.z >> 16) == tag &&
                 (v.w >> 16) == tag;
        }
        if (__builtin_amdgcn_ballot_w64(!ok) == 0) return true;
        poll_issue<NW>(buf, dst, lane);
    }
    return false;
}

// The 8 fp16 values of word wi of a tagged vector in LDS.
__device__ __forceinline__ f16x8 tagged_word(const u32x4* t, int wi) {
    const u32x4 a = t[2 * wi], b = t[2 * wi + 1];
    const uint32_t w[4] = {(a.x & 0xFFFFu) | (a.y << 16), (a.z & 0xFFFFu) | (a.w << 16),
                           (b.x & 0xFFFFu) | (b.y << 16), (b.z & 0xFFFFu) | (b.w << 16)};
    return __builtin_bit_cast(f16x8, w);
}

__device__ __forceinline__ void count_fault(uint32_t* sync, int lane) {
    if (lane == 0)
        __hip_atomic_fetch_add(sync + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- the two roles.  Both run the same sequence of block barriers; the
// steps every wave takes part in (x preparation, norms) are shared helpers.

// Residual stream and norm weights into LDS; the attention output prepared as
// O's x.  Prologue values were loaded by every thread (index clamped).
template <int H, int F, bool NEXT>
__device__ __forceinline__ void stage_inputs(DlLds<H, F>& lds, int tid, const f16x8& xin,
                                             const f16x8& hin, const f32x4 (&n0)[2],
                                             const f32x4 (&n1)[2]) {
    if (tid < H / 8) {
        reinterpret_cast<f16x8*>(lds.hres)[tid] = hin;
        reinterpret_cast<f32x4*>(lds.nw0)[2 * tid] = n0[0];
        reinterpret_cast<f32x4*>(lds.nw0)[2 * tid + 1] = n0[1];
        if (NEXT) {
            reinterpret_cast<f32x4*>(lds.nw1)[2 * tid] = n1[0];
            reinterpret_cast<f32x4*>(lds.nw1)[2 * tid + 1] = n1[1];
        }
    }
    prep_x<H>(lds.xs, lds.xc, tid, [&](int, int) { return xin; });
}

// h1 = half(h + o) into hres; rms over the unrounded sum; G's x.
template <int H, int F>
__device__ __forceinline__ void prep_g(DlLds<H, F>& lds, int tid, float eps) {
    f16x8 hv{};
    float ss = 0.0f;
    if (tid < H / 8) {
        const f16x8 a = reinterpret_cast<const f16x8*>(lds.hres)[tid];
        const f16x8 b = tagged_word(lds.tagged, tid);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float v = (float)a[e] + (float)b[e];
            ss += v * v;
            hv[e] = (f16)v;
        }
        reinterpret_cast<f16x8*>(lds.hres)[tid] = hv;
    }
    const float rms = rsqrtf(block_sum(ss, lds.red, tid) / (float)H + eps);
    prep_x<H>(lds.xs, lds.xc, tid, [&](int, int) {
        f16x8 n;
#pragma unroll
        for (int e = 0; e < 8; ++e) n[e] = (f16)((float)hv[e] * rms * lds.nw0[8 * tid + e]);
        return n;
    });
}

// D's x: the activation (K = F).
template <int H, int F>
__device__ __forceinline__ void prep_d(DlLds<H, F>& lds, int tid) {
    prep_x<F>(lds.xs, lds.xc, tid, [&](int wi, int) { return tagged_word(lds.tagged, wi); });
}

// h2 = half(h1 + d) (block 0 stores it as the residual stream out); rms over
// the stored h2; Q's x.
template <int H, int F>
__device__ __forceinline__ void prep_q(DlLds<H, F>& lds, int tid, float eps, uint16_t* h_out) {
    f16x8 hv{};
    float ss = 0.0f;
    if (tid < H / 8) {
        const f16x8 a = reinterpret_cast<const f16x8*>(lds.hres)[tid];
        const f16x8 d = tagged_word(lds.tagged, tid);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            hv[e] = (f16)((float)a[e] + (float)d[e]);
            ss += (float)hv[e] * (float)hv[e];
        }
        if (blockIdx.x == 0) reinterpret_cast<f16x8*>(h_out)[tid] = hv;
    }
    const float rms = rsqrtf(block_sum(ss, lds.red, tid) / (float)H + eps);
    prep_x<H>(lds.xs, lds.xc, tid, [&](int, int) {
        f16x8 n;
#pragma unroll
        for (int e = 0; e < 8; ++e) n[e] = (f16)((float)hv[e] * rms * lds.nw1[8 * tid + e]);
        return n;
    });
}

// Prologue loads (every thread; threads past the vector re-read word 0).
template <int H, bool NEXT>
__device__ __forceinline__ void load_inputs(const DecodeLayerParams& p, int tid, f16x8& xin,
                                            f16x8& hin, f32x4 (&n0)[2], f32x4 (&n1)[2]) {
    const int w = tid < H / 8 ? tid : 0;
    xin = reinterpret_cast<const f16x8*>(p.attn)[w];
    hin = reinterpret_cast<const f16x8*>(p.h)[w];
    n0[0] = reinterpret_cast<const f32x4*>(p.post_norm)[2 * w];
    n0[1] = reinterpret_cast<const f32x4*>(p.post_norm)[2 * w + 1];
    if (NEXT) {
        n1[0] = reinterpret_cast<const f32x4*>(p.next_norm)[2 * w];
        n1[1] = reinterpret_cast<const f32x4*>(p.next_norm)[2 * w + 1];
    }
}

template <int H, int F, int TO, int TG, int TD, int TQ, bool NEXT>
__device__ __forceinline__ void compute_role(const DecodeLayerParams& p, DlLds<H, F>& lds,
                                             uint32_t* lds_epoch, int tid) {
    using LH = Lanes<H>;
    using LF = Lanes<F>;
    const int lane = tid & 63, wave = tid >> 6;
    const int G = gridDim.x, GW = G * kCW;
    const int gw = wave * G + blockIdx.x;   // compute wave index (wave-major)
    uint2* sbw = lds.sb[wave];

    // The inputs and the o weights first; each later phase's weights are
    // issued right after the previous phase's rows are stored.  A CU holds
    // only some tens of KB of loads in flight and returns them in order, so a
    // wave issuing a large prefetch stalls until earlier loads return (issued
    // earlier, the prefetch would delay the phase computed in between), and a
    // poll queued behind a prefetch waits for it.  The exchange's first poll
    // is queued after the phase's first row-iteration: about a microsecond of
    // weights, by which time every block has stored its rows (a poll that
    // finds a row missing is queued again behind the rest of the phase).
    f16x8 xin, hin;
    f32x4 n0[2], n1[2];
    load_inputs<H, NEXT>(p, tid, xin, hin, n0, n1);
    const Mat mo[1] = {{p.wo, p.so, p.bo}};
    const Mat mg[2] = {{p.wg, p.sg, p.bg}, {p.wu, p.su, p.bu}};
    const Mat md[1] = {{p.wd, p.sd, p.bd}};
    const Mat mq[1] = {{p.wq, p.sq, p.bq}};
    Pref<LH::CPL, 1, TO> po;
    Pref<LH::CPL, 2, TG> pg;
    Pref<LF::CPL, 1, TD> pd;
    Pref<LH::CPL, 1, TQ> pq;
    pref_load<H, 1, TO>(po, mo, H, p.groups_h, p.gshift, gw, GW, lane);
    __builtin_amdgcn_sched_barrier(0);
    stage_inputs<H, F, NEXT>(lds, tid, xin, hin, n0, n1);               // waits for the inputs only
    lds_barrier();                                                     // B1
    const uint32_t epoch = *lds_epoch;
    const uint32_t tag_o = 3 * epoch + 1, tag_a = 3 * epoch + 2, tag_d = 3 * epoch + 3;

    // O: o rows out as tagged words
    XFrag<H> xh;
    load_xfrag<H>(xh, lds.xs, lds.xc, lane);
    pref_compute<H, 1, TO, 0, TO>(po, xh, sbw, H, p.groups_h, p.gshift, gw, GW, lane,
                                  [&](int r, const float* acc) { put_word(p.xo + r, acc[0], tag_o); });
    lds_barrier();                                                     // B2: o rows stored
    pref_load<H, 2, TG, 0, 1>(pg, mg, F, p.groups_h, p.gshift, gw, GW, lane);
    issue_barrier();                                                   // B2b: o poll queued next
    pref_load<H, 2, TG, 1, TG>(pg, mg, F, p.groups_h, p.gshift, gw, GW, lane);
    lds_barrier();                                                     // B3: o in LDS
    prep_g(lds, tid, p.eps);                                           // (+1 barrier)
    lds_barrier();                                                     // B5

    // G: act rows out as tagged words
    load_xfrag<H>(xh, lds.xs, lds.xc, lane);
    pref_compute<H, 2, TG, 0, TG>(pg, xh, sbw, F, p.groups_h, p.gshift, gw, GW, lane,
                                  [&](int r, const float* acc) {
                                      put_word(p.xa + r, silu_mul_f32(acc[0], acc[1]), tag_a);
                                  });
    lds_barrier();                                                     // B6
    pref_load<F, 1, TD, 0, 1>(pd, md, H, p.groups_f, p.gshift, gw, GW, lane);
    issue_barrier();                                                   // B6b: act poll queued next
    pref_load<F, 1, TD, 1, TD>(pd, md, H, p.groups_f, p.gshift, gw, GW, lane);
    lds_barrier();                                                     // B7: act in LDS
    prep_d(lds, tid);
    lds_barrier();                                                     // B8

    // D: d rows out (tagged), or h_out = half(h1 + d) on the last layer
    XFrag<F> xf;
    load_xfrag<F>(xf, lds.xs, lds.xc, lane);
    pref_compute<F, 1, TD, 0, TD>(pd, xf, sbw, H, p.groups_f, p.gshift, gw, GW, lane,
                                  [&](int r, const float* acc) {
                                      if (NEXT) put_word(p.xd + r, acc[0], tag_d);
                                      else p.h_out[r] = residual_add_f16(lds.hres[r], acc[0]);
                                  });
    if (!NEXT) return;
    lds_barrier();                                                     // B9
    pref_load<H, 1, TQ, 0, 1>(pq, mq, p.nq, p.groups_h, p.gshift, gw, GW, lane);
    issue_barrier();                                                   // B9b: d poll queued next
    pref_load<H, 1, TQ, 1, TQ>(pq, mq, p.nq, p.groups_h, p.gshift, gw, GW, lane);
    lds_barrier();                                                     // B10: d in LDS
    prep_q(lds, tid, p.eps, p.h_out);                                  // (+1 barrier)
    lds_barrier();                                                     // B12

    // Q: the next layer's q|k|v
    load_xfrag<H>(xh, lds.xs, lds.xc, lane);
    pref_compute<H, 1, TQ, 0, TQ>(pq, xh, sbw, p.nq, p.groups_h, p.gshift, gw, GW, lane,
                                  [&](int r, const float* acc) { p.qkv_out[r] = f2h(acc[0]); });
}

template <int H, int F, bool NEXT>
__device__ __forceinline__ void sync_role(const DecodeLayerParams& p, DlLds<H, F>& lds,
                                          uint32_t* lds_epoch, int tid) {
    const int lane = tid & 63;
    f16x8 xin, hin;
    f32x4 n0[2], n1[2];
    load_inputs<H, NEXT>(p, tid, xin, hin, n0, n1);
    const uint32_t epoch = __hip_atomic_load(p.sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (lane == 0) *lds_epoch = epoch;
    stage_inputs<H, F, NEXT>(lds, tid, xin, hin, n0, n1);
    lds_barrier();                                                     // B1
    lds_barrier();                                                     // B2
    poll_issue<H>(p.xo, lds.tagged, lane);
    issue_barrier();                                                   // B2b
    if (!poll_finish<H>(p.xo, 3 * epoch + 1, lds.tagged, lane, p.spin_limit)) count_fault(p.sync, lane);
    lds_barrier();                                                     // B3
    prep_g(lds, tid, p.eps);
    lds_barrier();                                                     // B5
    lds_barrier();                                                     // B6
    poll_issue<F>(p.xa, lds.tagged, lane);
    issue_barrier();                                                   // B6b
    if (!poll_finish<F>(p.xa, 3 * epoch + 2, lds.tagged, lane, p.spin_limit)) count_fault(p.sync, lane);
    // the last exchange of a layer without Q: every block has read the epoch
    if (!NEXT && blockIdx.x == 0 && lane == 0)
        __hip_atomic_store(p.sync, (epoch + 1) % kEpochs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    lds_barrier();                                                     // B7
    prep_d(lds, tid);
    lds_barrier();                                                     // B8
    if (!NEXT) return;
    lds_barrier();                                                     // B9
    poll_issue<H>(p.xd, lds.tagged, lane);
    issue_barrier();                                                   // B9b
    if (!poll_finish<H>(p.xd, 3 * epoch + 3, lds.tagged, lane, p.spin_limit)) count_fault(p.sync, lane);
    if (blockIdx.x == 0 && lane == 0)
        __hip_atomic_store(p.sync, (epoch + 1) % kEpochs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    lds_barrier();                                                     // B10
    prep_q(lds, tid, p.eps, p.h_out);
    lds_barrier();                                                     // B12
}

template <int H, int F, int TO, int TG, int TD, int TQ, bool NEXT>
__global__ __launch_bounds__(kThreads) void q4_decode_layer_kernel(DecodeLayerParams p) {
    __shared__ DlLds<H, F> lds;
    __shared__ uint32_t lds_epoch;
    static_assert(H / 8 <= kThreads, "hidden vector: at most one word per thread");
    const int tid = threadIdx.x;
    if ((tid >> 6) == kCW) sync_role<H, F, NEXT>(p, lds, &lds_epoch, tid);
    else compute_role<H, F, TO, TG, TD, TQ, NEXT>(p, lds, &lds_epoch, tid);
}

// Row-iterations per compute wave for N rows of K columns on G blocks.
template <int K>
int iters_per_wave(int N, int G) {
    const long it = (N + Lanes<K>::RPI - 1) / Lanes<K>::RPI;
    const long gw = (long)G * kCW;
    return (int)((it + gw - 1) / gw);
}

template <int H, int F, int TO, int TG, int TD, int TQ>
hipError_t launch_cfg(const DecodeLayerParams& p, int G, hipStream_t st) {
    if (p.wq) {
        hipLaunchKernelGGL((q4_decode_layer_kernel<H, F, TO, TG, TD, TQ, true>), dim3(G),
                           dim3(kThreads), 0, st, p);
    } else {
        hipLaunchKernelGGL((q4_decode_layer_kernel<H, F, TO, TG, TD, TQ, false>), dim3(G),
                           dim3(kThreads), 0, st, p);
    }
    return hipGetLastError();
}

// One 8-byte scale / bias load per lane covers an iteration: RPI rows of
// groups halves each, twice, within 64 lanes and split at a lane boundary;
// the row count a whole number of iterations.
template <int K>
bool sb_fits(int groups, int N) {
    const int sbh = Lanes<K>::RPI * groups;
    return sbh % 4 == 0 && sbh <= 128 && N % Lanes<K>::RPI == 0;
}

template <int H, int F, int TO, int TG, int TD, int TQ>
bool fits(const DecodeLayerParams& p, int G) {
    return p.H == H && p.F == F && sb_fits<H>(p.groups_h, H) && sb_fits<H>(p.groups_h, F) &&
           sb_fits<F>(p.groups_f, H) && (!p.wq || sb_fits<H>(p.groups_h, p.nq)) &&
           iters_per_wave<H>(H, G) <= TO &&
           iters_per_wave<H>(F, G) <= TG && iters_per_wave<F>(H, G) <= TD &&
           (!p.wq || iters_per_wave<H>(p.nq, G) <= TQ);
}

template <int H, int F, int TO, int TG, int TD, int TQ>
int occupancy() {
    int a = 0, b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &a, reinterpret_cast<const void*>(q4_decode_layer_kernel<H, F, TO, TG, TD, TQ, true>),
            kThreads, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &b, reinterpret_cast<const void*>(q4_decode_layer_kernel<H, F, TO, TG, TD, TQ, false>),
            kThreads, 0) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return a < b ? a : b;
}

// Shapes built: Llama-3.2-3B (hidden 3072, FFN 8192) and Llama-3.2-1B
// (2048, 8192) on 256 CUs.
#define SLTX_DL_CONFIGS(X) \
    X(3072, 8192, 1, 3, 2, 2) \
    X(2048, 8192, 2, 5, 2, 2)

}  // namespace

size_t decode_layer_sync_bytes(int H, int F) {
    return 256 + (size_t)(2 * H + F) * 4;
}

int decode_layer_supported(const DecodeLayerParams& p, int G) {
#define X(h, f, a, b, c, d) if (fits<h, f, a, b, c, d>(p, G)) return 1;
    SLTX_DL_CONFIGS(X)
#undef X
    return 0;
}

int decode_layer_resident(const DecodeLayerParams& p, int G, int cus) {
#define X(h, f, a, b, c, d) \
    if (fits<h, f, a, b, c, d>(p, G)) return (long)occupancy<h, f, a, b, c, d>() * cus >= G;
    SLTX_DL_CONFIGS(X)
#undef X
    return 0;
}

hipError_t launch_decode_layer(const DecodeLayerParams& p, int G, hipStream_t st) {
#define X(h, f, a, b, c, d) if (fits<h, f, a, b, c, d>(p, G)) return launch_cfg<h, f, a, b, c, d>(p, G, st);
    SLTX_DL_CONFIGS(X)
#undef X
    return hipErrorInvalidValue;
}

}  // namespace sltx
