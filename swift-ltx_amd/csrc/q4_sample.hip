// q4_sample.hip -- token selection after the lm_head, on the GPU.
//
// argmax (Ops.swift:757-781) and temperature / top-p / repetition-penalty
// sampling (sample, Ops.swift:785-810; sampleFromLogits, Ops.swift:2060-2098),
// which the reference runs on the CPU over all vocabulary logits per token.
//
// The probabilities follow the reference's fp32 steps: penalty (divide
// positive, multiply non-positive logits of the distinct seen tokens), divide
// by temperature, softmax (max, exp, sum, divide).  The softmax denominator
// is a fixed-order sum: each block b forms m_b = the max of its logits and
// s_b = sum of exp(l - m_b) (each thread over its tokens in index order, then
// a halving tree over the block's 256 threads); sum = the terms
// s_b * exp(m_b - max) over four 64-term halving trees, combined as
// (w0 + w1) + (w2 + w3) -- an online softmax, so one pass over the logits
// yields both.
// The nucleus and the draw use exact running sums instead of the reference's
// sequential fp32 ones: each probability p carries the integer mass
// floor(p * 2^52), and in the order (p descending, id ascending; the
// reference's sort is unstable) the cutoff is the first token whose inclusive
// running mass reaches ceil(top_p * 2^52) (all tokens if none does), and the
// chosen token is the first whose inclusive running mass reaches
// ceil(u * mass at the cutoff) -- the reference's "r -= p until r <= 0".
//
// Nothing is sorted in HBM.  Tokens are ranked by the 56-bit key
// D = (bits of p) << 24 | (2^24 - 1 - id), descending, and both positions are
// weighted radix selects over D, 12 bits a level:
//   sample_scale    l = penalised logit / temperature (the block's seen ids
//                   marked in an LDS bitmap); block max and exp-sum; clears
//                   the level-0 histogram
//   sample_prob     p = exp(l - max) / sum; level-0 histogram (p bits
//                   31..20: count and mass per bin)
//   sample_gather   each block finds, from the histogram, the bin holding the
//                   cutoff and the bins the draw can reach, and compacts their
//                   tokens (no grid-wide fence or last-block hand-off: on a
//                   chip whose XCDs have separate L2s those cost more than
//                   re-reading the 48 KB histogram per block)
//   sample_select   one workgroup: up to 64 candidates are sorted in one
//                   wave's registers and scanned; more go through levels 1-4
//                   (in LDS when they fit), a level stopping once its bin
//                   holds a single token
#include <mutex>

#include "q4_common.hpp"
#include "q4_launch.hpp"

namespace sltx {
namespace {

constexpr int kGridThreads = 256;   // grid kernels: 4 consecutive tokens a thread per step
constexpr int kMaxBlocks = 256;
constexpr int kSelThreads = 1024;   // sample_select
constexpr int kBins = 4096;         // 12-bit digits
constexpr int kCandLds = 8192;      // candidates sample_select holds in LDS
constexpr int kSelUnroll = 8;     // candidates each select thread loads before using them
constexpr uint32_t kIdMask = 0xFFFFFFu;
// seen-id bitmap of one scale block: up to 64 quads a thread (n <= 2^24
// with 256 blocks of 256 threads), 4 bits a quad
constexpr int kSeenWords = 64 * 4 * kGridThreads / 32;

__device__ __forceinline__ float load_logit(const void* p, int dtype, int i) {
    if (dtype == kF32) return reinterpret_cast<const float*>(p)[i];
    return h2f(reinterpret_cast<const uint16_t*>(p)[i]);
}

// floor(p * 2^52) for a non-negative fp32 p given by its bits (0 below 2^-52;
// p = m * 2^(e-150), so p * 2^52 = m * 2^(e-98)).
__device__ __forceinline__ unsigned long long mass_of(uint32_t key) {
    const int e = (int)(key >> 23);
    if (e == 0) return 0ull;
    const unsigned long long m = (key & 0x7FFFFFu) | 0x800000u;
    const int sh = e - 98;
    if (sh >= 0) return m << (sh < 39 ? sh : 39);   // p >= 2 only for non-finite input
    return sh <= -24 ? 0ull : m >> -sh;
}

__device__ __forceinline__ unsigned long long order_key(uint32_t key, uint32_t id) {
    return ((unsigned long long)key << 24) | (kIdMask - id);
}

// Adds one token (key, mass m) to bin d of an LDS histogram for every lane
// with ok set; all 64 lanes of the wave call it.  When every such lane has the
// same bin (tied, uniform or non-finite logits), one lane adds the wave's
// count and mass sum -- same-address LDS atomics serialise.  Lanes with the
// same key have the same mass, so a wave of one key adds count * mass; a
// wave of one bin but several keys sums its masses across the wave.
// Otherwise each lane adds its own.  Returns the lane that added for the
// whole wave (-1: each lane added its own).  Masses are integers, so the
// sums are exact in any order.
__device__ __forceinline__ int hist_add(bool ok, int d, uint32_t key, unsigned long long m,
                                        uint32_t* cnt, unsigned long long* mass) {
    const unsigned long long act = __ballot(ok);
    if (!act) return -1;
    const int lane = threadIdx.x & 63;
    const int lead = __ffsll((long long)act) - 1;
    const int d0 = __builtin_amdgcn_readlane(d, lead);
    if (__ballot(ok && d == d0) != act) {
        if (ok) {
            atomicAdd(&cnt[d], 1u);
            if (m) atomicAdd(&mass[d], m);
        }
        return -1;
    }
    unsigned long long sum;
    const uint32_t k0 = (uint32_t)__builtin_amdgcn_readlane((int)key, lead);
    if (__ballot(ok && key == k0) == act) {
        const unsigned long long m0 =
            ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(m >> 32), lead) << 32) |
            (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)m, lead);
        sum = m0 * (unsigned long long)__popcll(act);
    } else {
        sum = ok ? m : 0ull;
        for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    }
    if (lane == lead) {
        atomicAdd(&cnt[d0], (uint32_t)__popcll(act));
        if (sum) atomicAdd(&mass[d0], sum);
    }
    return lead;
}

__device__ __forceinline__ uint32_t lanes_below(unsigned long long mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ unsigned long long target_top_p(float top_p) {
    return (unsigned long long)ceil(fmin((double)top_p, 4.0) * 0x1p52);
}

__device__ __forceinline__ unsigned long long target_draw(float u, unsigned long long cum) {
    return (unsigned long long)ceil((double)u * (double)cum);
}

// Seen-id count: the host argument, or the history length in device memory,
// clamped to [0, hist_cap].
__device__ __forceinline__ int seen_count(const SampleParams& p) {
    if (!p.hist_len) return p.n_seen;
    const int c = *p.hist_len;
    return c < 0 ? 0 : c > p.hist_cap ? p.hist_cap : c;
}

// Index of this call's draw in u_seq (u_next taken modulo u_count).
__device__ __forceinline__ int draw_index(const SampleParams& p) {
    const int i = *p.u_next % p.u_count;
    return i < 0 ? i + p.u_count : i;
}

// The uniform draw: the host argument, or u_seq[u_next] with values outside
// [0, 1) (and NaN) clamped into it.
__device__ __forceinline__ float draw_of(const SampleParams& p) {
    if (!p.u_seq) return p.u;
    const float u = p.u_seq[draw_index(p)];
    return u >= 0.0f ? (u < 1.0f ? u : 0x1.fffffep-1f) : 0.0f;
}

// One lane: store the chosen token and, with device state, append it to the
// history (dropped when full) and advance the draw index.
__device__ __forceinline__ void finish_select(const SampleParams& p, int id) {
    *p.out = id;
    if (p.hist_len) {
        const int c = seen_count(p);
        if (c < p.hist_cap) {
            p.hist[c] = id;
            *p.hist_len = c + 1;
        }
    }
    if (p.u_seq) *p.u_next = (draw_index(p) + 1) % p.u_count;
}

// Exclusive prefix sum over the block's threads (in thread order).
template <int NT>
__device__ unsigned long long block_excl_scan(unsigned long long v, unsigned long long* wsum) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    unsigned long long x = v;
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) wsum[wid] = x;
    __syncthreads();
    if (wid == 0) {
        unsigned long long w = lane < NT / 64 ? wsum[lane] : 0ull;
        for (int o = 1; o < NT / 64; o <<= 1) {
            const unsigned long long y = __shfl_up(w, o, 64);
            if (lane >= o) w += y;
        }
        if (lane < NT / 64) wsum[lane] = w;
    }
    __syncthreads();
    const unsigned long long r = x - v + (wid > 0 ? wsum[wid - 1] : 0ull);
    __syncthreads();
    return r;
}

struct BinSel {
    int found, bin;
    uint32_t cnt;
    unsigned long long excl, incl, total;
};

struct SelScratch {
    unsigned long long wsum[16];
    int best;
};

// kBins bins in descending bin order, after `above` mass, spread over the
// block (BPT consecutive bins a thread).  load() reads the bins and scans
// their masses; find(target) gives the highest non-empty bin whose inclusive
// running mass reaches target (found), its exclusive / inclusive mass and
// count, and the total.  Whole block; cnt and mass may be global or LDS.
// Both end synchronised.
template <int NT>
struct BinScan {
    static constexpr int BPT = kBins / NT;
    uint32_t c[BPT];
    unsigned long long m[BPT];
    unsigned long long excl, tot;
    int top;   // this thread's bins: top, top-1, ..., top-BPT+1

    __device__ void load(const uint32_t* cnt, const unsigned long long* mass,
                         unsigned long long above, SelScratch& sc) {
        top = kBins - 1 - (int)threadIdx.x * BPT;
        tot = 0ull;
#pragma unroll
        for (int k = 0; k < BPT; ++k) {
            c[k] = cnt[top - k];
            m[k] = mass[top - k];
            tot += m[k];
        }
        excl = above + block_excl_scan<NT>(tot, sc.wsum);
    }

    __device__ void find(unsigned long long target, BinSel& out, SelScratch& sc) {
        if (threadIdx.x == 0) sc.best = -1;
        __syncthreads();
        int best = -1;
        unsigned long long run = excl;
#pragma unroll
        for (int k = 0; k < BPT; ++k) {
            run += m[k];
            if (best < 0 && c[k] && run >= target) best = top - k;
        }
        if (best >= 0) atomicMax(&sc.best, best);
        __syncthreads();
        const int B = sc.best;
        if ((int)threadIdx.x == NT - 1) {
            out.total = excl + tot;
            out.found = B >= 0;
        }
        if (B >= 0 && B <= top && B > top - BPT) {
            unsigned long long e = excl, mb = 0ull;
            uint32_t cb = 0u;
#pragma unroll
            for (int k = 0; k < BPT; ++k) {
                if (k < top - B) e += m[k];
                if (k == top - B) {
                    mb = m[k];
                    cb = c[k];
                }
            }
            out.bin = B;
            out.excl = e;
            out.incl = e + mb;
            out.cnt = cb;
        }
        __syncthreads();
    }
};

struct LevelHist {
    uint32_t cnt[kBins];
    unsigned long long mass[kBins];
    uint32_t id[kBins];
};

// Levels 1-4 of the weighted select inside level-0 bin `bin` (exclusive mass
// `above`): the token whose inclusive running mass first reaches target.
// Whole block; returns the id (-1 only for non-finite input) and sets cum_out
// to its inclusive mass.
__device__ int select_in_bin(const uint2* cand, int C, int bin, unsigned long long above,
                             unsigned long long target, LevelHist& H, SelScratch& sc, BinSel& bs,
                             unsigned long long& cum_out) {
    const int tid = threadIdx.x;
    unsigned long long P = (unsigned long long)bin << 44;
    unsigned long long Mk = 0xFFFull << 44;
    for (int lev = 1; lev <= 4; ++lev) {
        const int shift = lev == 1 ? 32 : lev == 2 ? 20 : lev == 3 ? 8 : 0;
        const unsigned long long wmask = lev == 4 ? 0xFFull : 0xFFFull;
        for (int b = tid; b < kBins; b += kSelThreads) {
            H.cnt[b] = 0u;
            H.mass[b] = 0ull;
        }
        __syncthreads();
        // Wave-uniform trip count (hist_add needs all 64 lanes); each lane
        // loads kSelUnroll candidates before using any, so that many memory
        // latencies overlap when the list is in global memory.
        for (int c0 = (tid & ~63) * kSelUnroll; c0 < C; c0 += kSelThreads * kSelUnroll) {
            uint2 ev[kSelUnroll];
#pragma unroll
            for (int u = 0; u < kSelUnroll; ++u) {
                const int c = c0 + u * 64 + (tid & 63);
                ev[u] = c < C ? cand[c] : make_uint2(0u, 0u);
            }
#pragma unroll
            for (int u = 0; u < kSelUnroll; ++u) {
                const int c = c0 + u * 64 + (tid & 63);
                const uint2 e = ev[u];
                const unsigned long long D = order_key(e.x, e.y);
                const bool ok = c < C && (D & Mk) == P;
                const int dg = (int)((D >> shift) & wmask);
                const int lead = hist_add(ok, dg, e.x, ok ? mass_of(e.x) : 0ull, H.cnt, H.mass);
                // read only when the bin holds one token
                if (ok && (lead < 0 || lead == (tid & 63))) H.id[dg] = e.y;
            }
        }
        __syncthreads();
        BinScan<kSelThreads> scan;
        scan.load(H.cnt, H.mass, above, sc);
        scan.find(target, bs, sc);
        if (!bs.found) return -1;
        P |= (unsigned long long)bs.bin << shift;
        Mk |= wmask << shift;
        above = bs.excl;
        if (bs.cnt == 1u) {
            cum_out = bs.incl;
            const int id = (int)H.id[bs.bin];
            __syncthreads();
            return id;
        }
    }
    return -1;   // not reached: the full key is unique
}

// The single token of level-0 bin `bin` among the candidates.
__device__ int only_in_bin(const uint2* cand, int C, int bin, int* s_id) {
    if (threadIdx.x == 0) *s_id = -1;
    __syncthreads();
    for (int c0 = threadIdx.x; c0 < C; c0 += kSelThreads * kSelUnroll) {
        uint2 ev[kSelUnroll];
#pragma unroll
        for (int u = 0; u < kSelUnroll; ++u) {
            const int c = c0 + u * kSelThreads;
            ev[u] = c < C ? cand[c] : make_uint2(0u, 0xFFFFFFFFu);
        }
#pragma unroll
        for (int u = 0; u < kSelUnroll; ++u)
            if (c0 + u * kSelThreads < C && (int)(ev[u].x >> 20) == bin) *s_id = (int)ev[u].y;
    }
    __syncthreads();
    const int r = *s_id;
    __syncthreads();
    return r;
}

// argmax helpers: NaNs never win, ties go to the lower index
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return bi < 0 || v > bv || (v == bv && i < bi);
}

__device__ void block_best(float& bv, int& bi, float* rv, int* ri) {
    const int t = threadIdx.x;
    rv[t] = bv;
    ri[t] = bi;
    __syncthreads();
    for (int s = kGridThreads / 2; s > 0; s >>= 1) {
        if (t < s && ri[t + s] >= 0 && better(rv[t + s], ri[t + s], rv[t], ri[t])) {
            rv[t] = rv[t + s];
            ri[t] = ri[t + s];
        }
        __syncthreads();
    }
    bv = rv[0];
    bi = ri[0];
}

}  // namespace

// ------------------------------------------------------------------ argmax --
// Per-block first maxima, then the first maximum of those; a NaN at index 0
// gives 0 (the reference's strict ">" scan from element 0).

__global__ __launch_bounds__(kGridThreads) void argmax_partial_kernel(const void* logits, int dtype,
                                                                      int n, float* pv, int* pi) {
    __shared__ float rv[kGridThreads];
    __shared__ int ri[kGridThreads];
    float bv = 0.0f;
    int bi = -1;
    const int T = gridDim.x * kGridThreads;
    for (int q = blockIdx.x * kGridThreads + threadIdx.x; 4 * q < n; q += T) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = 4 * q + k;
            if (i >= n) break;
            const float v = load_logit(logits, dtype, i);
            if (v == v && (bi < 0 || v > bv)) {   // increasing i: first maximum
                bv = v;
                bi = i;
            }
        }
    }
    block_best(bv, bi, rv, ri);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = bv;
        pi[blockIdx.x] = bi;
    }
}

__global__ __launch_bounds__(kGridThreads) void argmax_final_kernel(const void* logits, int dtype,
                                                                    const float* pv, const int* pi,
                                                                    int blocks, int32_t* out) {
    __shared__ float rv[kGridThreads];
    __shared__ int ri[kGridThreads];
    float bv = 0.0f;
    int bi = -1;
    if ((int)threadIdx.x < blocks) {
        bv = pv[threadIdx.x];
        bi = pi[threadIdx.x];
    }
    block_best(bv, bi, rv, ri);
    if (threadIdx.x == 0) {
        const float v0 = load_logit(logits, dtype, 0);
        *out = (v0 != v0 || bi < 0) ? 0 : bi;
    }
}

// ---------------------------------------------------------------- sampling --

// l = (seen ? penalised : logit) / temperature; per block the max m_b of l
// and s_b = sum of exp(l - m_b).  Thread t of block b handles quads
// q = 256 b + t + k T (tokens 4q..4q+3), k = 0, 1, ...; the block's seen ids
// are marked in an LDS bitmap indexed by (k, t, token within the quad).
__global__ __launch_bounds__(kGridThreads) void sample_scale_kernel(SampleParams p) {
    __shared__ float red[kGridThreads];
    __shared__ uint32_t seen_bm[kSeenWords];
    const int n = p.n;
    const int T = gridDim.x * kGridThreads;
    const int nq = (n + 3) / 4;
    for (int b = blockIdx.x * kGridThreads + threadIdx.x; b < kBins; b += T) {
        p.h0cnt[b] = 0u;
        p.h0mass[b] = 0ull;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) *p.ccount = 0u;
    const int n_seen = seen_count(p);
    if (n_seen > 0) {
        for (int w = threadIdx.x; w < kSeenWords; w += kGridThreads) seen_bm[w] = 0u;
        __syncthreads();
        for (int j = threadIdx.x; j < n_seen; j += kGridThreads) {
            const int t = p.seen[j];
            if (t < 0 || t >= n) continue;
            const int q = t >> 2, r = q % T;
            if (r / kGridThreads != (int)blockIdx.x) continue;
            const int bit = (q / T) * (4 * kGridThreads) + (r % kGridThreads) * 4 + (t & 3);
            atomicOr(&seen_bm[bit >> 5], 1u << (bit & 31));
        }
        __syncthreads();
    }
    float mx = -3.402823466e38f;   // -greatestFiniteMagnitude
    float l0[4] = {0.0f, 0.0f, 0.0f, 0.0f};   // the first quad, kept for the exp-sum pass
    int k = 0;
    for (int q = blockIdx.x * kGridThreads + threadIdx.x; q < nq; q += T, ++k) {
        const int bit0 = k * (4 * kGridThreads) + threadIdx.x * 4;
        const uint32_t seen = n_seen > 0 ? (seen_bm[bit0 >> 5] >> (bit0 & 31)) & 15u : 0u;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = 4 * q + e;
            if (i >= n) break;
            float l = load_logit(p.logits, p.dtype, i);
            if (seen & (1u << e)) l = l > 0.0f ? l / p.penalty : l * p.penalty;
            l = l / p.temperature;
            p.probs[i] = l;
            if (k == 0) l0[e] = l;
            mx = fmaxf(mx, l);
        }
    }
    red[threadIdx.x] = mx;
    __syncthreads();
    for (int s2 = kGridThreads / 2; s2 > 0; s2 >>= 1) {
        if ((int)threadIdx.x < s2) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s2]);
        __syncthreads();
    }
    const float mb = red[0];
    __syncthreads();
    float sm = 0.0f;
    for (int q = blockIdx.x * kGridThreads + threadIdx.x, kk = 0; q < nq; q += T, ++kk) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = 4 * q + e;
            if (i >= n) break;
            sm += expf((kk == 0 ? l0[e] : p.probs[i]) - mb);
        }
    }
    red[threadIdx.x] = sm;
    __syncthreads();
    for (int s2 = kGridThreads / 2; s2 > 0; s2 >>= 1) {
        if ((int)threadIdx.x < s2) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + s2];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        p.mpart[blockIdx.x] = mb;
        p.spart[blockIdx.x] = red[0];
    }
}

// p = exp(l - max) / sum, sum = the block exp-sums rescaled to the global
// max and added in a fixed order; level-0 histogram
__global__ __launch_bounds__(kGridThreads) void sample_prob_kernel(SampleParams p) {
    __shared__ uint32_t hc[kBins];
    __shared__ unsigned long long hm[kBins];
    __shared__ float s_sum, s_max, wred[kGridThreads / 64];
    const int n = p.n;
    const int T = gridDim.x * kGridThreads;
    for (int b = threadIdx.x; b < kBins; b += kGridThreads) {
        hc[b] = 0u;
        hm[b] = 0ull;
    }
    // this thread's first quad, requested before the fold below
    float l0[4];
    {
        const int q = blockIdx.x * kGridThreads + (int)threadIdx.x;
#pragma unroll
        for (int k = 0; k < 4; ++k) l0[k] = 4 * q + k < n ? p.probs[4 * q + k] : 0.0f;
    }
    // The global max and the denominator: thread t holds block t's pair; the
    // max is exact in any order; the sum of the rescaled terms runs as a
    // halving tree within each wave (lanes 32 apart first), then
    // (w0 + w1) + (w2 + w3).
    const int G = (int)gridDim.x;
    const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
    const float mt = t < G ? p.mpart[t] : -3.402823466e38f;
    const float st = t < G ? p.spart[t] : 0.0f;
    float wm = mt;
    for (int o = 32; o > 0; o >>= 1) wm = fmaxf(wm, __shfl_xor(wm, o, 64));
    if (lane == 0) wred[wid] = wm;
    __syncthreads();
    const float gmax = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
    float term = t < G ? st * expf(mt - gmax) : 0.0f;
    for (int o = 32; o > 0; o >>= 1) term += __shfl_down(term, o, 64);
    __syncthreads();   // every wave has read wred
    if (lane == 0) wred[wid] = term;
    __syncthreads();
    if (t == 0) {
        s_sum = (wred[0] + wred[1]) + (wred[2] + wred[3]);
        s_max = gmax;
    }
    __syncthreads();
    const float sm = s_sum, mx = s_max;
    // wave-uniform trip count: hist_add needs all 64 lanes
    const int q_first = blockIdx.x * kGridThreads + threadIdx.x;
    for (int qw = q_first - (threadIdx.x & 63); 4 * qw < n; qw += T) {
        const int q = qw + (threadIdx.x & 63);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = 4 * q + k;
            const bool ok = i < n;
            float pv = 0.0f;
            if (ok) {
                pv = expf((q == q_first ? l0[k] : p.probs[i]) - mx) / sm;
                p.probs[i] = pv;
            }
            const uint32_t key = __float_as_uint(pv);
            hist_add(ok, (int)(key >> 20), key, ok ? mass_of(key) : 0ull, hc, hm);
        }
    }
    __syncthreads();
    for (int b = threadIdx.x; b < kBins; b += kGridThreads) {
        if (hc[b]) atomicAdd(&p.h0cnt[b], hc[b]);
        if (hm[b]) atomicAdd(&p.h0mass[b], hm[b]);
    }
}

// Compacts the tokens of the cutoff's level-0 bin and of every bin the draw
// can land in: its target lies in [ceil(u * T1), ceil(u * incl(cutoff bin))]
// since the cutoff token's inclusive mass is at least T1 and at most its
// bin's.
__global__ __launch_bounds__(kGridThreads) void sample_gather_kernel(SampleParams p) {
    constexpr int kWaves = kGridThreads / 64;
    __shared__ uint32_t offs[kWaves * 4];   // per wave and sub-step: slot offset in the block
    __shared__ uint32_t s_base;
    __shared__ SelScratch sc;
    __shared__ BinSel s1, s2;
    const int n = p.n;
    const int T = gridDim.x * kGridThreads;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    // this thread's first quad, requested before the histogram scan so the
    // two memory latencies overlap
    uint32_t key0[4];
    {
        const int q = blockIdx.x * kGridThreads + (int)threadIdx.x;
#pragma unroll
        for (int k = 0; k < 4; ++k) key0[k] = 4 * q + k < n ? __float_as_uint(p.probs[4 * q + k]) : 0u;
    }
    const unsigned long long t1 = target_top_p(p.top_p);
    BinScan<kGridThreads> scan;
    scan.load(p.h0cnt, p.h0mass, 0ull, sc);
    scan.find(t1, s1, sc);
    unsigned long long tlo, thi;
    const float u = draw_of(p);
    if (s1.found) {
        tlo = target_draw(u, t1);
        thi = target_draw(u, s1.incl);
    } else {
        tlo = thi = target_draw(u, s1.total);
    }
    scan.find(thi, s2, sc);
    const int lo = s2.found ? s2.bin : 0;
    scan.find(tlo, s2, sc);
    const int hi = s2.found ? s2.bin : kBins - 1;
    const int b1 = s1.found ? s1.bin : -1;
    // block-uniform loop; one atomic a block reserves its slots
    for (int qb = blockIdx.x * kGridThreads; 4 * qb < n; qb += T) {
        const int q = qb + (int)threadIdx.x;
        uint32_t key[4];
        unsigned long long bal[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = 4 * q + k;
            key[k] = qb == (int)(blockIdx.x * kGridThreads) ? key0[k]
                     : i < n ? __float_as_uint(p.probs[i]) : 0u;
            const int b = (int)(key[k] >> 20);
            bal[k] = __ballot(i < n && (b == b1 || (b >= lo && b <= hi)));
        }
        if (lane == 0) {
#pragma unroll
            for (int k = 0; k < 4; ++k) offs[wid * 4 + k] = (uint32_t)__popcll(bal[k]);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            uint32_t tot = 0u;
            for (int j = 0; j < kWaves * 4; ++j) {
                const uint32_t c = offs[j];
                offs[j] = tot;
                tot += c;
            }
            s_base = tot ? atomicAdd(p.ccount, tot) : 0u;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if ((bal[k] >> lane) & 1ull)
                p.cand[s_base + offs[wid * 4 + k] + lanes_below(bal[k])] =
                    make_uint2(key[k], (uint32_t)(4 * q + k));
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(kSelThreads) void sample_select_kernel(SampleParams p) {
    __shared__ uint2 lc[kCandLds];
    __shared__ LevelHist H;
    __shared__ SelScratch sc;
    __shared__ BinSel s0, bs;
    __shared__ BinSel s1;
    __shared__ int s_id;
    const int C = (int)*p.ccount;
    // read before the first barrier: thread 0 advances the draw index at the end
    const float u = draw_of(p);
    const unsigned long long t1 = target_top_p(p.top_p);
    BinScan<kSelThreads> scan0;   // the level-0 histogram
    scan0.load(p.h0cnt, p.h0mass, 0ull, sc);
    scan0.find(t1, s1, sc);       // the cutoff's bin

    if (C <= 64) {
        // Few candidates (the usual nucleus of a peaked distribution): one
        // wave sorts them by key and scans their masses.  First the mass of
        // all bins above each bin, into H.mass.
        {
            unsigned long long run = scan0.excl;
#pragma unroll
            for (int k = 0; k < BinScan<kSelThreads>::BPT; ++k) {
                H.mass[scan0.top - k] = run;
                run += scan0.m[k];
            }
        }
        __syncthreads();
        if (threadIdx.x >= 64) return;
        const int lane = threadIdx.x;
        const uint2 e = lane < C ? p.cand[lane] : make_uint2(0u, 0u);
        unsigned long long sk = lane < C ? (1ull << 63) | order_key(e.x, e.y) : 0ull;
        // bitonic sort, descending, across the wave
        for (int k = 2; k <= 64; k <<= 1) {
            for (int j = k >> 1; j > 0; j >>= 1) {
                const unsigned long long o = __shfl_xor(sk, j, 64);
                const bool take_max = ((lane & j) == 0) == ((lane & k) == 0);
                sk = take_max ? (sk > o ? sk : o) : (sk < o ? sk : o);
            }
        }
        const bool valid = (sk >> 63) != 0ull;
        const uint32_t key = (uint32_t)(sk >> 24);
        const int id = (int)(kIdMask - (uint32_t)(sk & kIdMask));
        const int bin = valid ? (int)(key >> 20) : -1;
        const unsigned long long m = valid ? mass_of(key) : 0ull;
        // inclusive running mass inside each bin (bins are contiguous runs)
        unsigned long long S = m;
        for (int o = 1; o < 64; o <<= 1) {
            const unsigned long long y = __shfl_up(S, o, 64);
            if (lane >= o) S += y;
        }
        const int prev_bin = __shfl_up(bin, 1, 64);
        const bool head = valid && (lane == 0 || prev_bin != bin);
        const unsigned long long heads = __ballot(head) & ((2ull << lane) - 1ull);
        const int start = heads ? 63 - __clzll((long long)heads) : 0;
        const unsigned long long before = __shfl(S, start > 0 ? start - 1 : 0, 64);
        const unsigned long long cum =
            (valid ? H.mass[bin] : 0ull) + S - (start > 0 ? before : 0ull);
        unsigned long long cut = s1.total;
        if (s1.found) {
            const unsigned long long hit = __ballot(valid && bin == s1.bin && cum >= t1);
            cut = hit ? __shfl(cum, __ffsll((long long)hit) - 1, 64) : s1.incl;
        }
        const unsigned long long t2 = target_draw(u, cut);
        const unsigned long long hit2 = __ballot(valid && cum >= t2);
        const int chosen = __shfl(id, hit2 ? __ffsll((long long)hit2) - 1 : 0, 64);
        if (lane == 0) finish_select(p, hit2 ? chosen : 0);
        return;
    }

    const uint2* cand = p.cand;
    if (C <= kCandLds) {
        for (int c = threadIdx.x; c < C; c += kSelThreads) lc[c] = p.cand[c];
        cand = lc;
    }
    __syncthreads();
    // the cutoff: its inclusive mass
    unsigned long long cum = s1.total;
    if (s1.found) {
        if (s1.cnt == 1u)
            cum = s1.incl;
        else
            (void)select_in_bin(cand, C, s1.bin, s1.excl, t1, H, sc, bs, cum);
    }
    // the draw
    const unsigned long long t2 = target_draw(u, cum);
    scan0.find(t2, s0, sc);
    int id = -1;
    if (s0.found) {
        if (s0.cnt == 1u) {
            id = only_in_bin(cand, C, s0.bin, &s_id);
        } else {
            unsigned long long c2 = 0ull;
            id = select_in_bin(cand, C, s0.bin, s0.excl, t2, H, sc, bs, c2);
        }
    }
    if (threadIdx.x == 0) finish_select(p, id < 0 ? 0 : id);
}

// ------------------------------------------------------------------- host --

namespace {

int grid_blocks(int n) {
    const int b = (n + 4 * kGridThreads - 1) / (4 * kGridThreads);
    return b < kMaxBlocks ? b : kMaxBlocks;
}

size_t up256(size_t b) { return (b + 255) / 256 * 256; }

}  // namespace

size_t argmax_workspace_bytes() { return 2 * kMaxBlocks * 4; }

constexpr size_t sample_ws_bytes(size_t n) {
    return (n * 4 + 255) / 256 * 256 + 2 * ((kMaxBlocks * 4 + 255) / 256 * 256) +
           (kBins * 4 + 255) / 256 * 256 + (kBins * 8 + 255) / 256 * 256 + 256 +
           (n * 8 + 255) / 256 * 256;
}

size_t sample_workspace_bytes(int n) { return sample_ws_bytes((size_t)n); }

// Scratch of sltx_sample_top_p_noalloc: the sampler's workspace for up to
// kSampleNoAllocMaxN logits (3,197,184 bytes), in a file-scope device array,
// so that entry point allocates nothing.  Each GPU holds its own copy until
// the process ends, and every call on that GPU shares it (the scale kernel
// clears the counters each call; the other regions are written before they
// are read).  In host code `scratch` only names the symbol: kernels are given
// the device address resolved per device below.
static_assert(sample_ws_bytes(kSampleNoAllocMaxN) == 3197184, "noalloc scratch size");
static __device__ __align__(256) unsigned char scratch[sample_ws_bytes(kSampleNoAllocMaxN)];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];
}  // namespace

int sample_noalloc_scratch_init(int dev) {
    if (dev < 0 || dev >= kMaxDevices) return set_error(kErrHip, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[dev]) return kOk;
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
        return set_error(kErrHip, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                         hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
    return kOk;
}

void* sample_noalloc_scratch(int dev) {
    if (dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return g_scratch_ptr[dev];
}

hipError_t launch_argmax(const void* logits, int dtype, int n, int32_t* out, void* ws,
                         hipStream_t st) {
    const int G = grid_blocks(n);
    float* pv = static_cast<float*>(ws);
    int* pi = reinterpret_cast<int*>(pv + kMaxBlocks);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(G), dim3(kGridThreads), 0, st, logits, dtype, n,
                       pv, pi);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kGridThreads), 0, st, logits, dtype, pv,
                       pi, G, out);
    return hipGetLastError();
}

hipError_t launch_sample(SampleParams p, void* ws, hipStream_t st) {
    char* w = static_cast<char*>(ws);
    const size_t n = (size_t)p.n;
    p.probs = reinterpret_cast<float*>(w);
    w += up256(n * 4);
    p.mpart = reinterpret_cast<float*>(w);
    w += up256(kMaxBlocks * 4);
    p.spart = reinterpret_cast<float*>(w);
    w += up256(kMaxBlocks * 4);
    p.h0cnt = reinterpret_cast<uint32_t*>(w);
    w += up256(kBins * 4);
    p.h0mass = reinterpret_cast<unsigned long long*>(w);
    w += up256(kBins * 8);
    p.ccount = reinterpret_cast<uint32_t*>(w);
    w += 256;
    p.cand = reinterpret_cast<uint2*>(w);
    const int G = grid_blocks(p.n);
    hipLaunchKernelGGL(sample_scale_kernel, dim3(G), dim3(kGridThreads), 0, st, p);
    hipLaunchKernelGGL(sample_prob_kernel, dim3(G), dim3(kGridThreads), 0, st, p);
    hipLaunchKernelGGL(sample_gather_kernel, dim3(G), dim3(kGridThreads), 0, st, p);
    hipLaunchKernelGGL(sample_select_kernel, dim3(1), dim3(kSelThreads), 0, st, p);
    return hipGetLastError();
}

}  // namespace sltx
