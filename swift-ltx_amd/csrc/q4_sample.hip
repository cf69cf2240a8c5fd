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
//                   the level-0 and range histograms
//   sample_prob     p = exp(l - max) / sum; level-0 histogram (p bits
//                   31..20: count and mass per bin)
//   sample_gather   each block finds, from the histogram, the bin holding the
//                   cutoff and the bins the draw can reach; if their untied
//                   tokens fit the select kernel's LDS it compacts them
//                   (mode 0), otherwise it builds a range histogram over
//                   their keys in finer buckets (mode 1), sized from the
//                   smallest and largest key of those bins.  Bins and buckets
//                   of one key (ties) are never compacted: their tokens are
//                   found by rank, from counts of the tied key per 1024-token
//                   chunk kept during compaction.  (No grid-wide fence or
//                   last-block hand-off: on a chip whose XCDs have separate
//                   L2s those cost more than re-reading the 48 KB histogram
//                   per block.)
//   sample_narrow   mode 1: the same from the range histogram, compacting
//                   the untied tokens of the buckets that matter
//   sample_select   one workgroup: up to 64 candidates are sorted in one
//                   wave's registers and scanned; more go through the levels
//                   below their bucket, 12 bits of D a level (in LDS when
//                   they fit), until a level's bin holds at most 64 tokens,
//                   which one wave sorts
#include <algorithm>
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
constexpr int kSelUnroll = 8;      // candidates each select thread loads before using them
constexpr int kNthUnroll = 16;     // 16-byte key loads a lane has in flight in nth_with_key
constexpr int kTiedSlots = 4;      // tied keys with per-chunk counts
constexpr int kSmallLevel = 4096;  // tokens up to which a select level takes an 8-bit digit
constexpr uint32_t kIdMask = 0xFFFFFFu;
// seen-id bitmap of one scale block: up to 64 quads a thread (n <= 2^24
// with 256 blocks of 256 threads), 4 bits a quad
constexpr int kSeenWords = 64 * 4 * kGridThreads / 32;

// Wave-wide inclusive prefix sums in lane order through DPP: row shifts by
// 1, 2, 4, 8 (out-of-row sources read 0), then the last lane of rows 0 / 2
// added to rows 1 / 3 and lane 31 to rows 2-3 -- six steps at VALU latency
// instead of LDS-routed shuffles.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_move(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xF, true);
}

__device__ __forceinline__ uint32_t wave_incl_sum(uint32_t x) {
    x += dpp_move<0x111, 0xF>(x);
    x += dpp_move<0x112, 0xF>(x);
    x += dpp_move<0x114, 0xF>(x);
    x += dpp_move<0x118, 0xF>(x);
    x += dpp_move<0x142, 0xA>(x);
    x += dpp_move<0x143, 0xC>(x);
    return x;
}

template <int CTRL, int ROWS>
__device__ __forceinline__ unsigned long long dpp_move(unsigned long long v) {
    const uint32_t lo = dpp_move<CTRL, ROWS>((uint32_t)v);
    const uint32_t hi = dpp_move<CTRL, ROWS>((uint32_t)(v >> 32));
    return ((unsigned long long)hi << 32) | lo;
}

__device__ __forceinline__ unsigned long long wave_incl_sum(unsigned long long x) {
    x += dpp_move<0x111, 0xF>(x);
    x += dpp_move<0x112, 0xF>(x);
    x += dpp_move<0x114, 0xF>(x);
    x += dpp_move<0x118, 0xF>(x);
    x += dpp_move<0x142, 0xA>(x);
    x += dpp_move<0x143, 0xC>(x);
    return x;
}

// The whole wave's smallest / largest value, in every lane: the same DPP
// steps with `id` read where a shift has no source lane.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_move_id(uint32_t v, uint32_t id) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)id, (int)v, CTRL, ROWS, 0xF, false);
}

template <bool MAX>
__device__ __forceinline__ uint32_t wave_minmax(uint32_t x) {
    constexpr uint32_t id = MAX ? 0u : 0xFFFFFFFFu;
    auto f = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
    x = f(x, dpp_move_id<0x111, 0xF>(x, id));
    x = f(x, dpp_move_id<0x112, 0xF>(x, id));
    x = f(x, dpp_move_id<0x114, 0xF>(x, id));
    x = f(x, dpp_move_id<0x118, 0xF>(x, id));
    x = f(x, dpp_move_id<0x142, 0xA>(x, id));
    x = f(x, dpp_move_id<0x143, 0xC>(x, id));
    return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}

// The whole wave's sum, in every lane.
template <class T>
__device__ __forceinline__ T wave_sum(T x) {
    const T s = wave_incl_sum(x);
    if constexpr (sizeof(T) == 8) {
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)s, 63);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(s >> 32), 63);
        return (T)(((unsigned long long)hi << 32) | lo);
    } else {
        return (T)__builtin_amdgcn_readlane((int)s, 63);
    }
}

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
        sum = wave_sum(ok ? m : 0ull);
    }
    if (lane == lead) {
        atomicAdd(&cnt[d0], (uint32_t)__popcll(act));
        if (sum) atomicAdd(&mass[d0], sum);
    }
    return lead;
}

// Smallest and largest key of bin d for the lanes with ok set, kept in LDS
// next to the histogram (lead: hist_add's result, the lane that added for
// the whole wave, which then holds every active lane in one bin).
__device__ __forceinline__ void key_minmax(bool ok, int d, uint32_t key, int lead, uint32_t* kmin,
                                           uint32_t* kmax) {
    if (lead < 0) {
        if (ok) {
            atomicMin(&kmin[d], key);
            atomicMax(&kmax[d], key);
        }
        return;
    }
    const unsigned long long act = __ballot(ok);
    const uint32_t k0 = (uint32_t)__builtin_amdgcn_readlane((int)key, lead);
    uint32_t lo = k0, hi = k0;
    if (__ballot(ok && key == k0) != act) {
        lo = wave_minmax<false>(ok ? key : 0xFFFFFFFFu);
        hi = wave_minmax<true>(ok ? key : 0u);
    }
    if ((int)(threadIdx.x & 63) == lead) {
        atomicMin(&kmin[d], lo);
        atomicMax(&kmax[d], hi);
    }
}

// The buckets the select positions are found in.  Mode 0: level-0 bins,
// key >> 20.  Mode 1 (the range histogram): segment A, keys [a_lo, a_end) in
// buckets [0, kSplit) of 2^a_shift keys counted from a_base; segment B, keys
// [b_lo, b_end) in buckets [kSplit, kBins) of 2^b_shift keys counted from
// b_base (each base is its low key rounded down to the bucket width); the
// keys between the segments are in no bucket (their mass, `gap`, is added to
// segment A's running mass) and no candidate lies there.
constexpr int kSplit = kBins / 2;

struct Buckets {
    const uint32_t* cnt;
    const unsigned long long* mass;
    const uint32_t* kmin;
    const uint32_t* kmax;
    int ranged;
    uint32_t a_lo, a_base, b_lo, b_base;
    unsigned long long a_end, b_end;
    int a_shift, b_shift;
    unsigned long long gap;

    // bucket of a key, kBins if none
    __device__ int of(uint32_t key) const {
        if (!ranged) return (int)(key >> 20);
        if (key >= a_lo && (unsigned long long)key < a_end) return (int)((key - a_base) >> a_shift);
        if (key >= b_lo && (unsigned long long)key < b_end)
            return kSplit + (int)((key - b_base) >> b_shift);
        return kBins;
    }
    // bits of the order key D below bucket b's key prefix, and that prefix
    __device__ int low_bits(int b) const {
        return !ranged ? 44 : (b < kSplit ? a_shift : b_shift) + 24;
    }
    __device__ unsigned long long prefix(int b) const {
        if (!ranged) return (unsigned long long)b << 44;
        if (b < kSplit)
            return (unsigned long long)((a_base >> a_shift) + (uint32_t)b) << (a_shift + 24);
        return (unsigned long long)((b_base >> b_shift) + (uint32_t)(b - kSplit)) << (b_shift + 24);
    }
};

__device__ __forceinline__ Buckets level0_buckets(const SampleParams& p) {
    return Buckets{p.h0cnt, p.h0mass, p.h0min, p.h0max, 0, 0u, 0u, 0u, 0u, 0ull, 0ull, 20, 20,
                   0ull};
}

__device__ __forceinline__ Buckets range_buckets(const SampleParams& p, const SampleCtl& c) {
    return Buckets{p.h1cnt, p.h1mass, p.h1min, p.h1max, 1, c.a_lo, c.a_base, c.b_lo, c.b_base,
                   c.a_end, c.b_end, c.a_shift, c.b_shift, c.gap};
}

// The narrowest power-of-two bucket width (its log2) that puts the keys
// [lo, hi] into kSegBuckets buckets counted from lo rounded down to the
// width.  A segment has kSplit buckets; using fewer keeps the gather
// kernel's histogram merge short (one set of device atomics per non-empty
// bucket and block) while its buckets stay far narrower than a level-0 bin.
constexpr uint32_t kSegBuckets = 512;

__device__ __forceinline__ int seg_shift(uint32_t lo, uint32_t hi) {
    int sh = 0;
    while (sh < 32 && (hi >> sh) - (lo >> sh) >= kSegBuckets) ++sh;
    return sh;
}

// Bucket b holds more than one token and all share one key (LDS bitmap of
// BinScan::load_tied): in the order (p descending, id ascending) its tokens
// follow each other by id, each adding the same mass.
__device__ __forceinline__ bool is_tied(const uint32_t* tied_bm, int b) {
    return b >= 0 && b < kBins && ((tied_bm[b >> 5] >> (b & 31)) & 1u);
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
    const unsigned long long x = wave_incl_sum(v);
    if (lane == 63) wsum[wid] = x;
    __syncthreads();
    if (wid == 0) {
        const unsigned long long w = wave_incl_sum(lane < NT / 64 ? wsum[lane] : 0ull);
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
    int chunk;                 // nth_in_chunks: the chunk; select_in_bin: the id
    int nfew;
    unsigned long long rem;    // nth_in_chunks: rank left; select_in_bin: inclusive mass
};

// kBins buckets in descending order, after `above` mass, spread over the
// block (BPT consecutive buckets a thread).  load() reads the buckets and
// scans their masses; find(target) gives the highest non-empty bucket whose
// inclusive running mass reaches target (found), its exclusive / inclusive
// mass and count, and the total.  Whole block; cnt and mass may be global or
// LDS.  Both end synchronised.
template <int NT>
struct BinScan {
    static constexpr int BPT = kBins / NT;
    uint32_t c[BPT];
    unsigned long long m[BPT];
    uint32_t kmn[BPT], kmx[BPT];   // load_tied: each bucket's smallest and largest key
    unsigned long long excl, tot;
    int top;   // this thread's buckets: top, top-1, ..., top-BPT+1

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

    // load() over a histogram with key extremes: also marks the tied buckets
    // in tied_bm (kBins bits, LDS; written whole), and in mode 1 adds the
    // mass between the segments to segment A's running mass.
    __device__ void load_tied(const Buckets& bk, unsigned long long above, SelScratch& sc,
                              uint32_t* tied_bm) {
        top = kBins - 1 - (int)threadIdx.x * BPT;
        tot = 0ull;
#pragma unroll
        for (int k = 0; k < BPT; ++k) {
            c[k] = bk.cnt[top - k];
            m[k] = bk.mass[top - k];
            kmn[k] = bk.kmin[top - k];
            kmx[k] = bk.kmax[top - k];
        }
        uint32_t t = 0u;
#pragma unroll
        for (int k = 0; k < BPT; ++k) {
            tot += m[k];
            if (c[k] > 1u && kmn[k] == kmx[k]) t |= 1u << ((top - k) & 31);
        }
        // the 32 / BPT consecutive threads of one bitmap word
        for (int o = 1; o < 32 / BPT; o <<= 1) t |= (uint32_t)__shfl_xor((int)t, o, 64);
        if ((threadIdx.x & (32 / BPT - 1)) == 0) tied_bm[top >> 5] = t;
        excl = above + block_excl_scan<NT>(tot, sc.wsum) +
               (bk.ranged && top < kSplit ? bk.gap : 0ull);
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
        // buckets descend with the thread index: the wave's first hit holds
        // its highest, so one LDS atomic a wave (same-address atomics
        // serialise)
        const unsigned long long hit = __ballot(best >= 0);
        if (hit && (int)(threadIdx.x & 63) == __ffsll((long long)hit) - 1) atomicMax(&sc.best, best);
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

// Calls f(c, e) for every candidate index c < C (e = cand[c]) in a
// wave-uniform loop (hist_add needs all 64 lanes): candidate c goes to wave
// (c / 64) % 16, each lane loading kSelUnroll candidates before using any
// (memory latencies overlap when the list is in global memory); lanes past
// C get c >= C.
template <class F>
__device__ __forceinline__ void for_each_cand(const uint2* cand, int C, F f) {
    const int lane = threadIdx.x & 63;
    for (int c0 = (int)(threadIdx.x & ~63u); c0 < C; c0 += kSelThreads * kSelUnroll) {
        uint2 ev[kSelUnroll];
#pragma unroll
        for (int u = 0; u < kSelUnroll; ++u) {
            const int c = c0 + u * kSelThreads + lane;
            ev[u] = c < C ? cand[c] : make_uint2(0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < kSelUnroll; ++u) f(c0 + u * kSelThreads + lane, ev[u]);
    }
}

// The levels below bucket `bucket` (exclusive mass `above`) of the weighted
// select over the 56-bit order key D: 12 bits a level (fewer for the last);
// once a level's bin holds at most 64 tokens, one wave sorts them.  The
// token whose inclusive running mass first reaches target.  Whole block;
// returns the id (-1 only for non-finite input) and sets cum_out to its
// inclusive mass.
__device__ int select_in_bin(const uint2* cand, int C, const Buckets& bk, int bucket,
                             uint32_t count, unsigned long long above, unsigned long long target,
                             LevelHist& H, SelScratch& sc, BinSel& bs,
                             unsigned long long& cum_out) {
    const int tid = threadIdx.x, lane = tid & 63;
    int pos = bk.low_bits(bucket);
    unsigned long long P = bk.prefix(bucket);
    unsigned long long Mk = (0xFFFFFFFFFFFFFFull >> pos) << pos;
    uint32_t left = count;   // tokens under the prefix
    while (left > 64u && pos > 0) {
        // at most kSmallLevel tokens: an 8-bit digit, whose 256 bins one wave
        // scans (three barriers a level instead of the block-wide scan's eight)
        const bool small = left <= (uint32_t)kSmallLevel;
        const int width = small ? 8 : 12;
        const int shift = pos > width ? pos - width : 0;
        const unsigned long long wmask = (1ull << (pos - shift)) - 1ull;
        pos = shift;
        for (int b = tid; b < (small ? 256 : kBins); b += kSelThreads) {
            H.cnt[b] = 0u;
            H.mass[b] = 0ull;
        }
        __syncthreads();
        for_each_cand(cand, C, [&](int c, uint2 e) {
            const unsigned long long D = order_key(e.x, e.y);
            const bool ok = c < C && (D & Mk) == P;
            const int dg = (int)((D >> shift) & wmask);
            const int lead = hist_add(ok, dg, e.x, ok ? mass_of(e.x) : 0ull, H.cnt, H.mass);
            // read only when the bin holds one token
            if (ok && (lead < 0 || lead == lane)) H.id[dg] = e.y;
        });
        __syncthreads();
        if (small) {
            // lane l: bins 255 - 4l .. 252 - 4l (descending order)
            if (tid < 64) {
                uint32_t c4[4];
                unsigned long long m4[4], t = 0ull;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    c4[k] = H.cnt[255 - 4 * lane - k];
                    m4[k] = H.mass[255 - 4 * lane - k];
                    t += m4[k];
                }
                unsigned long long run = above + wave_incl_sum(t) - t;
                int hk = -1;
                uint32_t hc = 0u;
                unsigned long long e = 0ull, hm = 0ull;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (hk < 0 && c4[k] && run + m4[k] >= target) {
                        hk = k;
                        e = run;
                        hm = m4[k];
                        hc = c4[k];
                    }
                    run += m4[k];
                }
                const unsigned long long hits = __ballot(hk >= 0);
                if (lane == 0) bs.found = hits != 0ull;
                if (hits && lane == __ffsll((long long)hits) - 1) {
                    bs.bin = 255 - 4 * lane - hk;
                    bs.excl = e;
                    bs.incl = e + hm;
                    bs.cnt = hc;
                }
            }
            __syncthreads();
        } else {
            BinScan<kSelThreads> scan;
            scan.load(H.cnt, H.mass, above, sc);
            scan.find(target, bs, sc);
        }
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
        left = bs.cnt;
    }
    // at most 64 tokens left under the prefix: gather them (H.id is free),
    // and wave 0 sorts them by D and scans their masses after `above`
    if (tid == 0) sc.nfew = 0;
    __syncthreads();
    for_each_cand(cand, C, [&](int c, uint2 e) {
        if (c < C && (order_key(e.x, e.y) & Mk) == P) {
            const int slot = atomicAdd(&sc.nfew, 1);
            if (slot < 64) {
                H.id[2 * slot] = e.x;
                H.id[2 * slot + 1] = e.y;
            }
        }
    });
    __syncthreads();
    if (tid < 64) {
        const bool v = lane < sc.nfew;
        const uint32_t kx = v ? H.id[2 * lane] : 0u, ky = v ? H.id[2 * lane + 1] : 0u;
        unsigned long long sk = v ? (1ull << 63) | order_key(kx, ky) : 0ull;
        for (int k = 2; k <= 64; k <<= 1) {
            for (int j = k >> 1; j > 0; j >>= 1) {
                const unsigned long long o = __shfl_xor(sk, j, 64);
                const bool take_max = ((lane & j) == 0) == ((lane & k) == 0);
                sk = take_max ? (sk > o ? sk : o) : (sk < o ? sk : o);
            }
        }
        const bool valid = (sk >> 63) != 0ull;
        const unsigned long long S = wave_incl_sum(valid ? mass_of((uint32_t)(sk >> 24)) : 0ull);
        const unsigned long long hit = __ballot(valid && above + S >= target);
        if (lane == (hit ? __ffsll((long long)hit) - 1 : 0)) {
            sc.rem = hit ? above + S : 0ull;
            sc.chunk = hit ? (int)(kIdMask - (uint32_t)(sk & kIdMask)) : -1;
        }
    }
    __syncthreads();
    const int id = sc.chunk;
    cum_out = sc.rem;
    __syncthreads();
    return id;
}

// The single token of bucket `bin` among the candidates.
__device__ int only_in_bin(const uint2* cand, int C, const Buckets& bk, int bin, int* s_id) {
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
            if (c0 + u * kSelThreads < C && bk.of(ev[u].x) == bin) *s_id = (int)ev[u].y;
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
        p.h0min[b] = 0xFFFFFFFFu;
        p.h0max[b] = 0u;
        p.h1cnt[b] = 0u;
        p.h1mass[b] = 0ull;
        p.h1min[b] = 0xFFFFFFFFu;
        p.h1max[b] = 0u;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) p.ctl->ccount = 0u;
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
    __shared__ uint32_t hlo[kBins], hhi[kBins];
    __shared__ float s_sum, s_max, wred[kGridThreads / 64];
    const int n = p.n;
    const int T = gridDim.x * kGridThreads;
    for (int b = threadIdx.x; b < kBins; b += kGridThreads) {
        hc[b] = 0u;
        hm[b] = 0ull;
        hlo[b] = 0xFFFFFFFFu;
        hhi[b] = 0u;
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
            const int d = (int)(key >> 20);
            const int lead = hist_add(ok, d, key, ok ? mass_of(key) : 0ull, hc, hm);
            key_minmax(ok, d, key, lead, hlo, hhi);
        }
    }
    __syncthreads();
    for (int b = threadIdx.x; b < kBins; b += kGridThreads) {
        if (hc[b]) {
            atomicAdd(&p.h0cnt[b], hc[b]);
            atomicMin(&p.h0min[b], hlo[b]);
            atomicMax(&p.h0max[b], hhi[b]);
        }
        if (hm[b]) atomicAdd(&p.h0mass[b], hm[b]);
    }
}

namespace {

// Rank inside a tied bucket: the tokens of mass m after `excl` reach target
// t at the j-th one, j = ceil((t - excl) / m) (at least 1).
__device__ __forceinline__ unsigned long long tied_rank(unsigned long long excl,
                                                        unsigned long long t,
                                                        unsigned long long m) {
    if (m == 0ull || t <= excl) return 1ull;
    return (t - excl + m - 1ull) / m;
}

// The mass of each token of a tied bucket found by BinScan::find.
__device__ __forceinline__ unsigned long long tied_mass(const BinSel& s) {
    return (s.incl - s.excl) / s.cnt;
}

// The first quad of this thread's grid-stride walk (NT threads a block),
// requested early so its latency overlaps the histogram scans.
template <int NT>
__device__ __forceinline__ void first_quad(const SampleParams& p, uint32_t (&key0)[4]) {
    const int q = blockIdx.x * NT + (int)threadIdx.x;
#pragma unroll
    for (int k = 0; k < 4; ++k) key0[k] = 4 * q + k < p.n ? __float_as_uint(p.probs[4 * q + k]) : 0u;
}

// Draw-target bounds from the cutoff's bucket: the draw's target lies in
// [ceil(u * T1), ceil(u * incl)] since the cutoff token's inclusive mass is
// at least T1 and at most its bucket's; a bucket of one token or of one key
// fixes the cutoff's mass, so both bounds are the exact target.
__device__ __forceinline__ void draw_bounds(const BinSel& s1, const uint32_t* tied_bm, float u,
                                            unsigned long long t1, unsigned long long total,
                                            unsigned long long& tlo, unsigned long long& thi) {
    if (!s1.found) {
        tlo = thi = target_draw(u, total);
    } else if (s1.cnt == 1u) {
        tlo = thi = target_draw(u, s1.incl);
    } else if (is_tied(tied_bm, s1.bin)) {
        const unsigned long long m = tied_mass(s1);
        tlo = thi = target_draw(u, s1.excl + tied_rank(s1.excl, t1, m) * m);
    } else {
        tlo = target_draw(u, t1);
        thi = target_draw(u, s1.incl);
    }
}

// The keys of the first kTiedSlots tied buckets of [lo, hi], from the top,
// into tkey (LDS); their number into *ntied.  Whole block (NT >= 128).
template <int NT>
__device__ void pick_tied(const Buckets& bk, const uint32_t* tied_bm, int lo, int hi,
                          uint32_t* tkey, int* ntied, SelScratch& sc) {
    const int t = threadIdx.x;
    const int w = kBins / 32 - 1 - t;   // words from the top
    uint32_t bits = 0u;
    if (t < kBins / 32 && lo <= hi && w >= (lo >> 5) && w <= (hi >> 5)) {
        bits = tied_bm[w];
        if (w == (hi >> 5) && (hi & 31) != 31) bits &= (2u << (hi & 31)) - 1u;
        if (w == (lo >> 5)) bits &= ~0u << (lo & 31);
    }
    if (!__syncthreads_or(bits != 0u)) {   // block-uniform: no tied bucket in range
        if (t == 0) *ntied = 0;
        __syncthreads();
        return;
    }
    const unsigned long long before = block_excl_scan<NT>((unsigned long long)__popc(bits), sc.wsum);
    if (t == NT - 1) {
        const unsigned long long all = before + __popc(bits);
        *ntied = all < kTiedSlots ? (int)all : kTiedSlots;
    }
    for (unsigned long long k = before; bits && k < kTiedSlots; ++k) {
        const int b = 31 - __clz(bits);
        bits &= ~(1u << b);
        tkey[k] = bk.kmin[(w << 5) + b];
    }
    __syncthreads();
}

// Tokens of the block's quads (4 consecutive tokens a thread, NT threads,
// block-uniform loop) for which want(key) holds go to p.cand: one atomic a
// block and iteration reserves the slots (wave 0 scans the per-wave,
// per-sub-step counts).  For each of the ntied keys in tkey, the count of its
// tokens in each 1024-token chunk goes to p.tcnt.  key0: the block's first
// quad, already loaded.
template <int NT, class Want>
__device__ void compact(const SampleParams& p, const uint32_t (&key0)[4], Want want,
                        const uint32_t* tkey, int ntied, uint32_t* offs, uint32_t* tsum) {
    constexpr int kWaves = NT / 64;
    static_assert(kWaves * 4 <= 64, "one wave scans the slot counts");
    const int n = p.n;
    const int T = gridDim.x * NT;
    const int nchunk = (n + 1023) >> 10;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    for (int qb = blockIdx.x * NT; 4 * qb < n; qb += T) {
        const int q = qb + (int)threadIdx.x;
        uint32_t key[4];
        unsigned long long bal[4];
        uint32_t tc[kTiedSlots] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = 4 * q + k;
            key[k] = qb == (int)(blockIdx.x * NT) ? key0[k]
                     : i < n ? __float_as_uint(p.probs[i]) : 0u;
            bal[k] = __ballot(i < n && want(key[k]));
#pragma unroll
            for (int s = 0; s < kTiedSlots; ++s)
                if (s < ntied) tc[s] += (uint32_t)__popcll(__ballot(i < n && key[k] == tkey[s]));
        }
        if (lane == 0) {
#pragma unroll
            for (int k = 0; k < 4; ++k) offs[wid * 4 + k] = (uint32_t)__popcll(bal[k]);
#pragma unroll
            for (int s = 0; s < kTiedSlots; ++s) tsum[wid * kTiedSlots + s] = tc[s];
        }
        __syncthreads();
        if (wid == 0) {
            const uint32_t v = lane < kWaves * 4 ? offs[lane] : 0u;
            const uint32_t incl = wave_incl_sum(v);
            const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
            uint32_t base = 0u;
            if (lane == 0 && tot) base = atomicAdd(&p.ctl->ccount, tot);
            base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
            if (lane < kWaves * 4) offs[lane] = base + incl - v;
        } else if (ntied && (int)threadIdx.x - 64 < (NT / 256) * kTiedSlots) {
            // chunk g of this iteration (4 waves, 1024 tokens), slot s
            const int t = (int)threadIdx.x - 64;
            const int g = t / kTiedSlots, s = t % kTiedSlots;
            const int chunk = (qb >> 8) + g;
            if (s < ntied && chunk < nchunk)
                p.tcnt[s * nchunk + chunk] = tsum[(4 * g) * kTiedSlots + s] +
                                             tsum[(4 * g + 1) * kTiedSlots + s] +
                                             tsum[(4 * g + 2) * kTiedSlots + s] +
                                             tsum[(4 * g + 3) * kTiedSlots + s];
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if ((bal[k] >> lane) & 1ull)
                p.cand[offs[wid * 4 + k] + lanes_below(bal[k])] =
                    make_uint2(key[k], (uint32_t)(4 * q + k));
        }
        __syncthreads();
    }
}

}  // namespace

// Finds, from the level-0 histogram, the bin holding the cutoff and the bins
// the draw can land in.  When their untied tokens fit the select kernel's
// LDS (mode 0) it compacts them; otherwise (mode 1) it builds the range
// histogram over the keys of those bins (segment A: the cutoff's bin,
// segment B: the draw's bins), which the select kernel's blocks then narrow
// and compact.  No grid-wide fence or last-block hand-off here: on a chip
// whose XCDs have separate L2s those cost more than re-reading the 48 KB
// histogram per block.
__global__ __launch_bounds__(kGridThreads) void sample_gather_kernel(SampleParams p) {
    constexpr int kWaves = kGridThreads / 64;
    __shared__ uint32_t offs[kWaves * 4];   // per wave and sub-step: slot offset in the block
    __shared__ uint32_t tsum[kWaves * kTiedSlots];
    __shared__ uint32_t tied_bm[kBins / 32];
    __shared__ uint32_t s_tkey[kTiedSlots], s_cnt[kWaves], s_amn, s_amx;
    __shared__ int s_ntied;
    __shared__ SelScratch sc;
    __shared__ BinSel s1, s2;
    __shared__ uint32_t hc[kBins], hlo[kBins], hhi[kBins];
    __shared__ unsigned long long hm[kBins];
    const int n = p.n;
    const int T = gridDim.x * kGridThreads;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    uint32_t key0[4];
    first_quad<kGridThreads>(p, key0);
    const Buckets bk = level0_buckets(p);
    const unsigned long long t1 = target_top_p(p.top_p);
    BinScan<kGridThreads> scan;
    scan.load_tied(bk, 0ull, sc, tied_bm);
    scan.find(t1, s1, sc);
    unsigned long long tlo, thi;
    draw_bounds(s1, tied_bm, draw_of(p), t1, s1.total, tlo, thi);
    scan.find(thi, s2, sc);
    const int lo = s2.found ? s2.bin : 0;
    scan.find(tlo, s2, sc);
    const int hi = s2.found ? s2.bin : kBins - 1;
    const unsigned long long above_hi = s2.found ? s2.excl : 0ull;
    const int b1 = s1.found ? s1.bin : -1;
    auto want = [&](int b) { return (b == b1 || (b >= lo && b <= hi)) && !is_tied(tied_bm, b); };
    // segment A: the cutoff's bin (else the draw's first); B: the draw's
    // bins above it; the untied candidates and the mass between A and B
    const int a = b1 >= 0 ? b1 : lo;
    const int blo = max(lo, a + 1);
    uint32_t mine = 0u;
    unsigned long long gapm = 0ull;
#pragma unroll
    for (int k = 0; k < BinScan<kGridThreads>::BPT; ++k) {
        const int b = scan.top - k;
        if (want(b)) mine += scan.c[k];
        if (b > a && b < blo) gapm += scan.m[k];
    }
    mine = wave_sum(mine);
    gapm = wave_sum(gapm);
    if (lane == 0) {
        s_cnt[wid] = mine;
        sc.wsum[wid] = gapm;
    }
    __syncthreads();
    uint32_t C = 0u;
    unsigned long long gap = 0ull;
    for (int w = 0; w < kWaves; ++w) {
        C += s_cnt[w];
        gap += sc.wsum[w];
    }
    __syncthreads();   // sc.wsum is rewritten below
    const bool ranged = C > (uint32_t)kCandLds;
    if (!ranged) {
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            SampleCtl& c = *p.ctl;
            c.mode = 0;
            c.cut_found = s1.found;
            c.total = s1.total;
        }
        pick_tied<kGridThreads>(bk, tied_bm, lo, hi, s_tkey, &s_ntied, sc);
        const int nt = s_ntied;
        if (blockIdx.x == 0 && threadIdx.x < kTiedSlots) {
            if (threadIdx.x == 0) p.ctl->ntied = nt;
            if ((int)threadIdx.x < nt) p.ctl->tkey[threadIdx.x] = s_tkey[threadIdx.x];
        }
        compact<kGridThreads>(p, key0, [&](uint32_t key) { return want((int)(key >> 20)); },
                              s_tkey, nt, offs, tsum);
        return;
    }
    // The segments' key ranges, from the level-0 key extremes the scan holds:
    // A, bin a; B, the non-empty bins of [blo, hi] (min / max over the block).
    uint32_t bmn = 0xFFFFFFFFu, bmx = 0u;
#pragma unroll
    for (int k = 0; k < BinScan<kGridThreads>::BPT; ++k) {
        const int b = scan.top - k;
        if (b >= blo && b <= hi && scan.c[k]) {
            bmn = min(bmn, scan.kmn[k]);
            bmx = max(bmx, scan.kmx[k]);
        }
        if (b == a) {   // one thread
            s_amn = scan.c[k] ? scan.kmn[k] : 1u;
            s_amx = scan.c[k] ? scan.kmx[k] : 0u;
        }
    }
    bmn = wave_minmax<false>(bmn);
    bmx = wave_minmax<true>(bmx);
    if (lane == 0) {
        s_cnt[wid] = bmn;
        offs[wid] = bmx;
    }
    __syncthreads();
    for (int w = 0; w < kWaves; ++w) {
        bmn = min(bmn, s_cnt[w]);
        bmx = max(bmx, offs[w]);
    }
    const uint32_t amn = s_amn, amx = s_amx;
    const bool a_some = amn <= amx;
    const int a_shift = a_some ? seg_shift(amn, amx) : 0;
    const int b_shift = bmn <= bmx ? seg_shift(bmn, bmx) : 0;
    SampleCtl seg;
    seg.a_shift = a_shift;
    seg.b_shift = b_shift;
    seg.a_lo = amn;
    seg.a_base = (amn >> a_shift) << a_shift;
    seg.a_end = a_some ? (unsigned long long)amx + 1ull : 0ull;
    seg.b_lo = bmn <= bmx ? bmn : 1u;
    seg.b_base = bmn <= bmx ? (bmn >> b_shift) << b_shift : 0u;
    seg.b_end = bmn <= bmx ? (unsigned long long)bmx + 1ull : 0ull;
    seg.gap = gap;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        SampleCtl& c = *p.ctl;
        c.mode = 1;
        c.cut_found = s1.found;
        c.a_shift = seg.a_shift;
        c.b_shift = seg.b_shift;
        c.a_lo = seg.a_lo;
        c.a_base = seg.a_base;
        c.a_end = seg.a_end;
        c.b_lo = seg.b_lo;
        c.b_base = seg.b_base;
        c.b_end = seg.b_end;
        c.above = above_hi;
        c.gap = gap;
        c.total = s1.total;
    }
    // the range histogram: counts, masses and key extremes of its buckets
    const Buckets rb = range_buckets(p, seg);
    for (int b = threadIdx.x; b < kBins; b += kGridThreads) {
        hc[b] = 0u;
        hm[b] = 0ull;
        hlo[b] = 0xFFFFFFFFu;
        hhi[b] = 0u;
    }
    __syncthreads();
    const int q_first = blockIdx.x * kGridThreads + threadIdx.x;
    for (int qw = q_first - lane; 4 * qw < n; qw += T) {   // wave-uniform: hist_add
        const int q = qw + lane;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = 4 * q + k;
            const uint32_t key = q == q_first ? key0[k] : i < n ? __float_as_uint(p.probs[i]) : 0u;
            const int d0 = rb.of(key);
            const bool ok = i < n && d0 < kBins;
            const int d = ok ? d0 : 0;
            const int lead = hist_add(ok, d, key, ok ? mass_of(key) : 0ull, hc, hm);
            key_minmax(ok, d, key, lead, hlo, hhi);
        }
    }
    __syncthreads();
    for (int b = threadIdx.x; b < kBins; b += kGridThreads) {
        if (hc[b]) {
            atomicAdd(&p.h1cnt[b], hc[b]);
            atomicMin(&p.h1min[b], hlo[b]);
            atomicMax(&p.h1max[b], hhi[b]);
        }
        if (hm[b]) atomicAdd(&p.h1mass[b], hm[b]);
    }
}

namespace {

// This lane's matches of key K among tokens [a, b) (a a multiple of 4): 4
// consecutive tokens a lane, kNthUnroll 16-byte loads in flight.  The keys
// are read in whole quads: the probability region is padded to 256 bytes.
__device__ __forceinline__ uint32_t count_key(const uint32_t* kb, int a, int b, uint32_t K) {
    const int lane = threadIdx.x & 63;
    uint32_t c = 0u;
    for (int i0 = a + 4 * lane; i0 < b; i0 += 256 * kNthUnroll) {
        uint4 v[kNthUnroll];
#pragma unroll
        for (int u = 0; u < kNthUnroll; ++u) {
            const int i = i0 + 256 * u;
            v[u] = i < b ? *reinterpret_cast<const uint4*>(kb + i) : make_uint4(~K, ~K, ~K, ~K);
        }
#pragma unroll
        for (int u = 0; u < kNthUnroll; ++u) {
            const int i = i0 + 256 * u;
            c += (uint32_t)(v[u].x == K) + (uint32_t)(v[u].y == K && i + 1 < b) +
                 (uint32_t)(v[u].z == K && i + 2 < b) + (uint32_t)(v[u].w == K && i + 3 < b);
        }
    }
    return c;
}

// The j-th (1-based) token in index order whose key is K, or -1, without
// per-chunk counts (a tied bucket beyond the kTiedSlots counted): rounds of
// 16-way narrowing (the range splits into 16 parts of whole quads, a wave
// counts each, and the part holding the j-th becomes the range) until at
// most 256 tokens are left, which one wave finishes.  Whole block.
__device__ int nth_with_key(const float* probs, int n, uint32_t K, unsigned long long j,
                            SelScratch& sc, int* s_id) {
    constexpr int NW = kSelThreads / 64;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const uint32_t* kb = reinterpret_cast<const uint32_t*>(probs);
    int lo = 0, hi = n;
    unsigned long long r = j;
    if (threadIdx.x == 0) *s_id = -1;
    while (hi - lo > 256) {
        const int per = ((hi - lo + NW - 1) / NW + 3) & ~3;
        const int a = min(hi, lo + wid * per), b = min(hi, a + per);
        uint32_t c = count_key(kb, a, b, K);
        c = wave_sum(c);
        if (lane == 0) sc.wsum[wid] = c;
        __syncthreads();
        unsigned long long before = 0ull;
        int part = -1;
        for (int w = 0; w < NW; ++w) {
            const unsigned long long cw = sc.wsum[w];
            if (part < 0) {
                if (r <= before + cw) part = w;
                else before += cw;
            }
        }
        __syncthreads();   // wsum is written again next round
        if (part < 0) return -1;   // block-uniform: fewer than j such tokens
        lo = min(hi, lo + part * per);
        hi = min(hi, lo + per);
        r -= before;
    }
    if (wid == 0) {
        const int i = lo + 4 * lane;
        const uint4 v = i < hi ? *reinterpret_cast<const uint4*>(kb + i)
                               : make_uint4(~K, ~K, ~K, ~K);
        const uint32_t m = (uint32_t)(v.x == K) | (uint32_t)(v.y == K && i + 1 < hi) << 1 |
                           (uint32_t)(v.z == K && i + 2 < hi) << 2 |
                           (uint32_t)(v.w == K && i + 3 < hi) << 3;
        const uint32_t c = (uint32_t)__popc(m);
        const uint32_t S = wave_incl_sum(c);
        if ((unsigned long long)(S - c) < r && r <= (unsigned long long)S) {
            uint32_t k = (uint32_t)(r - (S - c)), e = 0u;   // the k-th set bit of m
            for (; e < 4u; ++e)
                if (((m >> e) & 1u) && --k == 0u) break;
            *s_id = i + (int)e;
        }
    }
    __syncthreads();
    const int id = *s_id;
    __syncthreads();
    return id;
}

// The j-th (1-based) token in index order whose key is K, from the
// per-chunk counts of its slot: a block scan over the chunk counts finds
// the chunk, and one token a thread (1024 threads: one chunk) finds the
// token in it.  Whole block; -1 if fewer than j.
__device__ int nth_in_chunks(const SampleParams& p, int slot, uint32_t K, unsigned long long j,
                             SelScratch& sc, int* s_id) {
    const int n = p.n, nchunk = (n + 1023) >> 10;
    const uint32_t* cnt = p.tcnt + slot * nchunk;
    if (threadIdx.x == 0) {
        sc.chunk = -1;
        *s_id = -1;
    }
    __syncthreads();
    unsigned long long base = 0ull;
    for (int c0 = 0; c0 < nchunk; c0 += kSelThreads) {   // block-uniform
        const int c = c0 + (int)threadIdx.x;
        const uint32_t v = c < nchunk ? cnt[c] : 0u;
        const unsigned long long ex = base + block_excl_scan<kSelThreads>(v, sc.wsum);
        if (v && ex < j && j <= ex + v) {
            sc.chunk = c;
            sc.rem = j - ex;
        }
        base += sc.wsum[kSelThreads / 64 - 1];
        __syncthreads();
    }
    const int chunk = sc.chunk;
    if (chunk < 0) return -1;   // block-uniform
    const unsigned long long r = sc.rem;
    const int i = (chunk << 10) + (int)threadIdx.x;
    const uint32_t hit = i < n && __float_as_uint(p.probs[i]) == K ? 1u : 0u;
    const unsigned long long ex = block_excl_scan<kSelThreads>(hit, sc.wsum);
    if (hit && ex + 1ull == r) *s_id = i;
    __syncthreads();
    const int id = *s_id;
    __syncthreads();
    return id;
}

}  // namespace

// Mode 1 only: the range histogram narrowed as the gather kernel did the
// level-0 one -- the bucket of the cutoff and the buckets the draw can
// reach -- and their untied tokens compacted (one quad a thread).
__global__ __launch_bounds__(kSelThreads) void sample_narrow_kernel(SampleParams p) {
    constexpr int kWaves = kSelThreads / 64;
    __shared__ SelScratch sc;
    __shared__ BinSel s1, s2;
    __shared__ uint32_t tied_bm[kBins / 32];
    __shared__ uint32_t offs[kWaves * 4], tsum[kWaves * kTiedSlots], s_tkey[kTiedSlots];
    __shared__ int s_ntied;
    SampleCtl& ctl = *p.ctl;
    if (ctl.mode == 0) return;
    uint32_t key0[4];
    first_quad<kSelThreads>(p, key0);
    const Buckets bk = range_buckets(p, ctl);
    const unsigned long long t1 = target_top_p(p.top_p);
    BinScan<kSelThreads> scan;
    scan.load_tied(bk, ctl.above, sc, tied_bm);
    if (ctl.cut_found) {
        scan.find(t1, s1, sc);
    } else {
        if (threadIdx.x == 0) s1.found = 0;
        __syncthreads();
    }
    unsigned long long tlo, thi;
    draw_bounds(s1, tied_bm, draw_of(p), t1, ctl.total, tlo, thi);
    scan.find(thi, s2, sc);
    const int lo = s2.found ? s2.bin : 0;
    scan.find(tlo, s2, sc);
    const int hi = s2.found ? s2.bin : kBins - 1;
    const int b1 = s1.found ? s1.bin : -1;
    pick_tied<kSelThreads>(bk, tied_bm, lo, hi, s_tkey, &s_ntied, sc);
    const int nt = s_ntied;
    if (blockIdx.x == 0 && threadIdx.x < kTiedSlots) {
        if (threadIdx.x == 0) ctl.ntied = nt;
        if ((int)threadIdx.x < nt) ctl.tkey[threadIdx.x] = s_tkey[threadIdx.x];
    }
    compact<kSelThreads>(p, key0, [&](uint32_t key) {
        const int b = bk.of(key);
        return (b == b1 || (b >= lo && b <= hi)) && b < kBins && !is_tied(tied_bm, b);
    }, s_tkey, nt, offs, tsum);
}

// Positions of the cutoff (its inclusive mass) and of the draw (its token)
// in the gather kernel's buckets, each: a bucket of one token (read off the
// histogram / the candidates), a tied bucket (by rank: the cutoff's mass
// directly, the draw's token from the per-chunk counts), at most 64
// candidates (one wave sorts them), or the levels below the bucket over its
// candidates (in LDS when they fit).  One workgroup.
__global__ __launch_bounds__(kSelThreads) void sample_select_kernel(SampleParams p) {
    __shared__ uint2 lc[kCandLds];
    __shared__ LevelHist H;
    __shared__ SelScratch sc;
    __shared__ BinSel s0, s1, bs;
    __shared__ uint32_t tied_bm[kBins / 32];
    __shared__ int s_id;
    __shared__ unsigned long long s_cum;
    const SampleCtl& ctl = *p.ctl;
    const int mode = ctl.mode;
    const Buckets bk = mode ? range_buckets(p, ctl) : level0_buckets(p);
    // read before the first barrier: thread 0 advances the draw index at the end
    const float u = draw_of(p);
    const unsigned long long t1 = target_top_p(p.top_p);
    BinScan<kSelThreads> scan0;
    scan0.load_tied(bk, mode ? ctl.above : 0ull, sc, tied_bm);
    if (ctl.cut_found) {
        scan0.find(t1, s1, sc);       // the cutoff's bucket
    } else {
        if (threadIdx.x == 0) s1.found = 0;
        __syncthreads();
    }
    const int C = (int)ctl.ccount;

    // Few candidates (the usual nucleus of a peaked distribution): wave 0
    // sorts them by key and gives each its inclusive running mass (the mass
    // of all buckets above its bucket, from the histogram, plus the running
    // mass inside its bucket).
    const bool few = C <= 64;
    const int lane = threadIdx.x & 63;
    int w_id = 0, w_bin = -1;
    unsigned long long w_cum = 0ull;
    bool w_valid = false;
    if (few) {
        {
            unsigned long long run = scan0.excl;
#pragma unroll
            for (int k = 0; k < BinScan<kSelThreads>::BPT; ++k) {
                H.mass[scan0.top - k] = run;
                run += scan0.m[k];
            }
        }
        __syncthreads();
        if (threadIdx.x < 64) {
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
            w_valid = (sk >> 63) != 0ull;
            const uint32_t key = (uint32_t)(sk >> 24);
            w_id = (int)(kIdMask - (uint32_t)(sk & kIdMask));
            w_bin = w_valid ? bk.of(key) : -1;
            if (w_bin >= kBins) w_bin = -1;   // not a candidate's key: never taken
            const unsigned long long m = w_valid ? mass_of(key) : 0ull;
            // inclusive running mass inside each bucket (buckets are contiguous runs)
            const unsigned long long S = wave_incl_sum(m);
            const int prev_bin = __shfl_up(w_bin, 1, 64);
            const bool head = w_valid && (lane == 0 || prev_bin != w_bin);
            const unsigned long long heads = __ballot(head) & ((2ull << lane) - 1ull);
            const int start = heads ? 63 - __clzll((long long)heads) : 0;
            const unsigned long long before = __shfl(S, start > 0 ? start - 1 : 0, 64);
            w_cum = (w_bin >= 0 ? H.mass[w_bin] : 0ull) + S - (start > 0 ? before : 0ull);
        }
    }
    const uint2* cand = p.cand;
    if (!few && C <= kCandLds) {
        for (int c = threadIdx.x; c < C; c += kSelThreads) lc[c] = p.cand[c];
        cand = lc;
    }
    __syncthreads();

    // the cutoff: its inclusive mass
    unsigned long long cum = ctl.total;
    if (s1.found) {
        if (s1.cnt == 1u) {
            cum = s1.incl;
        } else if (is_tied(tied_bm, s1.bin)) {
            const unsigned long long m = tied_mass(s1);
            cum = s1.excl + tied_rank(s1.excl, t1, m) * m;
        } else if (few) {
            if (threadIdx.x < 64) {
                const unsigned long long hit = __ballot(w_valid && w_bin == s1.bin && w_cum >= t1);
                const unsigned long long c = hit ? __shfl(w_cum, __ffsll((long long)hit) - 1, 64)
                                                 : s1.incl;
                if (threadIdx.x == 0) s_cum = c;
            }
            __syncthreads();
            cum = s_cum;
        } else {
            (void)select_in_bin(cand, C, bk, s1.bin, s1.cnt, s1.excl, t1, H, sc, bs, cum);
        }
    }
    // the draw
    const unsigned long long t2 = target_draw(u, cum);
    scan0.find(t2, s0, sc);
    int id = -1;
    if (s0.found) {
        if (is_tied(tied_bm, s0.bin)) {
            const uint32_t K = bk.kmin[s0.bin];
            const unsigned long long j = tied_rank(s0.excl, t2, tied_mass(s0));
            int slot = -1;
            for (int s = 0; s < ctl.ntied && s < kTiedSlots; ++s)
                if (slot < 0 && ctl.tkey[s] == K) slot = s;
            id = slot >= 0 ? nth_in_chunks(p, slot, K, j, sc, &s_id)
                           : nth_with_key(p.probs, p.n, K, j, sc, &s_id);
        } else if (few) {
            if (threadIdx.x == 0) s_id = -1;
            __syncthreads();
            if (threadIdx.x < 64) {
                const unsigned long long hit2 = __ballot(w_valid && w_cum >= t2);
                const int chosen = __shfl(w_id, hit2 ? __ffsll((long long)hit2) - 1 : 0, 64);
                if (threadIdx.x == 0 && hit2) s_id = chosen;
            }
            __syncthreads();
            id = s_id;
        } else if (s0.cnt == 1u) {
            id = only_in_bin(cand, C, bk, s0.bin, &s_id);
        } else {
            unsigned long long c2 = 0ull;
            id = select_in_bin(cand, C, bk, s0.bin, s0.cnt, s0.excl, t2, H, sc, bs, c2);
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

// probabilities, block maxima and exp-sums, the level-0 and range
// histograms (count, mass, key min and max), the control block, the tied-key
// chunk counts, candidates
constexpr size_t sample_ws_bytes(size_t n) {
    return (n * 4 + 255) / 256 * 256 + 2 * ((kMaxBlocks * 4 + 255) / 256 * 256) +
           2 * (3 * ((kBins * 4 + 255) / 256 * 256) + (kBins * 8 + 255) / 256 * 256) + 256 +
           (kTiedSlots * 4 * ((n + 1023) / 1024) + 255) / 256 * 256 + (n * 8 + 255) / 256 * 256;
}

size_t sample_workspace_bytes(int n) { return sample_ws_bytes((size_t)n); }

// Scratch of sltx_sample_top_p_noalloc: the sampler's workspace for up to
// kSampleNoAllocMaxN logits (3,315,968 bytes), in a file-scope device array,
// so that entry point allocates nothing.  Each GPU holds its own copy until
// the process ends, and every call on that GPU shares it (the scale kernel
// clears the counters each call; the other regions are written before they
// are read).  In host code `scratch` only names the symbol: kernels are given
// the device address resolved per device below.
static_assert(sample_ws_bytes(kSampleNoAllocMaxN) == 3315968, "noalloc scratch size");
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
    p.h0min = reinterpret_cast<uint32_t*>(w);
    w += up256(kBins * 4);
    p.h0max = reinterpret_cast<uint32_t*>(w);
    w += up256(kBins * 4);
    p.h1cnt = reinterpret_cast<uint32_t*>(w);
    w += up256(kBins * 4);
    p.h1mass = reinterpret_cast<unsigned long long*>(w);
    w += up256(kBins * 8);
    p.h1min = reinterpret_cast<uint32_t*>(w);
    w += up256(kBins * 4);
    p.h1max = reinterpret_cast<uint32_t*>(w);
    w += up256(kBins * 4);
    static_assert(sizeof(SampleCtl) <= 256, "control block");
    p.ctl = reinterpret_cast<SampleCtl*>(w);
    w += 256;
    p.tcnt = reinterpret_cast<uint32_t*>(w);
    w += up256((size_t)kTiedSlots * 4 * ((n + 1023) / 1024));
    p.cand = reinterpret_cast<uint2*>(w);
    const int G = grid_blocks(p.n);
    hipLaunchKernelGGL(sample_scale_kernel, dim3(G), dim3(kGridThreads), 0, st, p);
    hipLaunchKernelGGL(sample_prob_kernel, dim3(G), dim3(kGridThreads), 0, st, p);
    hipLaunchKernelGGL(sample_gather_kernel, dim3(G), dim3(kGridThreads), 0, st, p);
    const int Gn = std::min(kMaxBlocks, (p.n + 4 * kSelThreads - 1) / (4 * kSelThreads));
    hipLaunchKernelGGL(sample_narrow_kernel, dim3(Gn), dim3(kSelThreads), 0, st, p);
    hipLaunchKernelGGL(sample_select_kernel, dim3(1), dim3(kSelThreads), 0, st, p);
    return hipGetLastError();
}

}  // namespace sltx
