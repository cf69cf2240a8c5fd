// q4_sample.hip -- token selection after the lm_head, on the GPU.
//
// argmax (Ops.swift:757-781) and temperature / top-p / repetition-penalty
// sampling (sample, Ops.swift:785-810; sampleFromLogits, Ops.swift:2060-2098),
// which the reference runs on the CPU over all vocabulary logits per token.
// One workgroup of 1024 threads; the logits are read from HBM once into an fp32
// workspace (L2-resident, 0.5 MB for 128256 tokens).
//
// The probabilities follow the reference's fp32 steps: penalty (divide
// positive, multiply non-positive logits of the distinct seen tokens), divide
// by temperature, softmax (max, exp, sum, divide).  The softmax denominator is
// a fixed-order sum (per-thread strided sums, then a halving tree) instead of
// a sequential loop.
// The nucleus and the draw use exact running sums instead of the reference's
// sequential fp32 ones: each probability p carries the integer mass
// floor(p * 2^52), and in the order (p descending, id ascending; the
// reference's sort is unstable) the cutoff is the first token whose inclusive
// running mass reaches ceil(top_p * 2^52) (all tokens if none does), and the
// chosen token is the first whose inclusive running mass reaches
// ceil(u * mass at the cutoff) -- the reference's "r -= p until r <= 0".
// Nothing is sorted: both positions are weighted radix selects over the key
// (p bits, then 2^24-1-id), 8 bits a pass, with per-digit counts and masses
// in LDS; a pass stops early once its digit holds a single token.
#include "q4_common.hpp"
#include "q4_launch.hpp"

namespace sltx {
namespace {

constexpr int kSampleThreads = 1024;
constexpr int kSelPasses = 7;              // 4 over the probability bits, 3 over the id
constexpr uint32_t kIdMask = 0xFFFFFFu;    // ids < 2^24

__device__ __forceinline__ float load_logit(const void* p, int dtype, int i) {
    if (dtype == kF32) return reinterpret_cast<const float*>(p)[i];
    return h2f(reinterpret_cast<const uint16_t*>(p)[i]);
}

// block reductions (fixed order: per-thread partials, then a tree over LDS)
template <typename T, typename Op>
__device__ T block_reduce(T v, T* red, Op op) {
    red[threadIdx.x] = v;
    __syncthreads();
    for (int s = kSampleThreads / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) red[threadIdx.x] = op(red[threadIdx.x], red[threadIdx.x + s]);
        __syncthreads();
    }
    const T r = red[0];
    __syncthreads();
    return r;
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

// digit d of the order key: probability bits 31..0, then lo = 2^24-1-id bits
// 23..0, 8 bits a digit, most significant first
__device__ __forceinline__ uint32_t digit_of(int d, uint32_t key, uint32_t lo) {
    return d < 4 ? (key >> (24 - 8 * d)) & 255u : (lo >> (16 - 8 * (d - 4))) & 255u;
}

__device__ __forceinline__ unsigned long long wave_sum_u64(unsigned long long v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

struct SelHist {
    uint32_t cnt[kSelPasses][256];
    unsigned long long mass[kSelPasses][256];
    uint32_t pk[kSelPasses], pl[kSelPasses];   // prefixes each pass was counted under
    int valid[kSelPasses];
};

struct SelState {
    uint32_t pk, mk, pl, ml;     // key / lo prefix and mask chosen so far
    unsigned long long above;    // mass of the tokens before the current digit
    unsigned long long cum;      // found: inclusive mass at the token; else the total
    int found, done, idx;
};

// Weighted select: the first token, in key-descending order, whose inclusive
// running mass reaches target.  A pass's histogram is kept and reused by a
// later select that reaches the same prefix.  Whole block; ends synchronised.
__device__ void weighted_select(const float* pr, int n, unsigned long long target, SelState& S,
                                SelHist& H) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    if (tid == 0) {
        S.pk = S.mk = S.pl = S.ml = 0u;
        S.above = S.cum = 0ull;
        S.found = S.done = 0;
        S.idx = -1;
    }
    __syncthreads();
    for (int d = 0; d < kSelPasses; ++d) {
        const uint32_t pk = S.pk, mk = S.mk, pl = S.pl, ml = S.ml;
        const bool cached = H.valid[d] && H.pk[d] == pk && H.pl[d] == pl;
        __syncthreads();   // everyone has read S before thread 0 updates it
        if (!cached) {
            for (int b = tid; b < 256; b += kSampleThreads) {
                H.cnt[d][b] = 0u;
                H.mass[d][b] = 0ull;
            }
            __syncthreads();
            // wave-uniform loop: every lane runs every iteration (the
            // aggregation below shuffles across the whole wave)
            for (int i0 = tid & ~63; i0 < n; i0 += kSampleThreads) {
                const int i = i0 + lane;
                const uint32_t key = i < n ? __float_as_uint(pr[i]) : 0u;
                const uint32_t lo = kIdMask - (uint32_t)i;
                const bool act = i < n && (key & mk) == pk && (lo & ml) == pl;
                const uint32_t b = digit_of(d, key, lo);
                const unsigned long long m = mass_of(key);
                if (d == 0) {
                    // the first digit (sign + exponent bits) is shared by most
                    // of a wave: one atomic per distinct digit
                    unsigned long long rem = __ballot(act);
                    while (rem) {
                        const int leader = __ffsll((long long)rem) - 1;
                        const uint32_t bl = __builtin_amdgcn_readlane(b, leader);
                        const bool mine = act && b == bl;
                        const unsigned long long same = __ballot(mine);
                        const unsigned long long ms = wave_sum_u64(mine ? m : 0ull);
                        if (lane == leader) {
                            atomicAdd(&H.cnt[d][bl], (uint32_t)__popcll(same));
                            atomicAdd(&H.mass[d][bl], ms);
                        }
                        rem &= ~same;
                    }
                } else if (act) {
                    atomicAdd(&H.cnt[d][b], 1u);
                    if (m) atomicAdd(&H.mass[d][b], m);
                }
            }
            __syncthreads();
        }
        if (tid == 0) {
            if (!cached) {
                H.valid[d] = 1;
                H.pk[d] = pk;
                H.pl[d] = pl;
            }
            unsigned long long above = S.above;
            int sel = -1;
            for (int b = 255; b >= 0; --b) {
                if (!H.cnt[d][b]) continue;
                const unsigned long long m = H.mass[d][b];
                if (above + m >= target) {
                    sel = b;
                    break;
                }
                above += m;
            }
            if (sel < 0) {          // target beyond the total mass
                S.cum = above;
                S.done = 1;
            } else {
                if (d < 4) {
                    S.pk = pk | ((uint32_t)sel << (24 - 8 * d));
                    S.mk = mk | (255u << (24 - 8 * d));
                } else {
                    S.pl = pl | ((uint32_t)sel << (16 - 8 * (d - 4)));
                    S.ml = ml | (255u << (16 - 8 * (d - 4)));
                }
                S.above = above;
                S.cum = above + H.mass[d][sel];
                if (H.cnt[d][sel] == 1u) {
                    S.found = 1;
                    S.done = 1;
                }
            }
        }
        __syncthreads();
        if (S.done) break;
    }
    if (S.found) {   // the one token under the final prefix
        const uint32_t pk = S.pk, mk = S.mk, pl = S.pl, ml = S.ml;
        for (int i = tid; i < n; i += kSampleThreads) {
            const uint32_t key = __float_as_uint(pr[i]);
            const uint32_t lo = kIdMask - (uint32_t)i;
            if ((key & mk) == pk && (lo & ml) == pl) S.idx = i;
        }
        __syncthreads();
    }
}

}  // namespace

// argmax: first index of the maximum (NaNs never win; NaN at index 0 -> 0).
__global__ __launch_bounds__(kSampleThreads) void argmax_kernel(const void* logits, int dtype,
                                                                int n, int32_t* out) {
    __shared__ float rv[kSampleThreads];
    __shared__ int ri[kSampleThreads];
    float bv = 0.0f;
    int bi = -1;
    for (int i = threadIdx.x; i < n; i += kSampleThreads) {
        const float v = load_logit(logits, dtype, i);
        if (v != v) continue;
        if (bi < 0 || v > bv) {   // strided increasing i: first maximum per thread
            bv = v;
            bi = i;
        }
    }
    rv[threadIdx.x] = bv;
    ri[threadIdx.x] = bi;
    __syncthreads();
    for (int s = kSampleThreads / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            const float ov = rv[threadIdx.x + s];
            const int oi = ri[threadIdx.x + s];
            const int mi = ri[threadIdx.x];
            if (oi >= 0 && (mi < 0 || ov > rv[threadIdx.x] || (ov == rv[threadIdx.x] && oi < mi))) {
                rv[threadIdx.x] = ov;
                ri[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float v0 = load_logit(logits, dtype, 0);
        *out = (v0 != v0 || ri[0] < 0) ? 0 : ri[0];
    }
}

__global__ __launch_bounds__(kSampleThreads) void sample_kernel(SampleParams p) {
    __shared__ float redf[kSampleThreads];
    __shared__ SelHist hist;
    __shared__ SelState sel;
    const int n = p.n;
    float* pr = p.probs;

    // 1. fp32 copy of the logits; clear the seen-token bitmap and the
    //    histogram cache
    for (int i = threadIdx.x; i < n; i += kSampleThreads) pr[i] = load_logit(p.logits, p.dtype, i);
    for (int w = threadIdx.x; w < (n + 31) / 32; w += kSampleThreads) p.bitmap[w] = 0u;
    if (threadIdx.x < kSelPasses) hist.valid[threadIdx.x] = 0;
    __syncthreads();
    // 2. repetition penalty, once per distinct token (the reference's Set)
    for (int j = threadIdx.x; j < p.n_seen; j += kSampleThreads) {
        const int t = p.seen[j];
        if (t < 0 || t >= n) continue;
        const uint32_t bit = 1u << (t & 31);
        if (atomicOr(&p.bitmap[t >> 5], bit) & bit) continue;
        const float l = pr[t];
        pr[t] = l > 0.0f ? l / p.penalty : l * p.penalty;
    }
    __syncthreads();
    // 3. temperature, max
    float mx = -3.402823466e38f;   // -greatestFiniteMagnitude
    for (int i = threadIdx.x; i < n; i += kSampleThreads) {
        const float l = pr[i] / p.temperature;
        pr[i] = l;
        mx = fmaxf(mx, l);
    }
    mx = block_reduce(mx, redf, [](float a, float b) { return fmaxf(a, b); });
    // 4. exp and sum, 5. normalise
    float sm = 0.0f;
    for (int i = threadIdx.x; i < n; i += kSampleThreads) {
        const float e = expf(pr[i] - mx);
        pr[i] = e;
        sm += e;
    }
    sm = block_reduce(sm, redf, [](float a, float b) { return a + b; });
    for (int i = threadIdx.x; i < n; i += kSampleThreads) pr[i] = pr[i] / sm;
    __syncthreads();

    // 6. the nucleus: first token whose running mass reaches top_p
    const double tp = fmin((double)p.top_p, 4.0);
    weighted_select(pr, n, (unsigned long long)ceil(tp * 0x1p52), sel, hist);
    const unsigned long long cum = sel.cum;   // at the cutoff, or the total
    __syncthreads();
    // 7. the draw: first token whose running mass reaches u * cum
    weighted_select(pr, n, (unsigned long long)ceil((double)p.u * (double)cum), sel, hist);
    if (!sel.found) {   // only for non-finite probabilities: the first token
        __syncthreads();
        weighted_select(pr, n, 0ull, sel, hist);
    }
    if (threadIdx.x == 0) *p.out = sel.idx < 0 ? 0 : sel.idx;
}

size_t sample_workspace_bytes(int n) {
    const size_t probs = ((size_t)n * 4 + 255) / 256 * 256;
    const size_t bitmap = (((size_t)n + 31) / 32 * 4 + 255) / 256 * 256;
    return probs + bitmap;
}

hipError_t launch_argmax(const void* logits, int dtype, int n, int32_t* out, hipStream_t st) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kSampleThreads), 0, st, logits, dtype, n, out);
    return hipGetLastError();
}

hipError_t launch_sample(SampleParams p, void* ws, hipStream_t st) {
    char* w = static_cast<char*>(ws);
    const size_t probs = ((size_t)p.n * 4 + 255) / 256 * 256;
    p.probs = reinterpret_cast<float*>(w);
    p.bitmap = reinterpret_cast<uint32_t*>(w + probs);
    hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(kSampleThreads), 0, st, p);
    return hipGetLastError();
}

}  // namespace sltx
