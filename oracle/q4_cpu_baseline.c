/* q4_cpu_baseline.c -- CPU baselines of the 4-bit dequant matmul (test and
 * benchmark infrastructure: timed beside the GPU path, never shipped).
 * Built with -mavx2 -mfma -mf16c: fp16 <-> fp32 are the F16C instructions.
 *
 * Semantics of swift-ltx's matmul_q4 (Kernels.swift:444-620): w[n,k] =
 * s[n,k/g] * q[n,k] + b[n,k/g] (Kernels.swift:392-395), nibble k of row n =
 * bits 4*(k%8) of word k/8, fp32 accumulation, fp16 (round to nearest even)
 * store.  Swift is not installed here, so these are C restatements:
 *
 *   cpu_q4_scalar  one thread, the loop shape of the reference's only CPU
 *                  matmul (matmulCPU, LlamaModel.swift:478-493: for m, for n,
 *                  for k, one fp32 sum over an fp32 copy of the x row) with
 *                  the weight dequantized inline, the group's scale and bias
 *                  read once per group; built without auto-vectorization.
 *   cpu_q4_simd    the same product with an explicit 8-wide fp32 vector
 *                  (Swift's SIMD8<Float>): each packed word is dequantized as
 *                  one 8-lane vector (shift, mask, convert, fma with the
 *                  group's scale and bias) and multiplied into an 8-lane
 *                  accumulator, summed across lanes at the end of the row;
 *                  rows are split over pthreads.  For M > 1 a row is
 *                  dequantized once and dotted with every x row.
 */
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef float f8 __attribute__((vector_size(32)));
typedef int32_t i8v __attribute__((vector_size(32)));

#if defined(__F16C__)
#include <immintrin.h>
/* hardware conversions (x86 F16C), as Swift's Float(Float16) compiles to */
static inline float f16_to_f32(uint16_t h) { return _cvtsh_ss(h); }
static inline uint16_t f32_to_f16(float f) { return (uint16_t)_cvtss_sh(f, 0); }   /* nearest even */
#else
static inline float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {   /* subnormal: normalize */
            int e = -1;
            uint32_t m = man;
            do { ++e; m <<= 1; } while ((m & 0x400u) == 0);
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline uint16_t f32_to_f16(float f) {   /* round to nearest even */
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t a = x & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);          /* NaN */
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);         /* overflow -> inf */
    if (a < 0x38800000u) {                                            /* subnormal or zero */
        if (a < 0x33000000u) return (uint16_t)sign;
        const uint32_t m = (a & 0x7fffffu) | 0x800000u;
        const int shift = 113 - (int)(a >> 23) + 13;
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((a - 0x38000000u) >> 13);
    const uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
}
#endif

/* ------------------------------------------------------------- scalar --- */

__attribute__((optimize("no-tree-vectorize")))
void cpu_q4_scalar(const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                   uint16_t* y, int64_t M, int64_t N, int64_t K, int64_t g) {
    const int64_t packed = K / 8, groups = K / g;
    float* xf = (float*)malloc(sizeof(float) * (size_t)K);
    if (!xf) return;
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t k = 0; k < K; ++k) xf[k] = f16_to_f32(x[m * K + k]);   /* the fp32 row */
        for (int64_t n = 0; n < N; ++n) {
            const uint32_t* wr = w + n * packed;
            float sum = 0.0f;
            for (int64_t gi = 0; gi < groups; ++gi) {   /* k in order, one group at a time */
                const float sc = f16_to_f32(s[n * groups + gi]), bi = f16_to_f32(b[n * groups + gi]);
                for (int64_t k = gi * g; k < (gi + 1) * g; ++k) {
                    const float q = (float)((wr[k >> 3] >> (4 * (k & 7))) & 0xfu);
                    sum += xf[k] * (q * sc + bi);
                }
            }
            y[m * N + n] = f32_to_f16(sum);
        }
    }
    free(xf);
}

/* --------------------------------------------------------------- SIMD --- */

typedef struct {
    const float* xf;          /* [M, K] fp32 copy of x */
    const uint32_t* w;
    const uint16_t *s, *b;
    uint16_t* y;
    int64_t M, N, K, g, n0, n1;
} simd_job;

static inline float hsum8(f8 v) {
    return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
}

/* one packed word -> 8 fp32 weights: q * s + b, lane i = nibble i */
static inline f8 dequant8(uint32_t word, f8 sv, f8 bv) {
    const i8v shifts = {0, 4, 8, 12, 16, 20, 24, 28};
    const i8v wv = {(int32_t)word, (int32_t)word, (int32_t)word, (int32_t)word,
                    (int32_t)word, (int32_t)word, (int32_t)word, (int32_t)word};
    const i8v q = (i8v)((uint32_t __attribute__((vector_size(32))))wv >>
                        (uint32_t __attribute__((vector_size(32))))shifts) & 0xf;
    return __builtin_convertvector(q, f8) * sv + bv;
}

static void* simd_worker(void* arg) {
    simd_job* j = (simd_job*)arg;
    const int64_t K = j->K, packed = K / 8, groups = K / j->g, wpg = j->g / 8;
    f8* wrow = (f8*)aligned_alloc(32, sizeof(f8) * (size_t)packed);
    for (int64_t n = j->n0; n < j->n1; ++n) {
        const uint32_t* wr = j->w + n * packed;
        if (j->M == 1) {
            const f8* xv = (const f8*)j->xf;
            f8 acc = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int64_t gi = 0; gi < groups; ++gi) {
                const float sc = f16_to_f32(j->s[n * groups + gi]);
                const float bi = f16_to_f32(j->b[n * groups + gi]);
                const f8 sv = {sc, sc, sc, sc, sc, sc, sc, sc}, bv = {bi, bi, bi, bi, bi, bi, bi, bi};
                for (int64_t p = gi * wpg; p < (gi + 1) * wpg; ++p) acc += xv[p] * dequant8(wr[p], sv, bv);
            }
            j->y[n] = f32_to_f16(hsum8(acc));
            continue;
        }
        for (int64_t gi = 0; gi < groups; ++gi) {
            const float sc = f16_to_f32(j->s[n * groups + gi]);
            const float bi = f16_to_f32(j->b[n * groups + gi]);
            const f8 sv = {sc, sc, sc, sc, sc, sc, sc, sc}, bv = {bi, bi, bi, bi, bi, bi, bi, bi};
            for (int64_t p = gi * wpg; p < (gi + 1) * wpg; ++p) wrow[p] = dequant8(wr[p], sv, bv);
        }
        for (int64_t m = 0; m < j->M; ++m) {
            const f8* xv = (const f8*)(j->xf + m * K);
            f8 acc = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int64_t p = 0; p < packed; ++p) acc += xv[p] * wrow[p];
            j->y[m * j->N + n] = f32_to_f16(hsum8(acc));
        }
    }
    free(wrow);
    return NULL;
}

/* Returns the threads used (>= 1), or -1.  K % 8 == 0, g % 8 == 0. */
int cpu_q4_simd(const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                uint16_t* y, int64_t M, int64_t N, int64_t K, int64_t g, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    if (K % 8 != 0 || g % 8 != 0 || K % g != 0) return -1;
    float* xf = (float*)aligned_alloc(32, sizeof(float) * (size_t)(M * K + 8));
    if (!xf) return -1;
    for (int64_t i = 0; i < M * K; ++i) xf[i] = f16_to_f32(x[i]);
    pthread_t tid[256];
    simd_job jobs[256];
    const int64_t per = (N + threads - 1) / threads;
    int started = 0;
    for (int t = 0; t < threads; ++t) {
        const int64_t n0 = t * per, n1 = n0 + per < N ? n0 + per : N;
        if (n0 >= n1) break;
        simd_job jb = {xf, w, s, b, y, M, N, K, g, n0, n1};
        jobs[t] = jb;
        if (pthread_create(&tid[t], NULL, simd_worker, &jobs[t]) != 0) {
            for (int u = 0; u < started; ++u) pthread_join(tid[u], NULL);
            free(xf);
            return -1;
        }
        ++started;
    }
    for (int t = 0; t < started; ++t) pthread_join(tid[t], NULL);
    free(xf);
    return started;
}
