/*
 * q4_oracle.c -- CPU restatement of swift-ltx's MLX 4-bit dequant matmul.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP kernels
 * are compared against and the "port" CPU baseline that bench.py times beside
 * them.  Nothing in the shipped library links, loads or calls it; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the swift-ltx source tree, Sources/SwiftLLM/).
 *
 * Pinning (how each function is checked independently of itself, in
 * tests/test_oracle.py):
 *   oracle_f16_to_f32 / oracle_f32_to_f16   bit-exact vs numpy.float16 casts
 *                                            (library routine) on edge cases
 *                                            and 1M random bit patterns
 *   oracle_unpack_q4                        known-answer words (0x76543210...)
 *                                            and numpy pack/unpack round trip
 *   oracle_matmul_q4_f64                    brute-force pure-Python loops on
 *                                            tiny shapes, exact integer matmul
 *                                            (s=1,b=0), all-8 codes with b=-8s
 *                                            giving exactly 0, linearity,
 *                                            group-permutation invariance
 *   oracle_matmul_q4_emu                    within 2 fp16 ulp of the f64 oracle
 *   oracle_silu_mul / oracle_gelu_tanh_f32  closed forms via math.exp /
 *                                            math.tanh (fp64) and special
 *                                            values (0, +-large, clamp at 10)
 *   oracle_cpu_matmul_q4                    equals oracle_matmul_q4_f64 within
 *                                            fp32 rounding
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <pthread.h>
#include <stdlib.h>

/* ---------------------------------------------------------------- fp16 --- */

/* IEEE binary16 -> binary32, exact.  Metal `float(half)` (e.g. Kernels.swift:394). */
float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24 */
            float v = (float)man * 5.9604644775390625e-8f;
            memcpy(&bits, &v, 4);
            bits |= sign;
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

/* binary32 -> binary16, round-to-nearest-even, overflow to +-inf, no clamp.
 * Metal `half(float)` as used by matmul_q4's store (Kernels.swift:617) and
 * silu_mul (Kernels.swift:97). */
uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf or nan */
        if (ax == 0x7f800000u) return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t)((ax >> 13) & 0x3ffu);
    }
    int32_t e = (int32_t)(ax >> 23) - 127; /* unbiased exponent */
    uint32_t m = ax & 0x7fffffu;
    if (e > 15) return sign | 0x7c00u;
    if (e >= -14) { /* normal half range */
        uint32_t hm = m >> 13;
        uint32_t rem = m & 0x1fffu;
        uint32_t he = (uint32_t)(e + 15);
        uint32_t out = (he << 10) | hm;
        if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) out += 1; /* may carry into exp/inf */
        return sign | (uint16_t)out;
    }
    /* subnormal half (or zero): value in units of 2^-24 */
    if (e < -25) return sign; /* below half of smallest subnormal */
    uint32_t full = m | 0x800000u;          /* 24-bit significand, value = full * 2^(e-23) */
    int shift = -e - 1;                     /* units of 2^-24: full * 2^(e+1) */
    /* q = full >> shift (with shift in [14, 24]) */
    uint32_t q = full >> shift;
    uint32_t rem = full & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1;
    return sign | (uint16_t)q;
}

/* binary32 -> bfloat16, round-to-nearest-even (nan kept quiet). */
uint16_t oracle_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7fffu + lsb;
    return (uint16_t)(x >> 16);
}

float oracle_bf16_to_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* ------------------------------------------------------------- unpack --- */

/* Nibble k of row n is bits 4*(k%8)..+3 of word n*(K/8) + k/8, low nibble
 * first (Kernels.swift:385-390, embedding_q4_batch; :423-428 embedding_q4).
 * q: [N, K] uint8 out. */
void oracle_unpack_q4(const uint32_t* w, uint8_t* q, int64_t N, int64_t K) {
    int64_t packed_k = K / 8;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            uint32_t word = w[n * packed_k + k / 8];
            q[n * K + k] = (uint8_t)((word >> (4 * (k % 8))) & 0xfu);
        }
}

/* ---------------------------------------------------------- f64 oracle --- */

/* Closed form of the dequant matmul, in fp64:
 *   y[m,n] = sum_k x[m,k] * (s[n,k/g] * q[n,k] + b[n,k/g])
 * (dequant: Kernels.swift:392-395 `float(nibble)*scale + bias`; GEMV result:
 * Kernels.swift:444-620; the M>1 GEMM computes the same product, Ops.swift:312-381).
 * x is fp16 (x_is_bf16 = 0) or bf16 (x_is_bf16 = 1) bit patterns [M, K];
 * w [N, K/8]; s, b fp16 bit patterns [N, K/g]; y fp64 [M, N]. */
void oracle_matmul_q4_f64(const uint16_t* x, int x_is_bf16, const uint32_t* w,
                          const uint16_t* s, const uint16_t* b, double* y,
                          int64_t M, int64_t N, int64_t K, int64_t g) {
    int64_t packed_k = K / 8, groups = K / g;
    double* xd = (double*)malloc(sizeof(double) * (size_t)K);
    double* wd = (double*)malloc(sizeof(double) * (size_t)K);
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t k = 0; k < K; ++k) {
            uint32_t word = w[n * packed_k + k / 8];
            double q = (double)((word >> (4 * (k % 8))) & 0xfu);
            double sc = oracle_f16_to_f32(s[n * groups + k / g]);
            double bi = oracle_f16_to_f32(b[n * groups + k / g]);
            wd[k] = sc * q + bi;
        }
        for (int64_t m = 0; m < M; ++m) {
            for (int64_t k = 0; k < K; ++k)
                xd[k] = x_is_bf16 ? oracle_bf16_to_f32(x[m * K + k]) : oracle_f16_to_f32(x[m * K + k]);
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k) acc += xd[k] * wd[k];
            y[m * N + n] = acc;
        }
    }
    free(xd);
    free(wd);
}

/* ------------------------------------------------- matmul_q4 emulator --- */

/* fp32 emulation of matmul_q4's order of operations (Kernels.swift:444-620):
 * 32 lanes per output; lane l owns packs p = 4l + 128i .. +3 (loop :490);
 * per pack the 8 products float(q)*s*float(x) are added one by one (:547-585);
 * per 4-pack the bias term b0*sx0+b1*sx1+b2*sx2+b3*sx3 goes to a separate
 * accumulator (:594-600) where sx is the left-to-right fp32 sum of the pack's
 * 8 x values (:505-512); then sums += bias_sums and a 5-step xor butterfly
 * (:604-612); lane 0 stores half(sum) (:617).  Requires K % 32 == 0 (the
 * kernel reads packs in fours unchecked) and g % 8 == 0.  Out: fp16 bits. */
void oracle_matmul_q4_emu(const uint16_t* x, const uint32_t* w, const uint16_t* s,
                          const uint16_t* b, uint16_t* y, int64_t M, int64_t N,
                          int64_t K, int64_t g) {
    int64_t packed_k = K / 8, groups = K / g, ppg = g / 8;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float lane_sum[32];
            const uint32_t* wr = w + n * packed_k;
            const uint16_t* xr = x + m * K;
            for (int l = 0; l < 32; ++l) {
                float sums = 0.0f, bias_sums = 0.0f;
                for (int64_t p = (int64_t)l * 4; p < packed_k; p += 128) {
                    float sx[4];
                    for (int j = 0; j < 4; ++j) {
                        float acc = 0.0f;
                        for (int e = 0; e < 8; ++e) acc += oracle_f16_to_f32(xr[(p + j) * 8 + e]);
                        sx[j] = acc;
                    }
                    float bj[4];
                    for (int j = 0; j < 4; ++j) {
                        int64_t gi = (p + j) / ppg;
                        float sc = oracle_f16_to_f32(s[n * groups + gi]);
                        bj[j] = oracle_f16_to_f32(b[n * groups + gi]);
                        uint32_t pv = wr[p + j];
                        for (int e = 0; e < 8; ++e) {
                            float qf = (float)((pv >> (4 * e)) & 0xfu);
                            float prod = qf * sc;
                            prod = prod * oracle_f16_to_f32(xr[(p + j) * 8 + e]);
                            sums += prod;
                        }
                    }
                    float bt = bj[0] * sx[0];
                    bt += bj[1] * sx[1];
                    bt += bj[2] * sx[2];
                    bt += bj[3] * sx[3];
                    bias_sums += bt;
                }
                lane_sum[l] = sums + bias_sums;
            }
            for (int off = 1; off < 32; off <<= 1) {
                float tmp[32];
                for (int l = 0; l < 32; ++l) tmp[l] = lane_sum[l] + lane_sum[l ^ off];
                memcpy(lane_sum, tmp, sizeof(tmp));
            }
            y[m * N + n] = oracle_f32_to_f16(lane_sum[0]);
        }
}

/* ------------------------------------------------------ elementwise ops --- */

/* silu_mul (Kernels.swift:90-98): v = float(a); out = half((v/(1+exp(-v))) * float(b)). */
void oracle_silu_mul(const uint16_t* a, const uint16_t* b, uint16_t* out, int64_t count) {
    for (int64_t i = 0; i < count; ++i) {
        float v = oracle_f16_to_f32(a[i]);
        float r = (v / (1.0f + expf(-v))) * oracle_f16_to_f32(b[i]);
        out[i] = oracle_f32_to_f16(r);
    }
}

/* gelu_approximate_f32 (Kernels.swift:1774-1783):
 * inner = clamp(0.7978845608*(v + 0.044715*v^3), -10, 10); 0.5*v*(1+tanh(inner)). */
void oracle_gelu_tanh_f32(const float* x, float* out, int64_t count) {
    for (int64_t i = 0; i < count; ++i) {
        float v = x[i];
        float inner = 0.7978845608f * (v + 0.044715f * v * v * v);
        if (inner < -10.0f) inner = -10.0f;
        if (inner > 10.0f) inner = 10.0f;
        out[i] = 0.5f * v * (1.0f + tanhf(inner));
    }
}

/* ------------------------------------------------------- CPU baseline --- */

/* The "port" CPU baseline: the same dequant-matmul the GPU path computes,
 * in the loop shape of the reference's only CPU matmul (LlamaModel.swift:478-493:
 * for m, for n, for k, fp32 sum) with the weight dequantized on the fly per
 * Kernels.swift:392-395, fp32 accumulate, half() store.  Rows n are split over
 * `threads` pthreads.  y: fp16 bits [M, N]. */
typedef struct {
    const uint16_t *x, *s, *b;
    const uint32_t* w;
    uint16_t* y;
    int64_t M, N, K, g, n0, n1;
} cpu_job;

static void* cpu_worker(void* arg) {
    cpu_job* j = (cpu_job*)arg;
    int64_t packed_k = j->K / 8, groups = j->K / j->g;
    float* xf = (float*)malloc(sizeof(float) * (size_t)(j->M * j->K));
    for (int64_t i = 0; i < j->M * j->K; ++i) xf[i] = oracle_f16_to_f32(j->x[i]);
    float* wf = (float*)malloc(sizeof(float) * (size_t)j->K);
    for (int64_t n = j->n0; n < j->n1; ++n) {
        const uint32_t* wr = j->w + n * packed_k;
        for (int64_t k = 0; k < j->K; ++k) {
            float sc = oracle_f16_to_f32(j->s[n * groups + k / j->g]);
            float bi = oracle_f16_to_f32(j->b[n * groups + k / j->g]);
            wf[k] = (float)((wr[k / 8] >> (4 * (k % 8))) & 0xfu) * sc + bi;
        }
        for (int64_t m = 0; m < j->M; ++m) {
            const float* xr = xf + m * j->K;
            float sum = 0.0f;
            for (int64_t k = 0; k < j->K; ++k) sum += xr[k] * wf[k];
            j->y[m * j->N + n] = oracle_f32_to_f16(sum);
        }
    }
    free(wf);
    free(xf);
    return NULL;
}

int oracle_cpu_matmul_q4(const uint16_t* x, const uint32_t* w, const uint16_t* s,
                         const uint16_t* b, uint16_t* y, int64_t M, int64_t N,
                         int64_t K, int64_t g, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    cpu_job jobs[256];
    int64_t per = (N + threads - 1) / threads;
    int started = 0;
    for (int t = 0; t < threads; ++t) {
        int64_t n0 = t * per, n1 = n0 + per < N ? n0 + per : N;
        if (n0 >= n1) break;
        cpu_job jb = {x, s, b, w, y, M, N, K, g, n0, n1};
        jobs[t] = jb;
        if (pthread_create(&tid[t], NULL, cpu_worker, &jobs[t]) != 0) return -1;
        ++started;
    }
    for (int t = 0; t < started; ++t) pthread_join(tid[t], NULL);
    return started;
}
