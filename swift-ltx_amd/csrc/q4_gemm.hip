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
// Block tile 128 x 128 x 64, 256 threads = 4 waves in a 2 x 2 layout, each
// wave computing 64 x 64 with v_mfma_f32_32x32x16_{f16,bf16}.
//  * A tile (128 x 64, fp16 or bf16) is copied global -> registers -> LDS.
//  * W tile (128 rows x 64 nibbles = 32 B per row) is loaded one 16-byte
//    chunk per thread, dequantized in registers to fp16 (or bf16) with its
//    group's scale and bias, and written to LDS.  fp16: nibbles are spread to
//    bytes, paired with v_perm_b32, turned into 1024+q by mantissa insertion,
//    reduced to q exactly, then one fp16 FMA q*s+b (a single rounding).
//    bf16: q*s+b in fp32, rounded once to bf16.
//  * LDS rows are 128 bytes; 16-byte column c of row r is stored at c ^ (r & 7)
//    so the MFMA operand reads (32 rows, same column) are conflict-free.
//  * Two LDS stages: global loads for tile k+1 are issued before the MFMAs
//    of tile k and stored after them, one barrier per k-tile.
//  * Tile order is XCD-aware: the 8 XCDs receive workgroups round-robin, so
//    consecutive logical tiles (M fastest) are mapped to one XCD so that the
//    M-blocks sharing a weight column block share that XCD's L2.
#include "q4_common.hpp"
#include "q4_launch.hpp"

namespace sltx {


constexpr int BM = 128, BN = 128, BK = 64;
constexpr int kThreads = 256;

__device__ __forceinline__ int swz(int row, int col16) { return (row * 8 + (col16 ^ (row & 7))); }

// 32 nibbles -> 32 fp16 values s*q+b (k order), four 16-byte rows of 8.
__device__ __forceinline__ void dequant_f16(const u32x4 w, uint16_t s_bits, uint16_t b_bits,
                                            u32x4 out[4]) {
    const f16 s = __builtin_bit_cast(f16, s_bits), b = __builtin_bit_cast(f16, b_bits);
    const f16x2 s2 = {s, s}, b2 = {b, b};
    const f16x2 m1024 = {(f16)-1024.0f, (f16)-1024.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t lo = w[j] & 0x0F0F0F0Fu;          // bytes q6 q4 q2 q0
        const uint32_t hi = (w[j] >> 4) & 0x0F0F0F0Fu;   // bytes q7 q5 q3 q1
        uint32_t pr[4];
        pr[0] = __builtin_amdgcn_perm(hi, lo, 0x0C040C00u) | kMagic1024x2;  // q0, q1
        pr[1] = __builtin_amdgcn_perm(hi, lo, 0x0C050C01u) | kMagic1024x2;  // q2, q3
        pr[2] = __builtin_amdgcn_perm(hi, lo, 0x0C060C02u) | kMagic1024x2;  // q4, q5
        pr[3] = __builtin_amdgcn_perm(hi, lo, 0x0C070C03u) | kMagic1024x2;  // q6, q7
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const f16x2 q = as_f16x2(pr[e]) + m1024;   // exact small integers
            o[e] = as_u32(__builtin_elementwise_fma(q, s2, b2));  // v_pk_fma_f16: one rounding
        }
        out[j] = o;
    }
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
}

// 32 nibbles -> 32 bf16 values bf16(s*q+b) computed in fp32.
__device__ __forceinline__ void dequant_bf16(const u32x4 w, uint16_t s_bits, uint16_t b_bits,
                                             u32x4 out[4]) {
    const float s = h2f(s_bits), b = h2f(b_bits);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t lo = w[j] & 0x0F0F0F0Fu;
        const uint32_t hi = (w[j] >> 4) & 0x0F0F0F0Fu;
        float q[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            q[2 * e] = (float)((lo >> (8 * e)) & 0xFFu);
            q[2 * e + 1] = (float)((hi >> (8 * e)) & 0xFFu);
        }
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            o[e] = pack_bf16x2(fmaf(q[2 * e], s, b), fmaf(q[2 * e + 1], s, b));
        out[j] = o;
    }
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

struct GemmStage {
    u32x4 a[BM * BK / 8];   // 1024 x 16 B, swizzled [row][col16]
    u32x4 w[BN * BK / 8];
};

template <bool BF16, bool SILU>
__global__ __launch_bounds__(kThreads, 2) void q4_gemm_kernel(GemmParams p) {
    __shared__ GemmStage st[2];

    // ---- tile selection (XCD-aware) ----
    const int ntiles = p.tiles_m * p.tiles_n;
    int logical = blockIdx.x;
    if ((gridDim.x & 7) == 0) {
        const int per_xcd = gridDim.x >> 3;
        logical = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    }
    if (logical >= ntiles) return;
    const int tile_m = logical % p.tiles_m;
    const int tile_n = logical / p.tiles_m;
    const int m0 = tile_m * BM;
    // SILU: a tile covers 64 output columns, as 64 gate rows + 64 up rows.
    const int n0 = tile_n * (SILU ? BN / 2 : BN);

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;

    // ---- per-thread global load assignments ----
    // A: 4 chunks of 16 B: chunk q = tid + 256*i -> row q/8, col16 q%8.
    const uint16_t* A = reinterpret_cast<const uint16_t*>(p.a);
    // W: virtual row vr = tid/2, half = tid%2 (32 nibbles).
    const int vr = tid >> 1, whalf = tid & 1;
    int wn_row;
    const uint32_t* Wsel;
    const uint16_t *Ssel, *Bsel;
    if (SILU) {
        const int wv = vr >> 6, tn = (vr >> 5) & 1;
        wn_row = n0 + wv * 32 + (vr & 31);
        Wsel = tn ? p.w1 : p.w0;
        Ssel = tn ? p.s1 : p.s0;
        Bsel = tn ? p.b1 : p.b0;
    } else {
        wn_row = n0 + vr;
        Wsel = p.w0;
        Ssel = p.s0;
        Bsel = p.b0;
    }
    const bool w_ok = wn_row < p.N;
    const size_t w_row_off = (size_t)(w_ok ? wn_row : 0) * (p.K / 8);
    const size_t g_row_off = (size_t)(w_ok ? wn_row : 0) * p.groups;

    const int nk = (p.K + BK - 1) / BK;

    // Loads are unconditional with clamped addresses (a predicated load is
    // compiled into a branch with a wait inside it); out-of-range elements
    // are zeroed when the registers are written to LDS, after the MFMAs of
    // the current tile have hidden the load latency.
    u32x4 ra[4];
    bool ra_ok[4];
    u32x4 rw;
    uint32_t rs, rb;
    bool rw_ok;

    auto gload = [&](int kt) {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = tid + kThreads * i;
            const int row = q >> 3, c16 = q & 7;
            const int m = m0 + row, k = k0 + c16 * 8;
            ra_ok[i] = m < p.M && k < p.K;
            const int mc = m < p.M ? m : p.M - 1;
            const int kc = k < p.K ? k : p.K - 8;
            ra[i] = *reinterpret_cast<const u32x4*>(A + (size_t)mc * p.K + kc);
        }
        const int kw = k0 + whalf * 32;
        rw_ok = w_ok && kw < p.K;
        const int kwc = kw < p.K ? kw : p.K - 32;
        rw = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(Wsel + w_row_off + (kwc >> 3)));
        const size_t gi = g_row_off + ((kwc >> 5) >> p.gshift);
        rs = Ssel[gi];
        rb = Bsel[gi];
    };

    auto lstore = [&](int buf) {
        const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = tid + kThreads * i;
            st[buf].a[swz(q >> 3, q & 7)] = ra_ok[i] ? ra[i] : z;
        }
        u32x4 dq[4];
        const u32x4 wq = rw_ok ? rw : z;
        const uint16_t sq = rw_ok ? (uint16_t)rs : (uint16_t)0;
        const uint16_t bq = rw_ok ? (uint16_t)rb : (uint16_t)0;
        if (BF16)
            dequant_bf16(wq, sq, bq, dq);
        else
            dequant_f16(wq, sq, bq, dq);
#pragma unroll
        for (int j = 0; j < 4; ++j) st[buf].w[swz(vr, whalf * 4 + j)] = dq[j];
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    gload(0);
    lstore(0);
    __syncthreads();

    const int lrow = lane & 31, lk = lane >> 5;
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int c16 = ks * 2 + lk;
            u32x4 af[2], bf[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                af[t] = st[buf].a[swz(wm * 64 + t * 32 + lrow, c16)];
                bf[t] = st[buf].w[swz(wn * 64 + t * 32 + lrow, c16)];
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma32<BF16>(af[i], bf[j], acc[i][j]);
        }
        if (kt + 1 < nk) lstore(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue ----
    // 32x32 accumulator layout: lane l, element v -> row 8*(v/4) + 4*(l/32) + v%4,
    // column l%32.
    const int col_l = lane & 31;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int m = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * lk + (v & 3);
            if (m >= p.M) continue;
            if (SILU) {
                const int n = n0 + wn * 32 + col_l;
                if (n >= p.N) continue;
                const float out = silu_mul_f32(acc[i][0][v], acc[i][1][v]);
                const size_t o = (size_t)m * p.N + n;
                if (p.y_dtype == kF32)
                    reinterpret_cast<float*>(p.y)[o] = out;
                else if (p.y_dtype == kBF16)
                    reinterpret_cast<uint16_t*>(p.y)[o] = f2bf(out);
                else
                    reinterpret_cast<uint16_t*>(p.y)[o] = f2h(out);
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int n = n0 + wn * 64 + j * 32 + col_l;
                    if (n >= p.N) continue;
                    float out = acc[i][j][v];
                    if (p.bias) out += p.bias[n];
                    if (p.epilogue == kEpiGeluTanh) out = gelu_tanh_f32(out);
                    const size_t o = (size_t)m * p.N + n;
                    if (p.y_dtype == kF32)
                        reinterpret_cast<float*>(p.y)[o] = out;
                    else if (p.y_dtype == kBF16)
                        reinterpret_cast<uint16_t*>(p.y)[o] = f2bf(out);
                    else
                        reinterpret_cast<uint16_t*>(p.y)[o] = f2h(out);
                }
            }
        }
    }
}

hipError_t launch_gemm(GemmParams p, bool a_bf16, hipStream_t st) {
    const bool silu = p.epilogue == kEpiSiluMul;
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = (p.N + (silu ? BN / 2 : BN) - 1) / (silu ? BN / 2 : BN);
    const long ntiles = (long)p.tiles_m * p.tiles_n;
    if (ntiles <= 0) return hipSuccess;
    const long grid = (ntiles + 7) / 8 * 8;
    if (grid > 0x7fffffffL) return hipErrorInvalidValue;
    if (a_bf16) {
        if (silu)
            hipLaunchKernelGGL((q4_gemm_kernel<true, true>), dim3(grid), dim3(kThreads), 0, st, p);
        else
            hipLaunchKernelGGL((q4_gemm_kernel<true, false>), dim3(grid), dim3(kThreads), 0, st, p);
    } else {
        if (silu)
            hipLaunchKernelGGL((q4_gemm_kernel<false, true>), dim3(grid), dim3(kThreads), 0, st, p);
        else
            hipLaunchKernelGGL((q4_gemm_kernel<false, false>), dim3(grid), dim3(kThreads), 0, st, p);
    }
    return hipGetLastError();
}

}  // namespace sltx
