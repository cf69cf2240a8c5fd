// q4_launch.hpp -- kernel parameter blocks and host launchers shared between
// the kernel translation units and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sltx {

// GEMV (M == 1) operands; see q4_gemv.hip.
struct GemvParams {
    const uint16_t* x;      // [K] fp16
    const uint32_t* w0;     // [N, K/8]
    const uint16_t* s0;     // [N, K/g] fp16
    const uint16_t* b0;     // [N, K/g] fp16
    const uint32_t* w1;     // up weights (SwiGLU only, else null)
    const uint16_t* s1;
    const uint16_t* b1;
    uint16_t* y;            // [N] fp16
    int N;
    int K;
    int groups;             // K / g
    int gshift;             // log2(g / 32): chunk of 32 nibbles c lies in group c >> gshift
    // Prologue (GemvPro): the GEMV's input is x itself, rms_norm(x), or
    // rms_norm(x + xb) with the rounded sum written to res_out (by block 0).
    int pro;
    const uint16_t* xb;     // second addend (GemvPro::kResidualRms)
    const float* norm_w;    // [K] fp32 norm weight
    float eps;
    uint16_t* res_out;      // [K] fp16 residual stream out (kResidualRms)
    // Epilogue: y = half(residual + half(x . W^T)) when non-null.
    const uint16_t* residual;
    int gelu;               // two weight sets: gelu_tanh(g) * u instead of silu(g) * u
    // Two x rows (rows == 2, no prologue): x, residual and y are [2, N]
    // (x [2, K]), y in y_dtype (kF16, kF32 or kBF16), and one weight set may
    // add bias[n] (fp32) and apply GELU-tanh.  rows == 1: fp16 y, neither.
    int rows;
    int y_dtype;
    const float* bias;
    int gelu_tanh;
};
// Whether the two-row GEMV covers N x K (q4_gemv.hip).
bool gemv2_ok(int N, int K);

enum GemvPro : int { kProNone = 0, kProRms = 1, kProResidualRms = 2 };

// GEMM (M > 1) operands; see q4_gemm.hip.
struct GemmParams {
    const void* a;          // [M, K] fp16 or bf16
    const uint32_t* w0;     // [N, K/8]
    const uint16_t* s0;     // [N, K/g]
    const uint16_t* b0;
    const uint32_t* w1;     // up weights (SiLU-mul epilogue only)
    const uint16_t* s1;
    const uint16_t* b1;
    const float* bias;      // [N] fp32 or null
    void* y;                // [M, N] fp16 / bf16 / fp32
    int M, N, K;
    int groups;             // K / g
    int gshift;             // log2(g / 32)
    int tiles_m, tiles_n;   // filled by launch_gemm
    int y_dtype;            // DType
    int epilogue;           // Epilogue
    const uint16_t* residual;   // [M, N] fp16, epilogue kEpiResidual
    float* ws;              // split-K partials [splits][M][N or 2N] (null: no split)
    // Split-K arrival counters, one per output tile (kTickets of them), zero
    // between launches (the last block of a tile resets its own); null: none.
    unsigned* tickets;
    int splits;             // filled by launch_gemm
    int split_tiles;        // k-tiles per split (even), filled by launch_gemm
    uint32_t nib_mask;      // 0x0F0F0F0F, set by the launchers (a run-time value: see q4_gemm.hip)
    int a_f32;              // a is fp32, cast to fp16 with the +-65504 clamp as it is staged (GEMM only)
};

// 4-bit embedding gather (q4_embed.hip).
struct EmbedParams {
    const uint32_t* w;      // [vocab, K/8]
    const uint16_t* s;      // [vocab, K/g]
    const uint16_t* b;
    const int32_t* ids;     // [n] token ids (device)
    uint16_t* out;          // [n, K] fp16
    int vocab, K, groups;
    int glog2;              // log2(g)
};

// Token selection after the lm_head (q4_sample.hip).
// Written by the sampler's gather kernel (and, mode 1, its narrow kernel)
// for the kernels after it.  mode 0: the buckets are level-0 bins (key >> 20)
// and the gather kernel compacted the candidates; mode 1: the candidate bins
// held too many tokens, and a range histogram splits them into finer
// buckets -- segment A, the keys [a_lo, a_end) of the cutoff's bin in
// buckets [0, 2048) of 2^a_shift keys counted from a_base, and segment B,
// the keys [b_lo, b_end) of the draw's bins above it in buckets [2048, 4096)
// counted from b_base; each segment's range is the smallest to the largest
// key its bins hold, and each base is its low key rounded down to the bucket
// width.  Tied buckets (one key) get per-chunk counts of their key (up to 4:
// tkey).
struct SampleCtl {
    uint32_t ccount;              // compacted candidates
    int mode;
    int cut_found;                // the top-p target lies within the total mass
    int a_shift, b_shift;
    uint32_t a_lo, a_base, b_lo, b_base;
    int ntied;
    uint32_t tkey[4];
    unsigned long long a_end, b_end;
    unsigned long long above;     // mode 1: mass of the keys above the range
    unsigned long long gap;       // mode 1: mass of the bins between the segments
    unsigned long long total;     // mass of all tokens
};

struct SampleParams {
    const void* logits;     // [n] fp16 or fp32
    int dtype;              // kF16 / kF32
    int n;
    float temperature, top_p, penalty, u;
    const int32_t* seen;    // [n_seen] token ids (device)
    int n_seen;
    int32_t* out;           // [1] chosen token (device)
    // Device-resident state (sltx_sample_top_p_state), all null otherwise.
    // The seen ids are hist[0, *hist_len) (seen == hist), the draw is
    // u_seq[*u_next], and the select kernel appends the chosen token to the
    // history and advances u_next.
    int32_t* hist;          // [hist_cap] token history
    int32_t* hist_len;      // [1] valid entries
    int hist_cap;
    const float* u_seq;     // [u_count] uniform draws
    int32_t* u_next;        // [1] index of this call's draw
    int u_count;
    // carved from the workspace by launch_sample
    float* probs;           // [n] scaled logits, then probabilities
    float* mpart;           // block maxima
    float* spart;           // block exp-sums (relative to the block maxima)
    uint32_t* h0cnt;        // level-0 histogram (4096 bins)
    unsigned long long* h0mass;
    uint32_t* h0min;        // smallest and largest key (probability bits) of each
    uint32_t* h0max;        // level-0 bin: a bin of equal keys is all tied
    uint32_t* h1cnt;        // range histogram (4096 buckets), same fields
    unsigned long long* h1mass;
    uint32_t* h1min;
    uint32_t* h1max;
    SampleCtl* ctl;         // candidate count and where the candidates come from
    uint32_t* tcnt;         // [4][ceil(n / 1024)] tied-key counts per 1024-token chunk
    uint2* cand;            // [n] (probability bits, id)
};

// Arrival counters at the start of each per-stream workspace (zeroed when the
// buffer is allocated; every launch leaves them zero).
constexpr int kTickets = 4096;
constexpr size_t kTicketBytes = kTickets * sizeof(unsigned);

hipError_t launch_gemv(const GemvParams& p, bool swiglu, hipStream_t st);
hipError_t launch_embedding_q4(const EmbedParams& p, int n, hipStream_t st);
size_t sample_workspace_bytes(int n);
size_t argmax_workspace_bytes();
hipError_t launch_argmax(const void* logits, int dtype, int n, int32_t* out, void* ws,
                         hipStream_t st);
hipError_t launch_sample(SampleParams p, void* ws, hipStream_t st);
// Largest vocabulary sltx_sample_top_p_noalloc accepts; its scratch holds
// sample_workspace_bytes(kSampleNoAllocMaxN) bytes per GPU.
constexpr int kSampleNoAllocMaxN = 262144;
constexpr int kMaxDevices = 64;
// Resolves the device address of that scratch on device `dev` (the current
// device); called once per device by the library's init.  Status code.
int sample_noalloc_scratch_init(int dev);
// The address resolved for `dev`, or null before sample_noalloc_scratch_init.
void* sample_noalloc_scratch(int dev);
// Narrow-M route (q4_narrow.hip, M <= 4, one weight set): a wave owns 4
// weight rows and 1/S of K's 512-k runs on 4x4x4 MFMA blocks; RG row groups
// (S waves each) per block.  narrow_plan returns false when the shape or
// epilogue is not covered.
struct NarrowPlan {
    int S, RG;
};
bool narrow_plan(const GemmParams& p, bool a_bf16, NarrowPlan* out);
hipError_t launch_narrow(const GemmParams& p, const NarrowPlan& pl, hipStream_t st);
// Small-M route (q4_skinny.hip): W waves split K into STEPS 128-wide steps
// each, MT tiles of 16 activation rows, RT tiles of 16 weight rows per block.
// skinny_plan returns false when the shape or epilogue is not covered (the
// GEMM then runs).
struct SkinnyPlan {
    int W, MT, STEPS, RT;
    int OCC;   // blocks per CU the configuration is compiled for
    bool XL;   // X staged in LDS (one 16-row tile, M * K * 2 bytes that fit)
};
bool skinny_plan(const GemmParams& p, bool a_bf16, SkinnyPlan* out);
hipError_t launch_skinny(const GemmParams& p, const SkinnyPlan& pl, hipStream_t st);
// Mid-M route (q4_mid.hip, M <= 32, K % 1024 == 0, fp16 X): 32 output
// columns per block (one set, or a gate/up pair) over all K or, for one set
// over few blocks, half of it (mid_splits); 8 compute waves over K-groups
// and 8 copy waves feeding LDS in whole lines.  mid_plan returns false when
// the shape, epilogue or alignment is not covered.  With 2 splits p.ws must
// hold mid_ws_bytes and p.tickets be set: the last of a tile's two blocks
// adds the halves.
bool mid_plan(const GemmParams& p, bool a_bf16);
int mid_splits(const GemmParams& p);
size_t mid_ws_bytes(const GemmParams& p, int splits);
hipError_t launch_mid(const GemmParams& p, int splits, hipStream_t st);

// Wide-M route (q4_wide.hip, 32 < M <= 256, fp16 X): 64 weight rows (or a
// 32-row gate/up pair) per block over all of its K range, up to 128
// activation rows per block (more rows take more blocks), the 8 waves
// splitting K; optionally split over K across blocks (fp32 partials in the
// workspace; the last block of each output tile adds them).  wide_plan returns false when the
// shape, epilogue or alignment is not covered.
struct WidePlan {
    int tm;          // 32-row MFMA tiles per block (2..4)
    int mblocks;     // blocks along M
    int mrows;       // activation rows per M-block
    int nblocks;     // blocks along N
    int splits;      // K splits across blocks
    int kblk;        // k per split (a multiple of 128)
    size_t ws_bytes; // fp32 partials when splits > 1
};
bool wide_plan(const GemmParams& p, bool a_bf16, WidePlan* out);
// p.ws must hold pl.ws_bytes and p.tickets be set when pl.splits > 1: the
// last block of each output tile to finish adds the splits' partial sums
// (no reduce pass).
hipError_t launch_wide(GemmParams p, const WidePlan& pl, hipStream_t st);
// The split-K reduce pass: y = epilogue(sum of p.splits fp32 partials in p.ws).
hipError_t launch_splitk_reduce(const GemmParams& p, hipStream_t st);

// Bytes of split-K workspace the launch of `p` would use (0: it does not split).
size_t gemm_workspace_bytes(const GemmParams& p);
// Launches the GEMM; splits K only if p.ws is non-null (and then needs
// gemm_workspace_bytes(p) bytes there).
hipError_t launch_gemm(GemmParams p, bool a_bf16, hipStream_t st);
// Bytes of fp32 partials the fused residual + RMSNorm GEMM of `p` uses (its
// output always goes through the workspace, at one split or more).
size_t gemm_partials_workspace_bytes(const GemmParams& p);
// GEMM (no epilogue; p.residual is the residual input) into the workspace
// p.ws, then one pass per row: res_out = half(residual + half(sum of splits))
// and norm_out = rms_norm(res_out) with the sum of squares over the unrounded
// sum (sum_rounded false) or over res_out (true).  N % 8 == 0, N <= 16384.
hipError_t launch_gemm_residual_rms_norm(GemmParams p, bool a_bf16, const float* norm_w, float eps,
                                         uint16_t* res_out, uint16_t* norm_out, bool sum_rounded,
                                         hipStream_t st);
hipError_t launch_silu_mul(const uint16_t* a, const uint16_t* b, uint16_t* out, long count,
                           hipStream_t st);
// out = half(clamp(x, -65504, 65504)), count % 8 == 0, 16-byte aligned.
hipError_t launch_cast_f32_f16(const float* x, uint16_t* out, long count, hipStream_t st);
// Row-wise RMS norm, optionally of a + b (then the rounded sum goes to res_out).
hipError_t launch_rms_norm(const uint16_t* a, const uint16_t* b, const float* w, float eps,
                           uint16_t* res_out, uint16_t* out, int rows, int dim, hipStream_t st);
int gemv_pick_lanes(int K, int* cpl_out);

// Sets the calling thread's sltx_last_error() message; returns code.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

}  // namespace sltx
