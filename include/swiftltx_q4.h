/*
 * swiftltx_q4.h -- C ABI of the MI355X (gfx950) MLX 4-bit dequant matmul path.
 *
 * Drop-in for swift-ltx's quantized-matmul operators (Sources/SwiftLLM/Ops.swift)
 * and the weight layout its loader produces (ModelWeights.swift:7-11):
 *
 *   weight  uint32 [N, K/8]          nibble k of row n = bits 4*(k%8)..+3 of word k/8
 *   scales  fp16   [N, K/group_size]
 *   biases  fp16   [N, K/group_size]
 *   w[n,k] = scales[n,k/g] * q[n,k] + biases[n,k/g]      (Kernels.swift:392-395)
 *   out[m,n] = sum_k x[m,k] * w[n,k], fp32 accumulation
 *
 * Conventions (all entry points):
 *   - Every pointer is a device pointer the caller allocated; the library never
 *     frees or keeps them.  Outputs are written, never read.
 *   - Memory: the only device memory the library allocates is a per-stream
 *     workspace: fp32 partial sums for GEMMs with too few output tiles to
 *     fill the GPU (split-K, e.g. M=750 x N=3072, and at 8 < M <= 256 the
 *     mid- and wide-M K splits, e.g. M=32 x 4096 x 10240) and for every
 *     sltx_matmul_q4_residual_rms_norm, the block partials of
 *     sltx_argmax, and the probabilities and candidate list of
 *     sltx_sample_top_p[_state], after 16 KB of split-K arrival counters
 *     (zeroed when the buffer is allocated, left at zero by every launch);
 *     and a second one per stream for the fp16
 *     copy of fp32 activations (sltx_matmul_q4_ex).  There is one per (device, stream),
 *     grown on first need to at least twice its old size; a replaced buffer
 *     is not freed (a graph captured earlier may still use it): every buffer
 *     lives until sltx_release_workspace(stream) or the process exits.  A
 *     stream being captured into a HIP graph never allocates: if its
 *     workspace is missing or too small,
 *     that GEMM runs unsplit (the same product, its fp32 sums in another
 *     order; lower throughput).  Capture after
 *     one eager call on the same stream to get the split kernel into a graph
 *     (with torch, pass that stream to torch.cuda.graph(..., stream=s)).  A
 *     captured graph keeps using its stream's workspace: replay it on that
 *     stream, or keep that stream's other work from overlapping the replay.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the default stream) and
 *     nothing synchronises: results are visible to later work on that stream.
 *     This mirrors the reference's batched mode (MetalContext.swift:109-134).
 *   - Return value: SLTX_OK (0) or a negative sltx_status.  On failure nothing
 *     was enqueued and sltx_last_error() (thread-local) says why.  The
 *     reference has no error returns: it crashes (Kernels.swift:19,25-26) or,
 *     for unchecked shapes such as K % 32 != 0, reads out of bounds
 *     (Kernels.swift:490).  Here such shapes are rejected before any launch.
 *   - Shape rules: K > 0, K % 32 == 0, group_size in {32, 64, 128},
 *     K % group_size == 0, M >= 0, N >= 0 (M == 0 or N == 0 is a no-op).
 *     x and weight must be 16-byte aligned; scales, biases and 16-bit outputs
 *     2-byte aligned; fp32 outputs and bias 4-byte aligned.
 *   - A matmul's output must not overlap its activation input x (blocks re-read
 *     x while others store); such calls return SLTX_ERR_INVALID.  Where an
 *     entry point allows out == residual it says so.
 *   - Thread-safe: no hidden global mutable state beyond a once-per-device init.
 */
#ifndef SWIFTLTX_Q4_H
#define SWIFTLTX_Q4_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum sltx_status {
    SLTX_OK = 0,
    SLTX_ERR_INVALID = -1,     /* bad pointer, shape, alignment or enum */
    SLTX_ERR_UNSUPPORTED = -2, /* valid for the reference, not built here (e.g. group_size 16) */
    SLTX_ERR_HIP = -3          /* HIP runtime error (no device, launch failure, ...) */
} sltx_status;

typedef enum sltx_dtype {
    SLTX_F16 = 0,
    SLTX_BF16 = 1,
    SLTX_F32 = 2
} sltx_dtype;

typedef enum sltx_epilogue {
    SLTX_EPI_NONE = 0,
    SLTX_EPI_GELU_TANH = 2 /* out = gelu_tanh(acc + bias), Kernels.swift:1774-1783 */
} sltx_epilogue;

/* LinearWeight.quantized(weight:scales:biases:K:groupSize:) (ModelWeights.swift:7-11). */
typedef struct sltx_q4_weight {
    const uint32_t* weight; /* [N, K/8] */
    const uint16_t* scales; /* [N, K/group_size] fp16 */
    const uint16_t* biases; /* [N, K/group_size] fp16 */
    int32_t K;
    int32_t group_size;
} sltx_q4_weight;

/* ABI version of this header (bumped on any signature change). */
int sltx_abi_version(void);

/* Checks the current HIP device is usable (gfx950).  Called lazily by every
 * compute entry point; calling it first only moves the cost.  No counterpart
 * in the reference (MetalContext.shared, MetalContext.swift:52-65, is its
 * analogue). */
int sltx_init(void);

/* Message for the last non-zero status returned on this thread. */
const char* sltx_last_error(void);

/* Frees the workspace of `stream` on the current device, and every buffer it
 * replaced, after waiting for the work already queued on that stream.  A
 * later call on the stream allocates a new one.  Graphs captured on the
 * stream name the freed buffers: destroy them first (replaying one afterwards
 * is undefined).  SLTX_OK when the stream has no workspace; SLTX_ERR_INVALID
 * while the stream is being captured.  Callers that create and destroy
 * streams call this before hipStreamDestroy, else each stream's buffers stay
 * allocated until the process ends.  No counterpart in the reference (its
 * BufferPool, Tensor.swift:47-58, lives as long as the process). */
int sltx_release_workspace(void* stream);

/* matmulQ4(_:weight:scales:biases:M:K:N:groupSize:) -> Tensor  (Ops.swift:285-305)
 * out[M,N] fp16 = x[M,K] fp16 . dequant(W)^T.  M == 1 runs the HBM-streaming
 * GEMV (the reference's matmul_q4, Kernels.swift:444-620); M > 1 runs the
 * route sltx_gemm_route names: the same GEMV over two rows at M == 2 on sets
 * of at most 5120 x 4096, else an MFMA weight stream or the MFMA GEMM (the
 * reference re-reads W per row here; results agree within the stated
 * tolerance). */
int sltx_matmul_q4(const void* x, const uint32_t* weight, const uint16_t* scales,
                   const uint16_t* biases, void* out, int32_t M, int32_t K, int32_t N,
                   int32_t group_size, void* stream);

/* matmulQ4Fast(_:weight:scales:biases:M:K:N:groupSize:) -> Tensor  (Ops.swift:312-345)
 * Same product, fp16 out, through the M > 1 routes for every M (M == 1
 * included: the MFMA GEMM's numerics). */
int sltx_matmul_q4_fast(const void* x, const uint32_t* weight, const uint16_t* scales,
                        const uint16_t* biases, void* out, int32_t M, int32_t K, int32_t N,
                        int32_t group_size, void* stream);

/* matmulQ4FastF32(_:weight:scales:biases:M:K:N:groupSize:) -> Tensor  (Ops.swift:348-381)
 * Same product, fp32 out (no fp16 overflow). */
int sltx_matmul_q4_fast_f32(const void* x, const uint32_t* weight, const uint16_t* scales,
                            const uint16_t* biases, float* out, int32_t M, int32_t K, int32_t N,
                            int32_t group_size, void* stream);

/* siluMul(_:_:) -> Tensor  (Ops.swift:44-56; kernel silu_mul, Kernels.swift:90-98)
 * out[i] = half(silu(float(a[i])) * float(b[i])), count fp16 elements. */
int sltx_silu_mul(const void* a, const void* b, void* out, int64_t count, void* stream);

/* linear(_:_:M:K:N:fast:) -> Tensor for the .quantized case  (Ops.swift:741-752)
 * Routing rule kept: fast && M > 1 -> sltx_matmul_q4_fast, else sltx_matmul_q4.
 * w->K must equal K.  The reference's .float case is a CPU fp32 matmul
 * (LlamaModel.swift:478-493) and is outside this library. */
int sltx_linear(const void* x, const sltx_q4_weight* w, void* out, int32_t M, int32_t K,
                int32_t N, int32_t fast, void* stream);

/* Fused SwiGLU: out[M,N] fp16 = silu(x.Wg^T) * (x.Wu^T), in one pass over
 * both weight sets with the product formed from the fp32 accumulators.
 * Replaces linear(gate) + linear(up) + siluMul (LlamaModel.swift:275-277
 * prefill, :327-329 decode).  The reference rounds gate and up to fp16 before
 * silu_mul; this keeps them in fp32 (closer to the fp64 oracle).  M == 1 runs
 * the GEMV, M > 1 the GEMM.  gate and up must have equal K and group_size. */
int sltx_matmul_q4_silu_mul(const void* x, const sltx_q4_weight* gate, const sltx_q4_weight* up,
                            void* out, int32_t M, int32_t K, int32_t N, void* stream);

/* Extended GEMM: x_dtype in {SLTX_F16, SLTX_BF16, SLTX_F32}; out_dtype in
 * {SLTX_F16, SLTX_BF16, SLTX_F32}; bias (fp32 [N]) optional (NULL = none);
 * epilogue SLTX_EPI_NONE or SLTX_EPI_GELU_TANH.  out = epi(x . dequant(W)^T +
 * bias).  Covers DiTLinear.applyF32in's quantized branch
 * (DiTModel.swift:102-125: castF32toF16, matmulQ4FastF32, then addBiasF32F32,
 * Ops.swift:1780-1791) and the GELU-tanh that follows it in the DiT
 * feed-forward (DiTModel.swift:953, Kernels.swift:1774-1783).  fp32 x is
 * cast as the reference's cast_f32_to_f16 does, half(clamp(x, -65504,
 * 65504)) (Kernels.swift:816-822): for N <= 512 inside the MFMA GEMM as it
 * stages x; for wider outputs once, into a second per-stream buffer of M*K*2
 * bytes (allocated like the workspace), after which the fp16 routes run --
 * the same results as passing that cast as fp16 x.  A stream being captured
 * whose buffer is missing or too small uses the in-GEMM cast.  bf16 x is
 * multiplied as bf16. */
int sltx_matmul_q4_ex(const void* x, int32_t x_dtype, const sltx_q4_weight* w, const float* bias,
                      int32_t epilogue, void* out, int32_t out_dtype, int32_t M, int32_t N,
                      void* stream);

/* GeGLU: out[M,N] fp16 = gelu_tanh(x.Wg^T) * (x.Wu^T), GELU-tanh with the
 * inner clamp at +-10 (Kernels.swift:1785-1795), in one pass over both weight
 * sets.  Replaces matmulQ4Fast(wi_0) + matmulQ4Fast(wi_1) +
 * geluApproximateF16 + elemMulF16 in the T5 encoder FFN (T5Encoder.swift:191-199).
 * The reference rounds the two products (and the GELU) to fp16 and multiplies
 * in half precision; here both products stay fp32 and the result is rounded
 * once.  M == 1 runs the GEMV, M > 1 the GEMM. */
int sltx_matmul_q4_geglu(const void* x, const sltx_q4_weight* gate, const sltx_q4_weight* up,
                         void* out, int32_t M, int32_t K, int32_t N, void* stream);

/* embeddingQ4Batch(weight:scales:biases:tokenIds:K:groupSize:) -> Tensor [n, K]
 * (Ops.swift:163-187; kernel embedding_q4_batch, Kernels.swift:368-396), and
 * embeddingQ4 for one token (n = 1; Ops.swift:189-208, Kernels.swift:409-434):
 * out[t, k] fp16 = half(float(q[id_t, k]) * s + b), fp32 math.  table is the
 * quantized embedding (Llama ties it to the lm_head, ModelWeights.swift:126-130)
 * with vocab rows; token_ids is device int32 [n].  Ids outside [0, vocab)
 * give zero rows (the reference reads out of bounds).  out 16-byte aligned. */
int sltx_embedding_q4(const sltx_q4_weight* table, int32_t vocab, const int32_t* token_ids,
                      int32_t n, void* out, void* stream);

/* ---- Decode-layer fusion: the operators on either side of the projections ----
 * Norm weights are fp32 (ModelWeights.swift:123,147-148 loads them as float).
 * rms_norm(v)[k] = half(r[k] * rsqrt(mean(v^2) + eps) * weight[k]), r = the
 * fp16 input; the sum of squares runs in fp32 (rms_norm, Kernels.swift:40-86). */

/* rmsNorm(_:weight:eps:dim:) -> Tensor  (Ops.swift:8-27), rows x dim fp16.
 * For M > 1 (prefill); at M = 1 use the fused form below.  out may be x
 * itself (in place) but must not otherwise overlap it. */
int sltx_rms_norm(const void* x, const float* weight, float eps, void* out, int32_t rows,
                  int32_t dim, void* stream);

/* residualRmsNorm(_:_:weight:eps:dim:) -> (residual, normed)  (Ops.swift:256-279;
 * kernel residual_rms_norm, Kernels.swift:238-290): residual_out = half(a + b);
 * norm_out = rms_norm of it, with the sum of squares over the unrounded a + b.
 * residual_out and norm_out must not overlap; either may be a or b itself
 * (in place, e.g. h = h + o) but must not otherwise overlap them. */
int sltx_residual_rms_norm(const void* a, const void* b, const float* weight, float eps,
                           void* residual_out, void* norm_out, int32_t rows, int32_t dim,
                           void* stream);

/* rmsNorm + linear at M = 1 (LlamaModel.swift:288-292: input_layernorm, then
 * the q/k/v projections, here one weight with q|k|v rows concatenated):
 * out[1,N] fp16 = rms_norm(x) . dequant(W)^T, with K = w->K.  The normalized
 * vector is formed inside the GEMV and not written.  x and norm_weight 16-byte
 * aligned. */
int sltx_rmsnorm_matmul_q4(const void* x, const float* norm_weight, float eps,
                           const sltx_q4_weight* w, void* out, int32_t N, void* stream);

/* residualRmsNorm + linear(gate) + linear(up) + siluMul at M = 1
 * (LlamaModel.swift:326-329): residual_out[K] = half(a + b) (the residual
 * stream, needed by the final add); out[1,N] = silu(n . Wg^T) * (n . Wu^T)
 * with n = rms_norm(residual), fp32 gate/up products (as
 * sltx_matmul_q4_silu_mul).  a, b, norm_weight, residual_out 16-byte aligned;
 * residual_out must not overlap a or b. */
int sltx_residual_rmsnorm_matmul_q4_silu_mul(const void* a, const void* b,
                                             const float* norm_weight, float eps,
                                             void* residual_out, const sltx_q4_weight* gate,
                                             const sltx_q4_weight* up, void* out, int32_t N,
                                             void* stream);

/* linear + elemAdd  (LlamaModel.swift:330-331, Ops.swift:72-84; add kernel,
 * Kernels.swift:121-128): out[M,N] fp16 = half(residual + half(x . dequant(W)^T)),
 * the projection rounded to fp16 before the add as in the reference.  M == 1
 * runs the GEMV, M > 1 the GEMM.  out may be residual itself (in place) but
 * must not otherwise overlap it, nor x. */
int sltx_matmul_q4_residual(const void* x, const sltx_q4_weight* w, const void* residual,
                            void* out, int32_t M, int32_t N, void* stream);

/* linear + residual add + RMSNorm of the sum, for prefill rows (one call in
 * place of two or three):
 *   sum_rounded == 0: linear then residualRmsNorm(residual, o)  (the o_proj
 *     step, LlamaModel.swift:269-272; Ops.swift:256-279; Kernels.swift:238-290):
 *     the sum of squares is over the unrounded residual + o;
 *   sum_rounded != 0: linear, elemAdd, then the next layer's rmsNorm of the
 *     stored fp16 sum  (the down_proj step and the next input_layernorm,
 *     LlamaModel.swift:278-279, 233; Ops.swift:8-27, 72-84).
 * residual_out[M,N] = half(residual + half(x . dequant(W)^T)) and
 * norm_out = rms_norm(residual_out) with norm_weight (fp32 [N]); both equal,
 * bit for bit, the unfused sequence of this library's GEMM (M > 1 route) and
 * sltx_residual_rms_norm / sltx_rms_norm.  Always runs the GEMM (any M >= 1),
 * whose fp32 partial sums go through the per-stream workspace, then one pass
 * per row.  N % 8 == 0 and N <= 16384; residual, residual_out, norm_out,
 * norm_weight 16-byte aligned.  residual_out may be residual (in place);
 * norm_out must overlap neither, and no output may overlap x.  While the stream
 * is being captured the workspace must already exist (an eager call of the
 * same shape on that stream first), else the call fails.
 * No single reference entry point: it replaces the pairs named above. */
int sltx_matmul_q4_residual_rms_norm(const void* x, const sltx_q4_weight* w, const void* residual,
                                     const float* norm_weight, float eps, int32_t M, int32_t N,
                                     int32_t sum_rounded, void* residual_out, void* norm_out,
                                     void* stream);

/* ---- Token selection after the lm_head (LlamaModel.swift:153,161) ----
 * Both read n logits (SLTX_F16 or SLTX_F32, device) and write one int32 token
 * id to device memory, so the next step's embedding gather can consume it
 * without a host round trip. */

/* argmax(_:) -> Int  (Ops.swift:757-781): the first index of the maximum.
 * NaNs never win; a NaN at index 0 gives 0, as the reference's strict ">"
 * scan from element 0 does.  Uses 2 KB of the per-stream workspace (see
 * above): under graph capture call it once eagerly on that stream first. */
int sltx_argmax(const void* logits, int32_t dtype, int32_t n, int32_t* out_index, void* stream);

/* sample(_:temperature:topP:repetitionPenalty:seenTokens:) -> Int
 * (Ops.swift:785-806, sampleFromLogits Ops.swift:2060-2098), in fp32:
 * each distinct id of seen[0..n_seen) in [0, n) has its logit divided by
 * repetition_penalty when positive, else multiplied; all logits are divided
 * by temperature; softmax; tokens ordered by probability descending (ties by
 * ascending id: the reference's sort is unstable); the shortest prefix whose
 * running sum reaches top_p is kept (all tokens if none does); then
 * r = u * (that sum) and the first token of the prefix at which r minus the
 * running probabilities is <= 0 is chosen.  u is the caller's uniform draw in
 * [0, 1) (the reference calls Float.random).  temperature, top_p and
 * repetition_penalty > 0; n <= 2^24.  Running sums are exact (integer masses
 * floor(p * 2^52)) where the reference sums sequentially in fp32, and the
 * softmax denominator is a fixed-order tree: a draw within fp32 rounding of
 * a token boundary may pick the neighbouring token.  Uses the per-stream workspace (see above): under
 * graph capture it must already hold sample workspace for this n. */
int sltx_sample_top_p(const void* logits, int32_t dtype, int32_t n, float temperature,
                      float top_p, float repetition_penalty, const int32_t* seen,
                      int32_t n_seen, float u, int32_t* out_index, void* stream);

/* sltx_sample_top_p computed in a fixed scratch area instead of the
 * per-stream workspace: the same arguments, kernels and result, and no device
 * memory allocated by the call.  No counterpart in the reference (its sampler
 * runs on the CPU); it is for callers that cannot allocate: code being
 * captured into a HIP graph on a stream that never ran the sampler eagerly,
 * tight serving loops, and harnesses that forbid hipMalloc.  Limit:
 * n <= 262144 logits (SLTX_ERR_INVALID beyond).  The scratch is one
 * 3,315,968-byte device array per GPU, held until the process ends and
 * shared by every call on that GPU: calls that overlap on one GPU (on other
 * streams or threads) race on it and must be ordered by the caller. */
int sltx_sample_top_p_noalloc(const void* logits, int32_t dtype, int32_t n, float temperature,
                              float top_p, float repetition_penalty, const int32_t* seen,
                              int32_t n_seen, float u, int32_t* out_index, void* stream);

/* Sampler state kept in device memory, so that a sampled decode step takes no
 * per-token host argument and can be captured once as a HIP graph.  The
 * reference keeps the same state on the host: seenTokens = the prompt plus
 * every generated token (LlamaModel.swift:150-161) and Float.random for the
 * draw (Ops.swift:2092).  All pointers are device pointers, 4-byte aligned. */
typedef struct sltx_sample_state {
    int32_t* history;          /* token ids; history[0 .. *history_len) are the seen ids */
    int32_t* history_len;      /* [1] entries in use; clamped to [0, history_capacity] */
    int32_t history_capacity;  /* entries history can hold (>= 0) */
    const float* draws;        /* uniform draws in [0, 1): one per call */
    int32_t* next_draw;        /* [1] index of the next call's draw, taken modulo draw_count */
    int32_t draw_count;        /* entries in draws (>= 1) */
} sltx_sample_state;

/* sltx_sample_top_p with seen = history[0 .. *history_len) and
 * u = draws[*next_draw mod draw_count] read on the device (a draw outside
 * [0, 1), or NaN, is clamped into it).  After choosing, the call appends the
 * token to history (dropped once history_capacity entries are in use) and
 * sets *next_draw to the following index.  The reference has no separate
 * entry point for this: it is sample() with the state the reference keeps on
 * the host moved to device memory.  Calls on one state are ordered only by
 * their stream; calls that share a state on different streams race. */
int sltx_sample_top_p_state(const void* logits, int32_t dtype, int32_t n, float temperature,
                            float top_p, float repetition_penalty,
                            const sltx_sample_state* state, int32_t* out_index, void* stream);

/* Route query (no counterpart in the reference; for tests and tuning): the
 * kernel family sltx_matmul_q4_fast[_f32], sltx_matmul_q4_ex, the gated pair
 * entry points at M > 1 and sltx_matmul_q4_residual at M > 1 run for this
 * shape (gated: a gate/up pair), with 16-byte aligned operands.  Nothing is
 * launched and no device is needed.  Returns an sltx_route, or a negative
 * sltx_status for invalid arguments. */
typedef enum {
    SLTX_ROUTE_GEMM = 0,     /* MFMA GEMM, split over K when its tiles would not fill the GPU */
    SLTX_ROUTE_SMALL_M = 1,  /* small-M weight stream (M <= 32, 16x16x32 MFMA) */
    SLTX_ROUTE_NARROW = 2,   /* narrow weight stream (one weight set, M <= 4, 4x4x4 MFMA) */
    SLTX_ROUTE_MID = 3,      /* pipelined weight stream (8 < M <= 32, from M = 6 for a set of at most
                                4096 rows at K = 10240; X and W through LDS, 32x32x16 MFMA; such
                                sets split K in halves across blocks) */
    SLTX_ROUTE_WIDE = 4,     /* 32 < M <= 256: 64 weight rows per block over its K range, waves
                                split K; K split across blocks where the blocks are few */
    SLTX_ROUTE_GEMV = 5      /* M = 2, fp16 x, one weight set of at most 5120 x 4096: the GEMV
                                over both rows (each weight word dequantized once) */
} sltx_route;
int sltx_gemm_route(int32_t M, int32_t N, int32_t K, int32_t group_size, int32_t gated,
                    int32_t x_dtype);

/* ---- safetensors weights (SafeTensorsFile, SafeTensors.swift:41-118) ----
 * Reads the files swift-ltx's loader reads (ModelWeights.swift:40-154) into
 * caller-allocated device memory.  The header (8-byte LE length, JSON object,
 * optional "__metadata__") is parsed once at open; entries with other dtypes
 * are skipped as in the reference.  A tensor whose byte range does not match
 * its shape and dtype or lies outside the file makes the file invalid (the
 * reference would read out of bounds).  A file handle may be shared between
 * threads (device reads are serialised per handle). */
typedef struct sltx_st_file sltx_st_file;

/* TensorDType (SafeTensors.swift:15-31) */
typedef enum sltx_st_dtype {
    SLTX_ST_F32 = 0,
    SLTX_ST_F16 = 1,
    SLTX_ST_BF16 = 2,
    SLTX_ST_I8 = 3,
    SLTX_ST_U8 = 4,
    SLTX_ST_I32 = 5,
    SLTX_ST_U32 = 6
} sltx_st_dtype;

/* TensorInfo (SafeTensors.swift:7-13): offset is relative to the data region. */
typedef struct sltx_st_info {
    int32_t dtype;      /* sltx_st_dtype */
    int32_t ndim;       /* <= 8 */
    int64_t shape[8];
    uint64_t offset;
    uint64_t nbytes;
} sltx_st_info;

/* SafeTensorsFile(url:) (SafeTensors.swift:41-89).  *out is closed with
 * sltx_st_close. */
int sltx_st_open(const char* path, sltx_st_file** out);
void sltx_st_close(sltx_st_file* file);

/* Number of tensors, and their names in sorted order (index < count). */
int sltx_st_num_tensors(const sltx_st_file* file);
const char* sltx_st_name(const sltx_st_file* file, int32_t index);

/* tensors[name] (SafeTensors.swift:35): SLTX_ERR_INVALID if absent. */
int sltx_st_info_of(const sltx_st_file* file, const char* name, sltx_st_info* out);

/* readTensorRaw(_:into:) (SafeTensors.swift:205-214): raw bytes to host memory. */
int sltx_st_read_host(sltx_st_file* file, const char* name, void* dst, uint64_t capacity);

/* readTensorIntoBuffer (SafeTensors.swift:175-186) with a HIP device
 * destination: raw bytes, streamed through pinned staging buffers and
 * enqueued on stream; returns once the data is on the device.  Reading into
 * an offset of a larger allocation concatenates tensors (e.g. q|k|v rows). */
int sltx_st_read_device(sltx_st_file* file, const char* name, void* dst, uint64_t capacity,
                        void* stream);

/* loadFloat (ModelWeights.swift:96-108, bf16 branch of :66-75): an F32, F16
 * or BF16 tensor widened to fp32 on the host while streaming, count = capacity
 * in floats. */
int sltx_st_read_device_f32(sltx_st_file* file, const char* name, float* dst, uint64_t count,
                            void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SWIFTLTX_Q4_H */
