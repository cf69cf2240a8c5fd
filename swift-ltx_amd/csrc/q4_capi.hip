// q4_capi.hip -- the C ABI (include/swiftltx_q4.h): argument validation,
// routing and launch of the gfx950 kernels.  Validation runs before any HIP
// call, so error paths behave the same with or without a GPU.
#include <algorithm>
#include <cstdarg>
#include <map>
#include <mutex>
#include <tuple>
#include <utility>
#include <vector>
#include <string>
#include <cstdio>
#include <cstring>

#include "q4_common.hpp"
#include "q4_launch.hpp"
#include "swiftltx_q4.h"

namespace sltx {

thread_local std::string g_last_error;

// Records the thread's last error message and returns code (shared with the
// safetensors reader, q4_st.hip).
int set_error(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

namespace {

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(kErrHip, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int log2_group(int g) { return g == 32 ? 0 : g == 64 ? 1 : g == 128 ? 2 : -1; }

bool overlap(const void* a, size_t na, const void* b, size_t nb) {
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x < y + nb && y < x + na;
}

// Shape / pointer checks common to every matmul entry point.
int check_weight(const char* fn, const void* x, const uint32_t* w, const uint16_t* s,
                 const uint16_t* b, const void* out, int M, int K, int N, int g) {
    if (M < 0 || N < 0) return fail(kErrInvalid, "%s: negative M (%d) or N (%d)", fn, M, N);
    if (K <= 0) return fail(kErrInvalid, "%s: K must be positive (got %d)", fn, K);
    if (K % 32 != 0) return fail(kErrInvalid, "%s: K (%d) must be a multiple of 32", fn, K);
    if (g <= 0 || g % 8 != 0) return fail(kErrInvalid, "%s: group_size %d is not a positive multiple of 8", fn, g);
    if (K % g != 0) return fail(kErrInvalid, "%s: K (%d) is not a multiple of group_size (%d)", fn, K, g);
    if (log2_group(g) < 0)
        return fail(kErrUnsupported, "%s: group_size %d unsupported (32, 64 or 128)", fn, g);
    if (M == 0 || N == 0) return kOk;
    if (!x || !w || !s || !b || !out) return fail(kErrInvalid, "%s: null pointer argument", fn);
    if (!aligned(x, 16)) return fail(kErrInvalid, "%s: x must be 16-byte aligned", fn);
    if (!aligned(w, 16)) return fail(kErrInvalid, "%s: weight must be 16-byte aligned", fn);
    if (!aligned(s, 2) || !aligned(b, 2)) return fail(kErrInvalid, "%s: scales/biases must be 2-byte aligned", fn);
    return kOk;
}

// The output of a matmul must not overlap its activation input: every GEMV
// block re-reads x, and GEMM blocks read A tiles, while other blocks store.
int check_out_alias(const char* fn, const void* x, size_t xbytes, const void* out, size_t obytes) {
    if (overlap(x, xbytes, out, obytes)) return fail(kErrInvalid, "%s: out overlaps x", fn);
    return kOk;
}

// Once-per-device readiness check (gfx950 code object present and runnable).
std::mutex g_init_mu;
int g_dev_state[kMaxDevices];  // 0 unknown, 1 ok, -1 bad

int ensure_device() {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(kErrHip, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_init_mu);
    if (g_dev_state[dev] == 1) return kOk;
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        g_dev_state[dev] = -1;
        return fail(kErrUnsupported, "device %d is %s; this library is built for gfx950 only", dev,
                    prop.gcnArchName);
    }
    // the allocation-free sampler's scratch address on this device
    const int rc = sample_noalloc_scratch_init(dev);
    if (rc != kOk) return rc;
    g_dev_state[dev] = 1;
    return kOk;
}

int finish(hipError_t e, const char* fn) {
    if (e != hipSuccess) return hip_fail(e, fn);
    return kOk;
}

// Optional GEMV prologue / epilogue operands (see GemvParams).
struct GemvFuse {
    int pro = kProNone;
    const void* xb = nullptr;
    const float* norm_w = nullptr;
    float eps = 0.0f;
    void* res_out = nullptr;
    const void* residual = nullptr;
    bool gelu = false;
};

int run_gemv(const char* fn, const void* x, const sltx_q4_weight& w0, const sltx_q4_weight* w1,
             void* out, int K, int N, hipStream_t st, const GemvFuse& fz = GemvFuse()) {
    GemvParams p;
    p.x = static_cast<const uint16_t*>(x);
    p.w0 = w0.weight;
    p.s0 = w0.scales;
    p.b0 = w0.biases;
    p.w1 = w1 ? w1->weight : nullptr;
    p.s1 = w1 ? w1->scales : nullptr;
    p.b1 = w1 ? w1->biases : nullptr;
    p.y = static_cast<uint16_t*>(out);
    p.N = N;
    p.K = K;
    p.groups = K / w0.group_size;
    p.gshift = log2_group(w0.group_size);
    p.pro = fz.pro;
    p.xb = static_cast<const uint16_t*>(fz.xb);
    p.norm_w = fz.norm_w;
    p.eps = fz.eps;
    p.res_out = static_cast<uint16_t*>(fz.res_out);
    p.residual = static_cast<const uint16_t*>(fz.residual);
    p.gelu = fz.gelu ? 1 : 0;
    p.rows = 1;
    p.y_dtype = kF16;
    p.bias = nullptr;
    p.gelu_tanh = 0;
    return finish(launch_gemv(p, w1 != nullptr, st), fn);
}

// Two x rows on the GEMV (SLTX_ROUTE_GEMV): the M > 1 operands of p.
hipError_t launch_gemv2(const GemmParams& g, hipStream_t st) {
    GemvParams p;
    p.x = static_cast<const uint16_t*>(g.a);
    p.w0 = g.w0;
    p.s0 = g.s0;
    p.b0 = g.b0;
    p.w1 = g.w1;
    p.s1 = g.s1;
    p.b1 = g.b1;
    p.y = static_cast<uint16_t*>(g.y);
    p.N = g.N;
    p.K = g.K;
    p.groups = g.groups;
    p.gshift = g.gshift;
    p.pro = kProNone;
    p.xb = nullptr;
    p.norm_w = nullptr;
    p.eps = 0.0f;
    p.res_out = nullptr;
    p.residual = g.epilogue == kEpiResidual ? g.residual : nullptr;
    p.gelu = g.epilogue == kEpiGeluMul ? 1 : 0;
    p.rows = 2;
    p.y_dtype = g.y_dtype;
    p.bias = g.w1 ? nullptr : g.bias;
    p.gelu_tanh = !g.w1 && g.epilogue == kEpiGeluTanh ? 1 : 0;
    return launch_gemv(p, g.w1 != nullptr, st);
}

// Per-stream workspace (split-K partial sums, sampling scratch), one per
// (device, stream): calls on one stream are ordered, so they can share it;
// other streams get their own.  It grows on
// demand to at least twice its old size.  A replaced buffer is never freed:
// graphs captured earlier may still name it, so it is kept (with the current
// one) until the process ends; doubling bounds the retired total by the
// current size.  A stream that is being captured into a graph never
// allocates: if its workspace is missing or too small the GEMM runs unsplit
// and sampling returns an error.
// A stream has two such buffers: slot 0 for the kernels' scratch, slot 1 for
// the fp16 copy of fp32 activations that sltx_matmul_q4_ex casts before a
// GEMM whose scratch is in slot 0.  Slot 0 starts with the split-K arrival
// counters (kTicketBytes, zeroed on the stream when the buffer is allocated;
// each launch that uses them leaves them zero); `tickets` receives their
// address and the scratch follows them.
// sltx_release_workspace frees one stream's buffers (current and retired).
struct StreamWs {
    void* ptr = nullptr;
    size_t bytes = 0;
    std::vector<void*> retired;
};
std::mutex g_ws_mu;
std::map<std::tuple<int, hipStream_t, int>, StreamWs> g_ws;

float* stream_workspace(hipStream_t st, size_t need, int slot = 0, unsigned** tickets = nullptr) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    const size_t head = slot == 0 ? kTicketBytes : 0;
    need += head;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    auto& e = g_ws[{dev, st, slot}];
    if (e.bytes < need) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
            return nullptr;
        void* ptr = nullptr;
        const size_t bytes = std::max(need + need / 4, 2 * e.bytes);
        if (hipMalloc(&ptr, bytes) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        // not capturing: an ordinary memset ahead of the stream's later work
        if (head && hipMemsetAsync(ptr, 0, head, st) != hipSuccess) {
            (void)hipGetLastError();
            (void)hipFree(ptr);
            return nullptr;
        }
        if (e.ptr) e.retired.push_back(e.ptr);
        e.ptr = ptr;
        e.bytes = bytes;
    }
    if (tickets) *tickets = head ? static_cast<unsigned*>(e.ptr) : nullptr;
    return reinterpret_cast<float*>(static_cast<char*>(e.ptr) + head);
}

int release_workspace(hipStream_t st) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return hip_fail(err, "hipGetDevice");
    std::vector<void*> bufs;
    {
        std::lock_guard<std::mutex> lk(g_ws_mu);
        auto i0 = g_ws.find({dev, st, 0}), i1 = g_ws.find({dev, st, 1});
        if (i0 == g_ws.end() && i1 == g_ws.end()) return kOk;
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
            return fail(kErrInvalid, "sltx_release_workspace: the stream is being captured");
        for (auto it : {i0, i1}) {
            if (it == g_ws.end()) continue;
            bufs.insert(bufs.end(), it->second.retired.begin(), it->second.retired.end());
            bufs.push_back(it->second.ptr);
            g_ws.erase(it);
        }
    }
    // the stream's queued work may still use the buffers
    err = hipStreamSynchronize(st);
    if (err != hipSuccess) return hip_fail(err, "hipStreamSynchronize");
    for (void* p : bufs)
        if (p && (err = hipFree(p)) != hipSuccess) return hip_fail(err, "hipFree");
    return kOk;
}

// The route run_gemm takes for p (SLTX_ROUTE_*), and the plans it launches
// with.  One weight set at M <= 4: the narrow route (4x4x4 MFMA blocks,
// whole-line loads), unless the small-M route runs two row tiles per block
// at two blocks per CU (tall matrices such as the vocabulary head).
// Measured on the Llama, T5 and vocabulary-head shapes at M = 2, 4, 8, that
// is the faster route in every case; gated pairs and M > 4 are faster on the
// small-M route, up to M = 16.
int gemm_route(const GemmParams& p, bool a_bf16, NarrowPlan* np, SkinnyPlan* sp, WidePlan* wp) {
    if (p.a_f32) return SLTX_ROUTE_GEMM;   // the only kernel that casts fp32 activations
    // Two rows of fp16 x through one weight set of at most 5120 x 4096: the
    // GEMV, each weight word dequantized once for both rows.  Measured (us,
    // weights rotated over >= 2 GB) against the narrow route: Llama o 3.48 /
    // 4.11, q|k|v 5.18 / 5.35, T5 q/k/v/o 4.54 / 4.78; slower for Llama down
    // (K = 8192: 7.20 / 6.73) and, for the gate/up pair, than the small-M
    // route (8.98 / 8.74).
    if (p.M == 2 && !a_bf16 && p.w1 == nullptr && p.K <= 4096 && p.N <= 5120 &&
        gemv2_ok(p.N, p.K))
        return SLTX_ROUTE_GEMV;
    if (p.M > 32) return wide_plan(p, a_bf16, wp) ? SLTX_ROUTE_WIDE : SLTX_ROUTE_GEMM;
    const bool narrow = narrow_plan(p, a_bf16, np);
    const bool skinny = skinny_plan(p, a_bf16, sp);
    if (narrow && (!skinny || !(sp->RT == 2 && sp->OCC == 2))) return SLTX_ROUTE_NARROW;
    // The mid-M route: above 16 rows where it is built (at K > 3072 only
    // where the small-M route cannot run or above 24 rows), and one weight
    // set of 4096..16384 rows at K <= 3072 above 8 rows.  Measured (us per
    // launch, weights rotated over >= 2 GB), mid-M against small-M / GEMM:
    // - M = 20, 24, 32: Llama gate/up pair 11.7-11.9 against 13.4-15.3,
    //   q|k|v (5120 x 3072) 6.6-6.7 against 11.8-14.9, o (3072 x 3072)
    //   6.3-6.4 against 7.4-8.8, a single 8192 x 3072 set 7.4-7.6 against
    //   8.8-10.4; Llama down (3072 x 8192) 15.4 against the GEMM's 22.8-23.0,
    //   T5 wo (4096 x 10240) 14.4-14.9 against the GEMM's 26.9-28;
    //   T5 q/k/v/o (4096 x 4096) 9.9 / 9.9 / 9.9 against 8.9 / 9.6 / 10.9;
    //   the T5 GeGLU pair (2 x 10240 x 4096) 31.5 at M = 25-32 against 36.7
    //   at M = 32;
    // - M = 12, 16: q|k|v 6.5 against 8.5 / 9.5, the 8192-row set 7.3
    //   against 7.3 / 7.7; o 6.2 against 5.7 / 6.1, T5 q/k/v/o 9.8 against
    //   6.7 / 7.3, the vocabulary head (M = 8) 87 against 62 us.
    // One weight set that the mid-M route splits over K in two halves
    // (mid_splits: N <= 4096, K = 4096, 8192 or 10240) takes it above 5 rows
    // at K = 10240, 12 at K = 8192 and 16 at K = 4096.  Measured against the
    // small-M route: T5 wo 11.1 / 11.1 / 11.1 against 11.1 / 11.5 / 12.5 us
    // at M = 5 / 6 / 8, 10.9-11.2 against 12.6 / 14.3 / 16.0 at M = 9 / 12 /
    // 16; Llama down 11.4-11.5 against 10.3 / 11.2 / 12.6 at M = 10 / 12 /
    // 16; T5 q/k/v/o 7.9-8.1 against 6.9 / 7.3 / 8.9 / 9.6 at M = 14 / 16 /
    // 20 / 24.
    const bool kshort = p.K <= 3072;
    const bool mid_rows = (p.M > 16 && (kshort || !skinny || p.M > 24)) ||
                          (p.M > 8 && kshort && p.w1 == nullptr && p.N >= 4096 && p.N <= 16384) ||
                          (mid_splits(p) == 2 && p.M > (p.K >= 10240 ? 5 : p.K >= 8192 ? 12 : 16));
    if (mid_rows && mid_plan(p, a_bf16)) return SLTX_ROUTE_MID;
    if (skinny) return SLTX_ROUTE_SMALL_M;
    return SLTX_ROUTE_GEMM;
}

int run_gemm(const char* fn, const void* x, int x_dtype, const sltx_q4_weight& w0,
             const sltx_q4_weight* w1, const float* bias, int epilogue, void* out, int y_dtype,
             int M, int K, int N, hipStream_t st, const void* residual = nullptr) {
    GemmParams p{};
    p.a = x;
    p.w0 = w0.weight;
    p.s0 = w0.scales;
    p.b0 = w0.biases;
    p.w1 = w1 ? w1->weight : nullptr;
    p.s1 = w1 ? w1->scales : nullptr;
    p.b1 = w1 ? w1->biases : nullptr;
    p.bias = bias;
    p.y = out;
    p.M = M;
    p.N = N;
    p.K = K;
    p.groups = K / w0.group_size;
    p.gshift = log2_group(w0.group_size);
    p.tiles_m = p.tiles_n = 0;
    p.y_dtype = y_dtype;
    p.epilogue = w1 ? (epilogue == kEpiGeluMul ? kEpiGeluMul : kEpiSiluMul) : epilogue;
    p.residual = static_cast<const uint16_t*>(residual);
    p.ws = nullptr;
    p.splits = 1;
    p.split_tiles = 0;
    p.a_f32 = x_dtype == kF32 ? 1 : 0;
    NarrowPlan np;
    SkinnyPlan sp;
    WidePlan wp;
    const int route = gemm_route(p, x_dtype == kBF16, &np, &sp, &wp);
    if (route == SLTX_ROUTE_NARROW) return finish(launch_narrow(p, np, st), fn);
    if (route == SLTX_ROUTE_SMALL_M) return finish(launch_skinny(p, sp, st), fn);
    if (route == SLTX_ROUTE_GEMV) return finish(launch_gemv2(p, st), fn);
    if (route == SLTX_ROUTE_MID) {
        // two K halves where the blocks are few, when the stream's workspace
        // exists (not first allocated under capture); else the whole K
        int splits = mid_splits(p);
        if (splits > 1 && !(p.ws = stream_workspace(st, mid_ws_bytes(p, splits), 0, &p.tickets)))
            splits = 1;
        return finish(launch_mid(p, splits, st), fn);
    }
    if (route == SLTX_ROUTE_WIDE) {
        if (wp.splits > 1 && !(p.ws = stream_workspace(st, wp.ws_bytes, 0, &p.tickets))) {
            // no workspace (the stream is being captured): the same product
            // through the GEMM
            const size_t need = gemm_workspace_bytes(p);
            if (need > 0) p.ws = stream_workspace(st, need);
            return finish(launch_gemm(p, x_dtype == kBF16, st), fn);
        }
        return finish(launch_wide(p, wp, st), fn);
    }
    const size_t need = gemm_workspace_bytes(p);
    if (need > 0) p.ws = stream_workspace(st, need);
    return finish(launch_gemm(p, x_dtype == kBF16, st), fn);
}

int matmul_common(const char* fn, const void* x, const uint32_t* weight, const uint16_t* scales,
                  const uint16_t* biases, void* out, int M, int K, int N, int g, int y_dtype,
                  bool force_gemm, void* stream) {
    int rc = check_weight(fn, x, weight, scales, biases, out, M, K, N, g);
    if (rc != kOk) return rc;
    if (!aligned(out, y_dtype == kF32 ? 4 : 2)) return fail(kErrInvalid, "%s: misaligned out", fn);
    if (M == 0 || N == 0) return kOk;
    if ((rc = check_out_alias(fn, x, (size_t)M * K * 2, out,
                              (size_t)M * N * (y_dtype == kF32 ? 4 : 2))) != kOk)
        return rc;
    if ((rc = ensure_device()) != kOk) return rc;
    const sltx_q4_weight w = {weight, scales, biases, K, g};
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (M == 1 && !force_gemm && y_dtype == kF16) return run_gemv(fn, x, w, nullptr, out, K, N, st);
    return run_gemm(fn, x, kF16, w, nullptr, nullptr, kEpiNone, out, y_dtype, M, K, N, st);
}

// Checks shared by both sampling entry points.
int check_sample(const char* fn, const void* logits, int dtype, int n, float temperature,
                 float top_p, float repetition_penalty, const int32_t* out_index) {
    if (n <= 0) return fail(kErrInvalid, "%s: n must be positive (got %d)", fn, n);
    if (n > (1 << 24)) return fail(kErrInvalid, "%s: n = %d exceeds 2^24 tokens", fn, n);
    if (dtype != kF16 && dtype != kF32)
        return fail(kErrInvalid, "%s: dtype %d must be SLTX_F16 or SLTX_F32", fn, dtype);
    if (!(temperature > 0.0f) || !(top_p > 0.0f) || !(repetition_penalty > 0.0f))
        return fail(kErrInvalid, "%s: temperature, top_p and repetition_penalty must be positive", fn);
    if (!logits || !out_index) return fail(kErrInvalid, "%s: null pointer argument", fn);
    if (!aligned(logits, dtype == kF32 ? 4 : 2) || !aligned(out_index, 4))
        return fail(kErrInvalid, "%s: misaligned pointer", fn);
    return kOk;
}

int run_sample(const char* fn, SampleParams& p, void* stream) {
    int rc = ensure_device();
    if (rc != kOk) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    void* ws = stream_workspace(st, sample_workspace_bytes(p.n));
    if (!ws)
        return fail(kErrInvalid,
                    "%s: no workspace for n = %d on this stream (it is being captured: sample "
                    "once eagerly on the same stream first)", fn, p.n);
    return finish(launch_sample(p, ws, st), fn);
}

SampleParams sample_params(const void* logits, int dtype, int n, float temperature, float top_p,
                           float repetition_penalty, int32_t* out_index) {
    SampleParams p = {};
    p.logits = logits;
    p.dtype = dtype;
    p.n = n;
    p.temperature = temperature;
    p.top_p = top_p;
    p.penalty = repetition_penalty;
    p.out = out_index;
    return p;
}

}  // namespace
}  // namespace sltx

using namespace sltx;

extern "C" {

int sltx_abi_version(void) { return 1; }

int sltx_init(void) { return ensure_device(); }

int sltx_release_workspace(void* stream) {
    return release_workspace(static_cast<hipStream_t>(stream));
}

const char* sltx_last_error(void) { return g_last_error.c_str(); }

int sltx_matmul_q4(const void* x, const uint32_t* weight, const uint16_t* scales,
                   const uint16_t* biases, void* out, int32_t M, int32_t K, int32_t N,
                   int32_t group_size, void* stream) {
    return matmul_common("sltx_matmul_q4", x, weight, scales, biases, out, M, K, N, group_size,
                         kF16, false, stream);
}

int sltx_matmul_q4_fast(const void* x, const uint32_t* weight, const uint16_t* scales,
                        const uint16_t* biases, void* out, int32_t M, int32_t K, int32_t N,
                        int32_t group_size, void* stream) {
    return matmul_common("sltx_matmul_q4_fast", x, weight, scales, biases, out, M, K, N,
                         group_size, kF16, true, stream);
}

int sltx_matmul_q4_fast_f32(const void* x, const uint32_t* weight, const uint16_t* scales,
                            const uint16_t* biases, float* out, int32_t M, int32_t K, int32_t N,
                            int32_t group_size, void* stream) {
    return matmul_common("sltx_matmul_q4_fast_f32", x, weight, scales, biases, out, M, K, N,
                         group_size, kF32, true, stream);
}

int sltx_silu_mul(const void* a, const void* b, void* out, int64_t count, void* stream) {
    const char* fn = "sltx_silu_mul";
    if (count < 0) return fail(kErrInvalid, "%s: negative count", fn);
    if (count == 0) return kOk;
    if (!a || !b || !out) return fail(kErrInvalid, "%s: null pointer argument", fn);
    if (!aligned(a, 2) || !aligned(b, 2) || !aligned(out, 2))
        return fail(kErrInvalid, "%s: pointers must be 2-byte aligned", fn);
    int rc = ensure_device();
    if (rc != kOk) return rc;
    return finish(launch_silu_mul(static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b),
                                  static_cast<uint16_t*>(out), (long)count,
                                  static_cast<hipStream_t>(stream)),
                  fn);
}

int sltx_linear(const void* x, const sltx_q4_weight* w, void* out, int32_t M, int32_t K,
                int32_t N, int32_t fast, void* stream) {
    const char* fn = "sltx_linear";
    if (!w) return fail(kErrInvalid, "%s: null weight descriptor", fn);
    if (w->K != K) return fail(kErrInvalid, "%s: weight K (%d) != K (%d)", fn, w->K, K);
    if (fast && M > 1)
        return matmul_common(fn, x, w->weight, w->scales, w->biases, out, M, K, N, w->group_size,
                             kF16, true, stream);
    return matmul_common(fn, x, w->weight, w->scales, w->biases, out, M, K, N, w->group_size, kF16,
                         false, stream);
}

int sltx_matmul_q4_silu_mul(const void* x, const sltx_q4_weight* gate, const sltx_q4_weight* up,
                            void* out, int32_t M, int32_t K, int32_t N, void* stream) {
    const char* fn = "sltx_matmul_q4_silu_mul";
    if (!gate || !up) return fail(kErrInvalid, "%s: null weight descriptor", fn);
    if (gate->K != K || up->K != K) return fail(kErrInvalid, "%s: weight K mismatch", fn);
    if (gate->group_size != up->group_size)
        return fail(kErrInvalid, "%s: gate and up group_size differ", fn);
    int rc = check_weight(fn, x, gate->weight, gate->scales, gate->biases, out, M, K, N,
                          gate->group_size);
    if (rc != kOk) return rc;
    rc = check_weight(fn, x, up->weight, up->scales, up->biases, out, M, K, N, up->group_size);
    if (rc != kOk) return rc;
    if (!aligned(out, 2)) return fail(kErrInvalid, "%s: misaligned out", fn);
    if (M == 0 || N == 0) return kOk;
    if ((rc = check_out_alias(fn, x, (size_t)M * K * 2, out, (size_t)M * N * 2)) != kOk) return rc;
    if ((rc = ensure_device()) != kOk) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (M == 1) return run_gemv(fn, x, *gate, up, out, K, N, st);
    return run_gemm(fn, x, kF16, *gate, up, nullptr, kEpiNone, out, kF16, M, K, N, st);
}

int sltx_matmul_q4_ex(const void* x, int32_t x_dtype, const sltx_q4_weight* w, const float* bias,
                      int32_t epilogue, void* out, int32_t out_dtype, int32_t M, int32_t N,
                      void* stream) {
    const char* fn = "sltx_matmul_q4_ex";
    if (!w) return fail(kErrInvalid, "%s: null weight descriptor", fn);
    if (x_dtype != kF16 && x_dtype != kBF16 && x_dtype != kF32)
        return fail(kErrInvalid, "%s: x_dtype %d must be SLTX_F16, SLTX_BF16 or SLTX_F32", fn,
                    x_dtype);
    if (out_dtype != kF16 && out_dtype != kBF16 && out_dtype != kF32)
        return fail(kErrInvalid, "%s: out_dtype %d invalid", fn, out_dtype);
    if (epilogue != kEpiNone && epilogue != kEpiGeluTanh)
        return fail(kErrInvalid, "%s: epilogue %d invalid", fn, epilogue);
    int rc = check_weight(fn, x, w->weight, w->scales, w->biases, out, M, w->K, N, w->group_size);
    if (rc != kOk) return rc;
    if (!aligned(out, out_dtype == kF32 ? 4 : 2)) return fail(kErrInvalid, "%s: misaligned out", fn);
    if (bias && !aligned(bias, 4)) return fail(kErrInvalid, "%s: misaligned bias", fn);
    if (M == 0 || N == 0) return kOk;
    if ((rc = check_out_alias(fn, x, (size_t)M * w->K * (x_dtype == kF32 ? 4 : 2), out,
                              (size_t)M * N * (out_dtype == kF32 ? 4 : 2))) != kOk)
        return rc;
    if ((rc = ensure_device()) != kOk) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (x_dtype == kF32 && N > 2 * 256) {
        // Wide outputs: the fused cast (the GEMM's fp32 staging) would be
        // repeated by every one of the GEMM's column blocks, so x is cast once
        // into the stream's second buffer and the fp16 routes run.  Measured
        // at the DiT up shape (M = 6144, N = 8192, K = 2048): 343 us fused
        // against 220 us for bf16 x.  Without that buffer (a stream being
        // captured that never ran this shape eagerly) the fused cast runs.
        const size_t xb = (size_t)M * w->K * 2;
        void* x16 = stream_workspace(st, xb, 1);
        if (x16) {
            hipError_t e = launch_cast_f32_f16(static_cast<const float*>(x), static_cast<uint16_t*>(x16),
                                               (long)M * w->K, st);
            if (e != hipSuccess) return finish(e, fn);
            return run_gemm(fn, x16, kF16, *w, nullptr, bias, epilogue, out, out_dtype, M, w->K, N,
                            st);
        }
    }
    return run_gemm(fn, x, x_dtype, *w, nullptr, bias, epilogue, out, out_dtype, M, w->K, N, st);
}

int sltx_matmul_q4_geglu(const void* x, const sltx_q4_weight* gate, const sltx_q4_weight* up,
                         void* out, int32_t M, int32_t K, int32_t N, void* stream) {
    const char* fn = "sltx_matmul_q4_geglu";
    if (!gate || !up) return fail(kErrInvalid, "%s: null weight descriptor", fn);
    if (gate->K != K || up->K != K) return fail(kErrInvalid, "%s: weight K mismatch", fn);
    if (gate->group_size != up->group_size)
        return fail(kErrInvalid, "%s: gate and up group_size differ", fn);
    int rc = check_weight(fn, x, gate->weight, gate->scales, gate->biases, out, M, K, N,
                          gate->group_size);
    if (rc != kOk) return rc;
    rc = check_weight(fn, x, up->weight, up->scales, up->biases, out, M, K, N, up->group_size);
    if (rc != kOk) return rc;
    if (!aligned(out, 2)) return fail(kErrInvalid, "%s: misaligned out", fn);
    if (M == 0 || N == 0) return kOk;
    if ((rc = check_out_alias(fn, x, (size_t)M * K * 2, out, (size_t)M * N * 2)) != kOk) return rc;
    if ((rc = ensure_device()) != kOk) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (M == 1) {
        GemvFuse fz;
        fz.gelu = true;
        return run_gemv(fn, x, *gate, up, out, K, N, st, fz);
    }
    return run_gemm(fn, x, kF16, *gate, up, nullptr, kEpiGeluMul, out, kF16, M, K, N, st);
}

int sltx_embedding_q4(const sltx_q4_weight* table, int32_t vocab, const int32_t* token_ids,
                      int32_t n, void* out, void* stream) {
    const char* fn = "sltx_embedding_q4";
    if (!table) return fail(kErrInvalid, "%s: null weight descriptor", fn);
    if (vocab < 0 || n < 0) return fail(kErrInvalid, "%s: negative vocab (%d) or n (%d)", fn, vocab, n);
    const int K = table->K, g = table->group_size;
    if (K <= 0 || K % 32 != 0) return fail(kErrInvalid, "%s: K (%d) must be a positive multiple of 32", fn, K);
    if (g <= 0 || g % 8 != 0 || K % g != 0)
        return fail(kErrInvalid, "%s: group_size %d invalid for K %d", fn, g, K);
    if (log2_group(g) < 0) return fail(kErrUnsupported, "%s: group_size %d unsupported (32, 64 or 128)", fn, g);
    if (n == 0) return kOk;
    if (!table->weight || !table->scales || !table->biases || !token_ids || !out)
        return fail(kErrInvalid, "%s: null pointer argument", fn);
    if (!aligned(table->weight, 4) || !aligned(table->scales, 2) || !aligned(table->biases, 2) ||
        !aligned(token_ids, 4) || !aligned(out, 16))
        return fail(kErrInvalid, "%s: misaligned pointer (out must be 16-byte aligned)", fn);
    int rc = ensure_device();
    if (rc != kOk) return rc;
    EmbedParams p;
    p.w = table->weight;
    p.s = table->scales;
    p.b = table->biases;
    p.ids = token_ids;
    p.out = static_cast<uint16_t*>(out);
    p.vocab = vocab;
    p.K = K;
    p.groups = K / g;
    p.glog2 = log2_group(g) + 5;
    return finish(launch_embedding_q4(p, n, static_cast<hipStream_t>(stream)), fn);
}

int sltx_argmax(const void* logits, int32_t dtype, int32_t n, int32_t* out_index, void* stream) {
    const char* fn = "sltx_argmax";
    if (n <= 0) return fail(kErrInvalid, "%s: n must be positive (got %d)", fn, n);
    if (dtype != kF16 && dtype != kF32)
        return fail(kErrInvalid, "%s: dtype %d must be SLTX_F16 or SLTX_F32", fn, dtype);
    if (!logits || !out_index) return fail(kErrInvalid, "%s: null pointer argument", fn);
    if (!aligned(logits, dtype == kF32 ? 4 : 2) || !aligned(out_index, 4))
        return fail(kErrInvalid, "%s: misaligned pointer", fn);
    int rc = ensure_device();
    if (rc != kOk) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    void* ws = stream_workspace(st, argmax_workspace_bytes());
    if (!ws)
        return fail(kErrInvalid,
                    "%s: no workspace on this stream (it is being captured: call it once eagerly "
                    "on the same stream first)", fn);
    return finish(launch_argmax(logits, dtype, n, out_index, ws, st), fn);
}

int sltx_sample_top_p(const void* logits, int32_t dtype, int32_t n, float temperature,
                      float top_p, float repetition_penalty, const int32_t* seen, int32_t n_seen,
                      float u, int32_t* out_index, void* stream) {
    const char* fn = "sltx_sample_top_p";
    int rc = check_sample(fn, logits, dtype, n, temperature, top_p, repetition_penalty, out_index);
    if (rc != kOk) return rc;
    if (!(u >= 0.0f && u < 1.0f)) return fail(kErrInvalid, "%s: u must lie in [0, 1)", fn);
    if (n_seen < 0) return fail(kErrInvalid, "%s: negative n_seen", fn);
    if (n_seen > 0 && !seen) return fail(kErrInvalid, "%s: null pointer argument", fn);
    if (seen && !aligned(seen, 4)) return fail(kErrInvalid, "%s: misaligned pointer", fn);
    SampleParams p = sample_params(logits, dtype, n, temperature, top_p, repetition_penalty, out_index);
    p.u = u;
    p.seen = seen;
    p.n_seen = n_seen;
    return run_sample(fn, p, stream);
}

int sltx_sample_top_p_noalloc(const void* logits, int32_t dtype, int32_t n, float temperature,
                              float top_p, float repetition_penalty, const int32_t* seen,
                              int32_t n_seen, float u, int32_t* out_index, void* stream) {
    const char* fn = "sltx_sample_top_p_noalloc";
    int rc = check_sample(fn, logits, dtype, n, temperature, top_p, repetition_penalty, out_index);
    if (rc != kOk) return rc;
    if (n > kSampleNoAllocMaxN)
        return fail(kErrInvalid, "%s: n = %d exceeds the %d logits its fixed scratch holds", fn, n,
                    kSampleNoAllocMaxN);
    if (!(u >= 0.0f && u < 1.0f)) return fail(kErrInvalid, "%s: u must lie in [0, 1)", fn);
    if (n_seen < 0) return fail(kErrInvalid, "%s: negative n_seen", fn);
    if (n_seen > 0 && !seen) return fail(kErrInvalid, "%s: null pointer argument", fn);
    if (seen && !aligned(seen, 4)) return fail(kErrInvalid, "%s: misaligned pointer", fn);
    if ((rc = ensure_device()) != kOk) return rc;
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    void* ws = sample_noalloc_scratch(dev);
    if (!ws) return fail(kErrHip, "%s: no scratch address for device %d", fn, dev);
    SampleParams p = sample_params(logits, dtype, n, temperature, top_p, repetition_penalty, out_index);
    p.u = u;
    p.seen = seen;
    p.n_seen = n_seen;
    return finish(launch_sample(p, ws, static_cast<hipStream_t>(stream)), fn);
}

int sltx_sample_top_p_state(const void* logits, int32_t dtype, int32_t n, float temperature,
                            float top_p, float repetition_penalty, const sltx_sample_state* state,
                            int32_t* out_index, void* stream) {
    const char* fn = "sltx_sample_top_p_state";
    int rc = check_sample(fn, logits, dtype, n, temperature, top_p, repetition_penalty, out_index);
    if (rc != kOk) return rc;
    if (!state) return fail(kErrInvalid, "%s: null state", fn);
    const sltx_sample_state& s = *state;
    if (s.history_capacity < 0) return fail(kErrInvalid, "%s: negative history_capacity", fn);
    if (s.draw_count < 1) return fail(kErrInvalid, "%s: draw_count must be at least 1", fn);
    if (!s.history_len || !s.draws || !s.next_draw || (s.history_capacity > 0 && !s.history))
        return fail(kErrInvalid, "%s: null pointer in state", fn);
    if (!aligned(s.history_len, 4) || !aligned(s.draws, 4) || !aligned(s.next_draw, 4) ||
        (s.history && !aligned(s.history, 4)))
        return fail(kErrInvalid, "%s: misaligned pointer in state", fn);
    SampleParams p = sample_params(logits, dtype, n, temperature, top_p, repetition_penalty, out_index);
    p.seen = s.history;
    p.hist = s.history;
    p.hist_len = s.history_len;
    p.hist_cap = s.history_capacity;
    p.u_seq = s.draws;
    p.u_next = s.next_draw;
    p.u_count = s.draw_count;
    return run_sample(fn, p, stream);
}

int sltx_rms_norm(const void* x, const float* weight, float eps, void* out, int32_t rows,
                  int32_t dim, void* stream) {
    const char* fn = "sltx_rms_norm";
    if (rows < 0 || dim < 0) return fail(kErrInvalid, "%s: negative rows (%d) or dim (%d)", fn, rows, dim);
    if (rows == 0 || dim == 0) return kOk;
    if (!x || !weight || !out) return fail(kErrInvalid, "%s: null pointer argument", fn);
    if (!aligned(x, 2) || !aligned(out, 2) || !aligned(weight, 4))
        return fail(kErrInvalid, "%s: misaligned pointer", fn);
    // In place (out == x) is safe: each element is read and written by one
    // thread of its row's block.  Any other overlap races across blocks.
    const size_t nb = (size_t)rows * dim * 2;
    if (out != x && overlap(out, nb, x, nb))
        return fail(kErrInvalid, "%s: out and x overlap without being equal", fn);
    int rc = ensure_device();
    if (rc != kOk) return rc;
    return finish(launch_rms_norm(static_cast<const uint16_t*>(x), nullptr, weight, eps, nullptr,
                                  static_cast<uint16_t*>(out), rows, dim,
                                  static_cast<hipStream_t>(stream)),
                  fn);
}

int sltx_residual_rms_norm(const void* a, const void* b, const float* weight, float eps,
                           void* residual_out, void* norm_out, int32_t rows, int32_t dim,
                           void* stream) {
    const char* fn = "sltx_residual_rms_norm";
    if (rows < 0 || dim < 0) return fail(kErrInvalid, "%s: negative rows (%d) or dim (%d)", fn, rows, dim);
    if (rows == 0 || dim == 0) return kOk;
    if (!a || !b || !weight || !residual_out || !norm_out)
        return fail(kErrInvalid, "%s: null pointer argument", fn);
    if (!aligned(a, 2) || !aligned(b, 2) || !aligned(residual_out, 2) || !aligned(norm_out, 2) ||
        !aligned(weight, 4))
        return fail(kErrInvalid, "%s: misaligned pointer", fn);
    const size_t nb = (size_t)rows * dim * 2;
    if (overlap(residual_out, nb, norm_out, nb))
        return fail(kErrInvalid, "%s: residual_out and norm_out overlap", fn);
    // Each output may be an input itself (in place, e.g. h = h + o): every
    // element is read and written by one thread of its row's block.  Any
    // other overlap races across blocks.
    for (const void* in : {a, b}) {
        if (residual_out != in && overlap(residual_out, nb, in, nb))
            return fail(kErrInvalid, "%s: residual_out overlaps an input without being equal", fn);
        if (norm_out != in && overlap(norm_out, nb, in, nb))
            return fail(kErrInvalid, "%s: norm_out overlaps an input without being equal", fn);
    }
    int rc = ensure_device();
    if (rc != kOk) return rc;
    return finish(launch_rms_norm(static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b),
                                  weight, eps, static_cast<uint16_t*>(residual_out),
                                  static_cast<uint16_t*>(norm_out), rows, dim,
                                  static_cast<hipStream_t>(stream)),
                  fn);
}

int sltx_rmsnorm_matmul_q4(const void* x, const float* norm_weight, float eps,
                           const sltx_q4_weight* w, void* out, int32_t N, void* stream) {
    const char* fn = "sltx_rmsnorm_matmul_q4";
    if (!w) return fail(kErrInvalid, "%s: null weight descriptor", fn);
    int rc = check_weight(fn, x, w->weight, w->scales, w->biases, out, 1, w->K, N, w->group_size);
    if (rc != kOk) return rc;
    if (N == 0) return kOk;
    if (!norm_weight) return fail(kErrInvalid, "%s: null norm_weight", fn);
    if (!aligned(norm_weight, 16)) return fail(kErrInvalid, "%s: norm_weight must be 16-byte aligned", fn);
    if (!aligned(out, 2)) return fail(kErrInvalid, "%s: misaligned out", fn);
    if ((rc = check_out_alias(fn, x, (size_t)w->K * 2, out, (size_t)N * 2)) != kOk) return rc;
    if ((rc = ensure_device()) != kOk) return rc;
    GemvFuse fz;
    fz.pro = kProRms;
    fz.norm_w = norm_weight;
    fz.eps = eps;
    return run_gemv(fn, x, *w, nullptr, out, w->K, N, static_cast<hipStream_t>(stream), fz);
}

int sltx_residual_rmsnorm_matmul_q4_silu_mul(const void* a, const void* b,
                                             const float* norm_weight, float eps,
                                             void* residual_out, const sltx_q4_weight* gate,
                                             const sltx_q4_weight* up, void* out, int32_t N,
                                             void* stream) {
    const char* fn = "sltx_residual_rmsnorm_matmul_q4_silu_mul";
    if (!gate || !up) return fail(kErrInvalid, "%s: null weight descriptor", fn);
    if (gate->K != up->K) return fail(kErrInvalid, "%s: gate and up K differ", fn);
    if (gate->group_size != up->group_size)
        return fail(kErrInvalid, "%s: gate and up group_size differ", fn);
    const int K = gate->K;
    int rc = check_weight(fn, a, gate->weight, gate->scales, gate->biases, out, 1, K, N,
                          gate->group_size);
    if (rc != kOk) return rc;
    rc = check_weight(fn, a, up->weight, up->scales, up->biases, out, 1, K, N, up->group_size);
    if (rc != kOk) return rc;
    if (N == 0) return kOk;
    if (!b || !norm_weight || !residual_out) return fail(kErrInvalid, "%s: null pointer argument", fn);
    if (!aligned(b, 16) || !aligned(norm_weight, 16) || !aligned(residual_out, 16))
        return fail(kErrInvalid, "%s: b, norm_weight and residual_out must be 16-byte aligned", fn);
    if (!aligned(out, 2)) return fail(kErrInvalid, "%s: misaligned out", fn);
    const size_t kb = (size_t)K * 2;
    if (overlap(residual_out, kb, a, kb) || overlap(residual_out, kb, b, kb))
        return fail(kErrInvalid, "%s: residual_out overlaps an input", fn);
    const size_t ob = (size_t)N * 2;
    if (overlap(out, ob, a, kb) || overlap(out, ob, b, kb) || overlap(out, ob, residual_out, kb))
        return fail(kErrInvalid, "%s: out overlaps an input or residual_out", fn);
    if ((rc = ensure_device()) != kOk) return rc;
    GemvFuse fz;
    fz.pro = kProResidualRms;
    fz.xb = b;
    fz.norm_w = norm_weight;
    fz.eps = eps;
    fz.res_out = residual_out;
    return run_gemv(fn, a, *gate, up, out, K, N, static_cast<hipStream_t>(stream), fz);
}

int sltx_matmul_q4_residual(const void* x, const sltx_q4_weight* w, const void* residual,
                            void* out, int32_t M, int32_t N, void* stream) {
    const char* fn = "sltx_matmul_q4_residual";
    if (!w) return fail(kErrInvalid, "%s: null weight descriptor", fn);
    int rc = check_weight(fn, x, w->weight, w->scales, w->biases, out, M, w->K, N, w->group_size);
    if (rc != kOk) return rc;
    if (M == 0 || N == 0) return kOk;
    if (!residual) return fail(kErrInvalid, "%s: null residual", fn);
    if (!aligned(residual, 2) || !aligned(out, 2)) return fail(kErrInvalid, "%s: misaligned pointer", fn);
    const size_t ob = (size_t)M * N * 2;
    if (residual != out && overlap(residual, ob, out, ob))
        return fail(kErrInvalid, "%s: residual and out overlap without being equal", fn);
    if (overlap(x, (size_t)M * w->K * 2, out, ob)) return fail(kErrInvalid, "%s: out overlaps x", fn);
    if ((rc = ensure_device()) != kOk) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (M == 1) {
        GemvFuse fz;
        fz.residual = residual;
        return run_gemv(fn, x, *w, nullptr, out, w->K, N, st, fz);
    }
    return run_gemm(fn, x, kF16, *w, nullptr, nullptr, kEpiResidual, out, kF16, M, w->K, N, st,
                    residual);
}

int sltx_matmul_q4_residual_rms_norm(const void* x, const sltx_q4_weight* w, const void* residual,
                                     const float* norm_weight, float eps, int32_t M, int32_t N,
                                     int32_t sum_rounded, void* residual_out, void* norm_out,
                                     void* stream) {
    const char* fn = "sltx_matmul_q4_residual_rms_norm";
    if (!w) return fail(kErrInvalid, "%s: null weight descriptor", fn);
    int rc = check_weight(fn, x, w->weight, w->scales, w->biases, residual_out, M, w->K, N,
                          w->group_size);
    if (rc != kOk) return rc;
    if (M == 0 || N == 0) return kOk;
    if (!residual || !norm_weight || !norm_out) return fail(kErrInvalid, "%s: null pointer argument", fn);
    if (N % 8 != 0 || N > 16384)
        return fail(kErrUnsupported, "%s: N (%d) must be a multiple of 8 and at most 16384", fn, N);
    if (!aligned(residual, 16) || !aligned(residual_out, 16) || !aligned(norm_out, 16) ||
        !aligned(norm_weight, 16))
        return fail(kErrInvalid,
                    "%s: residual, residual_out, norm_out and norm_weight must be 16-byte aligned", fn);
    const size_t ob = (size_t)M * N * 2, xb = (size_t)M * w->K * 2;
    if (residual != residual_out && overlap(residual, ob, residual_out, ob))
        return fail(kErrInvalid, "%s: residual and residual_out overlap without being equal", fn);
    if (overlap(norm_out, ob, residual_out, ob) || overlap(norm_out, ob, residual, ob))
        return fail(kErrInvalid, "%s: norm_out overlaps residual or residual_out", fn);
    if (overlap(x, xb, residual_out, ob) || overlap(x, xb, norm_out, ob))
        return fail(kErrInvalid, "%s: an output overlaps x", fn);
    if ((rc = ensure_device()) != kOk) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    GemmParams p{};
    p.a = x;
    p.w0 = w->weight;
    p.s0 = w->scales;
    p.b0 = w->biases;
    p.w1 = nullptr;
    p.s1 = nullptr;
    p.b1 = nullptr;
    p.bias = nullptr;
    p.y = residual_out;   // not written by the GEMM: its output is the fp32 partials
    p.M = M;
    p.N = N;
    p.K = w->K;
    p.groups = w->K / w->group_size;
    p.gshift = log2_group(w->group_size);
    p.tiles_m = p.tiles_n = 0;
    p.y_dtype = kF16;
    p.epilogue = kEpiNone;
    p.residual = static_cast<const uint16_t*>(residual);
    p.splits = 1;
    p.split_tiles = 0;
    p.ws = stream_workspace(st, gemm_partials_workspace_bytes(p));
    if (!p.ws)
        return fail(kErrInvalid,
                    "%s: no workspace on this stream (it is being captured: call it once eagerly "
                    "on the same stream first)", fn);
    return finish(launch_gemm_residual_rms_norm(p, false, norm_weight, eps,
                                                static_cast<uint16_t*>(residual_out),
                                                static_cast<uint16_t*>(norm_out), sum_rounded != 0, st),
                  fn);
}

int sltx_gemm_route(int32_t M, int32_t N, int32_t K, int32_t group_size, int32_t gated,
                    int32_t x_dtype) {
    const char* fn = "sltx_gemm_route";
    if (M < 1 || N < 1 || K <= 0 || K % 32 != 0)
        return fail(kErrInvalid, "%s: M, N must be >= 1 and K a positive multiple of 32", fn);
    if (group_size <= 0 || K % group_size != 0 || log2_group(group_size) < 0)
        return fail(kErrInvalid, "%s: group_size must be 32, 64 or 128 and divide K", fn);
    if (x_dtype != kF16 && x_dtype != kBF16 && x_dtype != kF32)
        return fail(kErrInvalid, "%s: bad x_dtype", fn);
    // operands at 256-byte aligned stand-in addresses: the plans read only
    // the shape and the pointers' alignment
    const void* al = reinterpret_cast<const void*>(uintptr_t{256});
    GemmParams p{};
    p.a = al;
    p.w0 = static_cast<const uint32_t*>(al);
    p.s0 = p.b0 = static_cast<const uint16_t*>(al);
    p.w1 = gated ? p.w0 : nullptr;
    p.s1 = p.b1 = gated ? p.s0 : nullptr;
    p.M = M;
    p.N = N;
    p.K = K;
    p.groups = K / group_size;
    p.gshift = log2_group(group_size);
    p.y_dtype = kF16;
    p.epilogue = gated ? kEpiSiluMul : kEpiNone;
    p.splits = 1;
    // fp32 x: wide outputs are cast once and take the fp16 routes
    p.a_f32 = x_dtype == kF32 && N <= 2 * 256 ? 1 : 0;
    NarrowPlan np;
    SkinnyPlan sp;
    WidePlan wp;
    return gemm_route(p, x_dtype == kBF16, &np, &sp, &wp);
}

}  // extern "C"
