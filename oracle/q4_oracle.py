"""NumPy restatement of swift-ltx's MLX 4-bit dequant matmul, plus a ctypes
loader for the C restatement in q4_oracle.c.

TEST INFRASTRUCTURE ONLY: this module is the checker the HIP kernels are
compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import it; the shipped library never does.

Reference citations are relative to the swift-ltx tree (Sources/SwiftLLM/).

Layout (ModelWeights.swift:7-11, LinearWeight.quantized):
    weight  uint32 [N, K/8]   nibble k of row n = bits 4*(k%8).. of word k/8
    scales  fp16   [N, K/g]
    biases  fp16   [N, K/g]
    w[n,k] = scales[n,k/g] * q[n,k] + biases[n,k/g]     (Kernels.swift:392-395)
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# SLTX_ORACLE_LIB_DIR selects prebuilt libraries (the sanitized build of
# build_c_sanitized, for the CPU tests); they are never rebuilt there.
PREBUILT_DIR = os.environ.get("SLTX_ORACLE_LIB_DIR")
LIB_DIR = PREBUILT_DIR or os.path.join(HERE, "_build")
LIB_PATH = os.path.join(LIB_DIR, "libq4oracle.so")
CPU_LIB_PATH = os.path.join(LIB_DIR, "libq4cpu.so")


# --------------------------------------------------------------- packing ---

def pack_q4(q: np.ndarray) -> np.ndarray:
    """[N, K] codes 0..15 -> [N, K/8] uint32, low nibble first
    (inverse of the unpack at Kernels.swift:385-390)."""
    q = np.asarray(q, dtype=np.uint32)
    n, k = q.shape
    assert k % 8 == 0
    q = q.reshape(n, k // 8, 8)
    shifts = (np.arange(8, dtype=np.uint32) * 4)[None, None, :]
    return np.bitwise_or.reduce(q << shifts, axis=2).astype(np.uint32)


def unpack_q4(w: np.ndarray) -> np.ndarray:
    """[N, K/8] uint32 -> [N, K] uint8 codes; nibble k is
    (word >> (4*(k%8))) & 0xF (Kernels.swift:390, :428)."""
    w = np.asarray(w, dtype=np.uint32)
    n, pk = w.shape
    shifts = (np.arange(8, dtype=np.uint32) * 4)[None, None, :]
    return ((w[:, :, None] >> shifts) & 0xF).astype(np.uint8).reshape(n, pk * 8)


def dequant_f64(w: np.ndarray, scales: np.ndarray, biases: np.ndarray, group: int) -> np.ndarray:
    """w = s*q + b per group, in fp64 (Kernels.swift:392-395, :430-433)."""
    q = unpack_q4(w).astype(np.float64)
    n, k = q.shape
    s = np.repeat(scales.astype(np.float64), group, axis=1)
    b = np.repeat(biases.astype(np.float64), group, axis=1)
    assert s.shape == (n, k)
    return s * q + b


def matmul_q4_f64(x: np.ndarray, w: np.ndarray, scales: np.ndarray, biases: np.ndarray,
                  group: int) -> np.ndarray:
    """fp64 closed form y = x . dequant(W)^T, x [M,K] (fp16 or fp32-held bf16
    values) -> [M,N] fp64.  matmul_q4 (Kernels.swift:444-620) for M==1 and the
    quantized GEMM (Ops.swift:312-381) for M>1 compute this product."""
    return np.asarray(x, dtype=np.float64) @ dequant_f64(w, scales, biases, group).T


def cast_f32_to_f16_ref(x: np.ndarray) -> np.ndarray:
    """cast_f32_to_f16 (Kernels.swift:816-822): half(clamp(x, -65504, 65504)),
    the fp32 -> fp16 cast DiTLinear.applyF32in runs before matmulQ4FastF32
    (DiTModel.swift:104-110).  Metal's clamp is fmin(fmax(x, lo), hi), and
    fmax / fmin return the other operand when one is NaN, so NaN becomes
    -65504; the cast rounds to nearest even."""
    x = np.asarray(x, dtype=np.float32)
    return np.fmin(np.fmax(x, np.float32(-65504.0)), np.float32(65504.0)).astype(np.float16)


def silu_mul_f64(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """silu(a)*b in fp64 (Kernels.swift:90-98 computes it in fp32)."""
    a = np.asarray(a, dtype=np.float64)
    with np.errstate(over="ignore"):
        return a / (1.0 + np.exp(-a)) * np.asarray(b, dtype=np.float64)


def gelu_tanh_f64(v: np.ndarray) -> np.ndarray:
    """GELU tanh approximation with the inner clamp at +-10
    (gelu_approximate_f32, Kernels.swift:1774-1783), fp64."""
    v = np.asarray(v, dtype=np.float64)
    inner = np.clip(0.7978845608 * (v + 0.044715 * v ** 3), -10.0, 10.0)
    return 0.5 * v * (1.0 + np.tanh(inner))


# ------------------------------------------------- norms and residual add ---

def rms_norm_ref(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """rms_norm (Kernels.swift:40-86) over the last axis: fp16 x, fp32 weight.
    sum of squares of float(x) (here in fp64; the kernel's fp32 sum differs
    below fp32 rounding), rms = rsqrt(mean + eps) rounded to fp32, then
    out = half(float(x) * rms * weight) evaluated in fp32 left to right."""
    xf = np.asarray(x, dtype=np.float16).astype(np.float32)
    ss = np.sum(xf.astype(np.float64) ** 2, axis=-1, keepdims=True)
    rms = (1.0 / np.sqrt(ss / xf.shape[-1] + eps)).astype(np.float32)
    return ((xf * rms) * np.asarray(weight, dtype=np.float32)).astype(np.float16)


def residual_rms_norm_ref(a: np.ndarray, b: np.ndarray, weight: np.ndarray,
                          eps: float) -> tuple[np.ndarray, np.ndarray]:
    """residual_rms_norm (Kernels.swift:238-290): v = float(a) + float(b);
    residual = half(v); the sum of squares uses the unrounded v; the norm is
    applied to the rounded residual.  Returns (residual, normed), fp16."""
    v = (np.asarray(a, dtype=np.float16).astype(np.float32)
         + np.asarray(b, dtype=np.float16).astype(np.float32))
    residual = v.astype(np.float16)
    ss = np.sum(v.astype(np.float64) ** 2, axis=-1, keepdims=True)
    rms = (1.0 / np.sqrt(ss / v.shape[-1] + eps)).astype(np.float32)
    normed = ((residual.astype(np.float32) * rms) * np.asarray(weight, dtype=np.float32))
    return residual, normed.astype(np.float16)


def residual_add_ref(residual: np.ndarray, y: np.ndarray) -> np.ndarray:
    """linear then elemAdd (LlamaModel.swift:330-331; add kernel,
    Kernels.swift:121-128): the projection is fp16 first, the sum is rounded
    to fp16 again."""
    yh = np.asarray(y, dtype=np.float64).astype(np.float16)
    return (np.asarray(residual, dtype=np.float16).astype(np.float32)
            + yh.astype(np.float32)).astype(np.float16)


def embedding_q4_ref(w: np.ndarray, scales: np.ndarray, biases: np.ndarray, ids, group: int
                     ) -> np.ndarray:
    """embedding_q4_batch (Kernels.swift:368-396): rows ids of the 4-bit table,
    out = half(float(q) * s + b) with the product and sum in fp32 (q*s is exact
    in fp32, so a fused multiply-add rounds the same).  Ids outside
    [0, vocab) give zero rows (where the reference reads out of bounds)."""
    ids = np.asarray(ids, dtype=np.int64)
    vocab, K = w.shape[0], w.shape[1] * 8
    out = np.zeros((len(ids), K), dtype=np.float16)
    ok = (ids >= 0) & (ids < vocab)
    if ok.any():
        r = ids[ok]
        q = unpack_q4(w[r]).astype(np.float32)
        s = np.repeat(np.asarray(scales[r], np.float16).astype(np.float32), group, axis=1)
        b = np.repeat(np.asarray(biases[r], np.float16).astype(np.float32), group, axis=1)
        out[ok] = (q * s + b).astype(np.float16)
    return out


# -------------------------------------------------------- token selection --

def argmax_ref(logits) -> int:
    """argmax (Ops.swift:757-781): scan from element 0 keeping the first
    strictly greater value, so NaNs never win and a NaN at index 0 gives 0."""
    v = np.asarray(logits).astype(np.float32)
    if np.isnan(v[0]):
        return 0
    return int(np.argmax(np.where(np.isnan(v), -np.inf, v)))


def sample_ref(logits, temperature: float, top_p: float, penalty: float, seen, u: float,
               detail: bool = False, gpu_sums: bool = False):
    """sample + sampleFromLogits (Ops.swift:785-806, 2060-2098) in fp32:
    penalty on each distinct seen id < n (divide positive, multiply the rest),
    divide by temperature, softmax, order by probability descending, shortest
    prefix with running sum >= top_p (else all), r = u * that sum, then
    r -= p_i until r <= 0.  The reference's sort is unstable; ties are ordered
    here by ascending id.

    gpu_sums=False: the reference's sequential fp32 sums (numpy's
    add.accumulate is sequential) for the softmax denominator and the running
    sums.
    gpu_sums=True: the sums the GPU kernels form instead, for a tighter check
    of them: an online softmax over G = min(256, ceil(n/1024)) blocks of 256
    threads, thread j holding tokens 4q..4q+3 for q = j, j + 256G, ...: block
    b's max m_b, its s_b = sum of exp(l - m_b) (each thread in token order,
    then a halving tree over the block), and the denominator: the terms
    s_b * exp(m_b - max), padded to 256 and summed as four 64-term halving
    trees combined as (w0 + w1) + (w2 + w3); p = exp(l - max) / that;
    and exact running sums of the integer masses
    floor(p * 2^52): cutoff = first token whose inclusive mass reaches
    ceil(top_p * 2^52), chosen = first whose inclusive mass reaches
    ceil(u * mass at the cutoff).

    Returns the token, or (token, info) with the order, sorted probabilities,
    cutoff and running sum there when detail is set."""
    f32 = np.float32
    lg = np.asarray(logits).astype(f32).copy()
    n = lg.size
    pen = f32(penalty)
    for t in sorted(set(int(t) for t in (seen if seen is not None else []))):
        if 0 <= t < n:
            lg[t] = lg[t] / pen if lg[t] > 0 else lg[t] * pen
    lg = lg / f32(temperature)
    mx = f32(-3.4028234663852886e38)   # -greatestFiniteMagnitude
    live = lg[~np.isnan(lg)]
    if live.size:
        mx = max(mx, f32(live.max()))
    with np.errstate(over="ignore", under="ignore", invalid="ignore"):
        e = np.exp(lg - mx).astype(f32)
        if gpu_sums:
            G = min(256, -(-n // 1024))
            T = 256 * G
            R = -(-n // (4 * T))
            L3 = np.full(R * 4 * T, -np.inf, f32)
            L3[:n] = lg
            L3 = L3.reshape(R, T, 4)
            mb = L3.reshape(R, G, 256, 4).max(axis=(0, 2, 3)).astype(f32)   # block maxima
            E = np.exp(L3 - np.repeat(mb, 256)[None, :, None]).astype(f32)
            seq = E.transpose(0, 2, 1).reshape(R * 4, T)
            blk = np.add.accumulate(seq, axis=0, dtype=f32)[-1].reshape(G, 256).copy()
            h = 128
            while h:
                blk[:, :h] = blk[:, :h] + blk[:, h:2 * h]
                h //= 2
            M = f32(mb.max())
            terms = np.zeros(256, f32)
            terms[:G] = (blk[:, 0] * np.exp(mb - M).astype(f32)).astype(f32)
            w = terms.reshape(4, 64).copy()
            h = 32
            while h:
                w[:, :h] = w[:, :h] + w[:, h:2 * h]
                h //= 2
            s = f32(f32(w[0, 0] + w[1, 0]) + f32(w[2, 0] + w[3, 0]))
            e = np.exp(lg - M).astype(f32)
        else:
            s = np.add.accumulate(e, dtype=f32)[-1]
        p = (e / s).astype(f32)
    order = np.lexsort((np.arange(n), -p))
    ps = p[order]
    if gpu_sums:
        mass = np.floor(ps.astype(np.float64) * 2.0 ** 52).astype(np.uint64)
        cum = np.cumsum(mass, dtype=np.uint64)
        t1 = np.uint64(math.ceil(min(float(f32(top_p)), 4.0) * 2.0 ** 52))
        k1 = int(np.searchsorted(cum, t1, "left"))
        cutoff = k1 + 1 if k1 < n else n
        cum_prob = int(cum[cutoff - 1])
        t2 = np.uint64(math.ceil(float(f32(u)) * float(cum_prob)))
        tok = int(order[int(np.searchsorted(cum, t2, "left"))])
        cum_out, r = cum_prob * 2.0 ** -52, float(t2) * 2.0 ** -52
    else:
        cum = np.add.accumulate(ps, dtype=f32)
        hit = np.nonzero(cum >= f32(top_p))[0]
        cutoff = int(hit[0]) + 1 if hit.size else n
        cum_prob = cum[cutoff - 1]
        r = f32(u) * cum_prob
        walk = np.subtract.accumulate(np.concatenate([[r], ps[:cutoff]]).astype(f32),
                                      dtype=f32)[1:]
        le = np.nonzero(walk <= 0)[0]
        tok = int(order[le[0]]) if le.size else int(order[0])
        cum_out, r = float(cum_prob), float(r)
    if detail:
        info = {"order": order, "probs": ps, "cutoff": cutoff, "cum": cum_out, "r": r}
        if not gpu_sums:   # the rounding the sequential fp32 sums carry here
            c64 = np.cumsum(ps.astype(np.float64))
            info["cum_err"] = np.abs(cum.astype(np.float64) - c64)
            s64 = np.sum(e.astype(np.float64))
            info["sum_rel_err"] = abs(float(s) - s64) / s64 if s64 > 0 else 0.0
        return tok, info
    return tok


# ----------------------------------------------------- bf16 (numpy has none) --

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    r[nan] = 0x7FC0
    return r


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# -------------------------------------------------------------- inputs ---

def make_inputs(M: int, N: int, K: int, group: int = 64, seed: int = 0, x_dtype: str = "f16",
                n_weights: int = 1):
    """Synthetic inputs with the benchmark's input distributions:
    x ~ N(0,1) (fp16, or bf16 bits when x_dtype == 'bf16'); codes uniform 0..15;
    scales ~ |N(0, 0.02)| fp16; biases = -8*scales (exact in fp16).
    Draw order from one default_rng(seed): x, then per weight set (codes, scales).
    Returns (x, [(W, scales, biases), ...])."""
    rng = np.random.default_rng(seed)
    xf = rng.standard_normal((M, K), dtype=np.float32)
    if x_dtype == "bf16":
        x = f32_to_bf16_bits(xf)
    else:
        x = xf.astype(np.float16)
    sets = []
    for _ in range(n_weights):
        q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
        s = np.abs(0.02 * rng.standard_normal((N, K // group), dtype=np.float32)).astype(np.float16)
        b = (-8.0 * s.astype(np.float32)).astype(np.float16)
        sets.append((pack_q4(q), s, b))
    return x, sets


def x_values(x: np.ndarray, x_dtype: str = "f16") -> np.ndarray:
    """fp64 values of an fp16 array or a bf16 bit-pattern array."""
    if x_dtype == "bf16":
        return bf16_bits_to_f32(x).astype(np.float64)
    return np.asarray(x, dtype=np.float64)


# ------------------------------------------------------------- metrics ---

def max_rel_err(y, ref) -> float:
    """The parity gate's metric: max_i |y_i - ref_i| / max_i |ref_i|."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = float(np.max(np.abs(ref))) if ref.size else 0.0
    if ref.size == 0:
        return 0.0
    return float(np.max(np.abs(y - ref))) / max(den, 1e-30)


def elementwise_ok(y, ref, rtol: float, atol_rms: float) -> tuple[bool, float]:
    """|y-ref| <= rtol*|ref| + atol_rms*rms(ref) for every element; returns
    (ok, worst ratio of error to allowance)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if ref.size == 0:
        return True, 0.0
    rms = math.sqrt(float(np.mean(ref * ref))) or 1e-30
    allow = rtol * np.abs(ref) + atol_rms * rms
    ratio = np.abs(y - ref) / allow
    worst = float(np.max(ratio))
    return bool(worst <= 1.0 and np.all(np.isfinite(y))), worst


# ----------------------------------------------------------- C library ---

def build_c(force: bool = False) -> str:
    """Compile q4_oracle.c into _build/libq4oracle.so with gcc."""
    if PREBUILT_DIR:
        return LIB_PATH
    src = os.path.join(HERE, "q4_oracle.c")
    src2 = os.path.join(HERE, "q4_cpu_baseline.c")
    if (not force and all(os.path.exists(p) for p in (LIB_PATH, CPU_LIB_PATH))
            and min(os.path.getmtime(LIB_PATH), os.path.getmtime(CPU_LIB_PATH))
            >= max(os.path.getmtime(src), os.path.getmtime(src2))):
        return LIB_PATH
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB_PATH + ".tmp%d" % os.getpid()
    subprocess.run(["gcc", "-O2", "-fPIC", "-shared", "-std=c11", "-ffp-contract=off",
                    "-o", tmp, src, "-lm", "-lpthread"], check=True)
    os.replace(tmp, LIB_PATH)
    # The CPU baselines (q4_cpu_baseline.c): vectorized for AVX2 + FMA (every
    # x86-64-v3 host, the GPU boxes' EPYCs included), fp contraction allowed.
    tmp2 = CPU_LIB_PATH + ".tmp%d" % os.getpid()
    subprocess.run(["gcc", "-O3", "-mavx2", "-mfma", "-mf16c", "-fPIC", "-shared", "-std=gnu11", "-o", tmp2,
                    src2, "-lpthread"], check=True)
    os.replace(tmp2, CPU_LIB_PATH)
    return LIB_PATH


def build_c_sanitized(out_dir: str) -> None:
    """q4_oracle.c and q4_cpu_baseline.c built with clang's AddressSanitizer
    and UndefinedBehaviorSanitizer into out_dir (same file names and flags as
    build_c, plus the sanitizers; the process that loads them must preload
    clang's ASan runtime)."""
    clang = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin", "clang")
    san = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
           "-fno-omit-frame-pointer", "-g", "-shared-libsan"]
    os.makedirs(out_dir, exist_ok=True)
    subprocess.run([clang, "-O2", "-fPIC", "-shared", "-std=c11", "-ffp-contract=off", *san,
                    "-o", os.path.join(out_dir, "libq4oracle.so"),
                    os.path.join(HERE, "q4_oracle.c"), "-lm", "-lpthread"], check=True)
    subprocess.run([clang, "-O3", "-mavx2", "-mfma", "-mf16c", "-fPIC", "-shared", "-std=gnu11",
                    *san, "-o", os.path.join(out_dir, "libq4cpu.so"),
                    os.path.join(HERE, "q4_cpu_baseline.c"), "-lpthread"], check=True)


_cpu_lib = None


def cpu_lib():
    """ctypes handle of the CPU baselines (q4_cpu_baseline.c)."""
    global _cpu_lib
    if _cpu_lib is None:
        if not os.path.exists(CPU_LIB_PATH):
            build_c(force=True)
        L = ctypes.CDLL(CPU_LIB_PATH)
        P, I64 = ctypes.c_void_p, ctypes.c_int64
        L.cpu_q4_scalar.argtypes = [P, P, P, P, P, I64, I64, I64, I64]
        L.cpu_q4_scalar.restype = None
        L.cpu_q4_simd.argtypes = [P, P, P, P, P, I64, I64, I64, I64, ctypes.c_int]
        L.cpu_q4_simd.restype = ctypes.c_int
        _cpu_lib = L
    return _cpu_lib


def _q4_args(x, w, s, b):
    x = np.ascontiguousarray(x, dtype=np.float16).view(np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.float16).view(np.uint16)
    b = np.ascontiguousarray(b, dtype=np.float16).view(np.uint16)
    return x, w, s, b


class CpuQ4:
    """Inputs of one dequant matmul converted once for the CPU baselines, so
    that timing a run times only the C call."""

    def __init__(self, x, w, s, b, group):
        self.x, self.w, self.s, self.b = _q4_args(x, w, s, b)
        self.M, self.K = self.x.shape
        self.N = self.w.shape[0]
        self.group = group
        self.y = np.empty((self.M, self.N), dtype=np.uint16)

    def scalar(self, rows=None) -> np.ndarray:
        """Single-thread scalar baseline (matmulCPU's loop shape,
        LlamaModel.swift:478-493, with the 4-bit dequant inline) over the first
        `rows` rows of x (all by default)."""
        m = self.M if rows is None else rows
        cpu_lib().cpu_q4_scalar(_p(self.x), _p(self.w), _p(self.s), _p(self.b), _p(self.y), m,
                                self.N, self.K, self.group)
        return self.y[:m].view(np.float16)

    def simd(self, threads=1) -> np.ndarray:
        """8-wide fp32 (SIMD8<Float>) baseline over `threads` pthreads."""
        rc = cpu_lib().cpu_q4_simd(_p(self.x), _p(self.w), _p(self.s), _p(self.b), _p(self.y),
                                   self.M, self.N, self.K, self.group, threads)
        if rc < 0:
            raise RuntimeError("cpu_q4_simd failed")
        return self.y.view(np.float16)


def cpu_q4_scalar(x, w, s, b, group) -> np.ndarray:
    """CpuQ4(...).scalar() on a copy of the output."""
    return CpuQ4(x, w, s, b, group).scalar().copy()


def cpu_q4_simd(x, w, s, b, group, threads=1) -> np.ndarray:
    """CpuQ4(...).simd(threads) on a copy of the output."""
    return CpuQ4(x, w, s, b, group).simd(threads).copy()


_lib = None


def lib():
    """ctypes handle of the C oracle (built on first use if missing)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build_c()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_f16_to_f32.restype = ctypes.c_float
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_unpack_q4.argtypes = [P, P, I64, I64]
        L.oracle_matmul_q4_f64.argtypes = [P, ctypes.c_int, P, P, P, P, I64, I64, I64, I64]
        L.oracle_matmul_q4_emu.argtypes = [P, P, P, P, P, I64, I64, I64, I64]
        L.oracle_silu_mul.argtypes = [P, P, P, I64]
        L.oracle_gelu_tanh_f32.argtypes = [P, P, I64]
        L.oracle_cpu_matmul_q4.argtypes = [P, P, P, P, P, I64, I64, I64, I64, ctypes.c_int]
        L.oracle_cpu_matmul_q4.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def c_f16_to_f32(h: np.ndarray) -> np.ndarray:
    L = lib()
    return np.array([L.oracle_f16_to_f32(int(v)) for v in np.asarray(h, np.uint16).ravel()],
                    dtype=np.float32)


def c_unpack_q4(w: np.ndarray, K: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint32)
    q = np.empty((w.shape[0], K), dtype=np.uint8)
    lib().oracle_unpack_q4(_p(w), _p(q), w.shape[0], K)
    return q


def c_matmul_q4_f64(x, w, s, b, group, x_dtype="f16") -> np.ndarray:
    x = np.ascontiguousarray(x).view(np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.float16).view(np.uint16)
    b = np.ascontiguousarray(b, dtype=np.float16).view(np.uint16)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), dtype=np.float64)
    lib().oracle_matmul_q4_f64(_p(x), 1 if x_dtype == "bf16" else 0, _p(w), _p(s), _p(b),
                               _p(y), M, N, K, group)
    return y


def c_matmul_q4_emu(x, w, s, b, group) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float16).view(np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.float16).view(np.uint16)
    b = np.ascontiguousarray(b, dtype=np.float16).view(np.uint16)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), dtype=np.uint16)
    lib().oracle_matmul_q4_emu(_p(x), _p(w), _p(s), _p(b), _p(y), M, N, K, group)
    return y.view(np.float16)


def c_silu_mul(a, b) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float16).view(np.uint16)
    b = np.ascontiguousarray(b, dtype=np.float16).view(np.uint16)
    out = np.empty_like(a)
    lib().oracle_silu_mul(_p(a), _p(b), _p(out), a.size)
    return out.view(np.float16)


def c_gelu_tanh_f32(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().oracle_gelu_tanh_f32(_p(x), _p(out), x.size)
    return out


def c_cpu_matmul_q4(x, w, s, b, group, threads=1) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float16).view(np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s = np.ascontiguousarray(s, dtype=np.float16).view(np.uint16)
    b = np.ascontiguousarray(b, dtype=np.float16).view(np.uint16)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), dtype=np.uint16)
    rc = lib().oracle_cpu_matmul_q4(_p(x), _p(w), _p(s), _p(b), _p(y), M, N, K, group, threads)
    if rc < 0:
        raise RuntimeError("oracle_cpu_matmul_q4 failed")
    return y.view(np.float16)
