"""swift-ltx MI355X 4-bit dequant matmul path: Python mirror of the reference's
Ops entry points over the C ABI in include/swiftltx_q4.h.

The shipped compute path is libswiftltx_q4.so (hand-written HIP for gfx950);
this module only marshals torch device tensors into it with ctypes.  There is
no fallback: if the library is missing, every entry point raises.

Reference interface mirrored (Sources/SwiftLLM/ of swift-ltx):
    matmulQ4        Ops.swift:285-305      -> matmul_q4
    matmulQ4Fast    Ops.swift:312-345      -> matmul_q4_fast
    matmulQ4FastF32 Ops.swift:348-381      -> matmul_q4_fast_f32
    siluMul         Ops.swift:44-56        -> silu_mul
    linear          Ops.swift:741-752      -> linear
    LinearWeight    ModelWeights.swift:7-11 -> Q4Weight
The reference returns a new Tensor from its buffer pool and crashes on error;
here each call returns a new torch tensor (or writes `out=`) and raises
SltxError carrying the library's status code and message.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
# SLTX_LIB_PATH selects another build of the same library (the sanitized
# host-only build of build_sanitized.py, for the CPU tests).
LIB_PATH = os.environ.get("SLTX_LIB_PATH") or os.path.join(PKG_DIR, "lib", "libswiftltx_q4.so")

SLTX_OK = 0
SLTX_ERR_INVALID = -1
SLTX_ERR_UNSUPPORTED = -2
SLTX_ERR_HIP = -3

SLTX_F16 = 0
SLTX_BF16 = 1
SLTX_F32 = 2

SLTX_EPI_NONE = 0
SLTX_EPI_GELU_TANH = 2

# Every symbol include/swiftltx_q4.h declares.
EXPORTED = (
    "sltx_abi_version",
    "sltx_init",
    "sltx_last_error",
    "sltx_release_workspace",
    "sltx_matmul_q4",
    "sltx_matmul_q4_fast",
    "sltx_matmul_q4_fast_f32",
    "sltx_silu_mul",
    "sltx_linear",
    "sltx_matmul_q4_silu_mul",
    "sltx_matmul_q4_ex",
    "sltx_matmul_q4_geglu",
    "sltx_embedding_q4",
    "sltx_rms_norm",
    "sltx_residual_rms_norm",
    "sltx_rmsnorm_matmul_q4",
    "sltx_residual_rmsnorm_matmul_q4_silu_mul",
    "sltx_matmul_q4_residual",
    "sltx_matmul_q4_residual_rms_norm",
    "sltx_gemm_route",
    "sltx_argmax",
    "sltx_sample_top_p",
    "sltx_sample_top_p_noalloc",
    "sltx_sample_top_p_state",
    "sltx_st_open",
    "sltx_st_close",
    "sltx_st_num_tensors",
    "sltx_st_name",
    "sltx_st_info_of",
    "sltx_st_read_host",
    "sltx_st_read_device",
    "sltx_st_read_device_f32",
)


class SltxError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class CQ4Weight(ctypes.Structure):
    """sltx_q4_weight."""
    _fields_ = [
        ("weight", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("biases", ctypes.c_void_p),
        ("K", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
    ]


class CSampleState(ctypes.Structure):
    """sltx_sample_state."""
    _fields_ = [
        ("history", ctypes.c_void_p),
        ("history_len", ctypes.c_void_p),
        ("history_capacity", ctypes.c_int32),
        ("draws", ctypes.c_void_p),
        ("next_draw", ctypes.c_void_p),
        ("draw_count", ctypes.c_int32),
    ]


_lib = None


class CStInfo(ctypes.Structure):
    """sltx_st_info: TensorInfo (SafeTensors.swift:7-13)."""
    _fields_ = [("dtype", ctypes.c_int32), ("ndim", ctypes.c_int32),
                ("shape", ctypes.c_int64 * 8), ("offset", ctypes.c_uint64),
                ("nbytes", ctypes.c_uint64)]


def lib():
    """The loaded C library.  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} not found: build it with `python swift-ltx_amd/build.py` "
                "(there is no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        P, I32, I64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
        L.sltx_abi_version.restype = ctypes.c_int
        L.sltx_init.restype = ctypes.c_int
        L.sltx_last_error.restype = ctypes.c_char_p
        L.sltx_release_workspace.argtypes = [P]
        L.sltx_release_workspace.restype = ctypes.c_int
        mm = [P, P, P, P, P, I32, I32, I32, I32, P]
        for n in ("sltx_matmul_q4", "sltx_matmul_q4_fast", "sltx_matmul_q4_fast_f32"):
            getattr(L, n).argtypes = mm
            getattr(L, n).restype = ctypes.c_int
        L.sltx_silu_mul.argtypes = [P, P, P, I64, P]
        L.sltx_silu_mul.restype = ctypes.c_int
        W = ctypes.POINTER(CQ4Weight)
        L.sltx_linear.argtypes = [P, W, P, I32, I32, I32, I32, P]
        L.sltx_linear.restype = ctypes.c_int
        L.sltx_matmul_q4_silu_mul.argtypes = [P, W, W, P, I32, I32, I32, P]
        L.sltx_matmul_q4_silu_mul.restype = ctypes.c_int
        L.sltx_matmul_q4_ex.argtypes = [P, I32, W, P, I32, P, I32, I32, I32, P]
        L.sltx_matmul_q4_ex.restype = ctypes.c_int
        F = ctypes.c_float
        L.sltx_matmul_q4_geglu.argtypes = [P, W, W, P, I32, I32, I32, P]
        L.sltx_matmul_q4_geglu.restype = ctypes.c_int
        L.sltx_embedding_q4.argtypes = [W, I32, P, I32, P, P]
        L.sltx_embedding_q4.restype = ctypes.c_int
        L.sltx_rms_norm.argtypes = [P, P, F, P, I32, I32, P]
        L.sltx_residual_rms_norm.argtypes = [P, P, P, F, P, P, I32, I32, P]
        L.sltx_rmsnorm_matmul_q4.argtypes = [P, P, F, W, P, I32, P]
        L.sltx_residual_rmsnorm_matmul_q4_silu_mul.argtypes = [P, P, P, F, P, W, W, P, I32, P]
        L.sltx_matmul_q4_residual.argtypes = [P, W, P, P, I32, I32, P]
        L.sltx_matmul_q4_residual_rms_norm.argtypes = [P, W, P, P, F, I32, I32, I32, P, P, P]
        L.sltx_gemm_route.argtypes = [I32, I32, I32, I32, I32, I32]
        L.sltx_gemm_route.restype = ctypes.c_int
        L.sltx_argmax.argtypes = [P, I32, I32, P, P]
        L.sltx_sample_top_p.argtypes = [P, I32, I32, F, F, F, P, I32, F, P, P]
        L.sltx_sample_top_p_noalloc.argtypes = [P, I32, I32, F, F, F, P, I32, F, P, P]
        L.sltx_sample_top_p_state.argtypes = [P, I32, I32, F, F, F,
                                              ctypes.POINTER(CSampleState), P, P]
        for n in ("sltx_rms_norm", "sltx_residual_rms_norm", "sltx_rmsnorm_matmul_q4",
                  "sltx_residual_rmsnorm_matmul_q4_silu_mul", "sltx_matmul_q4_residual",
                  "sltx_matmul_q4_residual_rms_norm",
                  "sltx_argmax", "sltx_sample_top_p", "sltx_sample_top_p_noalloc",
                  "sltx_sample_top_p_state"):
            getattr(L, n).restype = ctypes.c_int
        VP = ctypes.c_void_p
        L.sltx_st_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(VP)]
        L.sltx_st_open.restype = ctypes.c_int
        L.sltx_st_close.argtypes = [VP]
        L.sltx_st_close.restype = None
        L.sltx_st_num_tensors.argtypes = [VP]
        L.sltx_st_num_tensors.restype = ctypes.c_int
        L.sltx_st_name.argtypes = [VP, I32]
        L.sltx_st_name.restype = ctypes.c_char_p
        L.sltx_st_info_of.argtypes = [VP, ctypes.c_char_p, ctypes.POINTER(CStInfo)]
        L.sltx_st_info_of.restype = ctypes.c_int
        U64 = ctypes.c_uint64
        L.sltx_st_read_host.argtypes = [VP, ctypes.c_char_p, VP, U64]
        L.sltx_st_read_host.restype = ctypes.c_int
        L.sltx_st_read_device.argtypes = [VP, ctypes.c_char_p, VP, U64, VP]
        L.sltx_st_read_device.restype = ctypes.c_int
        L.sltx_st_read_device_f32.argtypes = [VP, ctypes.c_char_p, VP, U64, VP]
        L.sltx_st_read_device_f32.restype = ctypes.c_int
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != SLTX_OK:
        msg = lib().sltx_last_error().decode(errors="replace")
        raise SltxError(rc, msg)


def last_error() -> str:
    return lib().sltx_last_error().decode(errors="replace")


def release_workspace(stream=None):
    """Frees the library's workspace for `stream` (default: the current
    stream) after its queued work; see sltx_release_workspace."""
    check(lib().sltx_release_workspace(_stream(stream)))


# ------------------------------------------------------------ torch glue ---

def _torch():
    import torch
    return torch


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(stream) -> int | None:
    torch = _torch()
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _dtype_code(dt) -> int:
    torch = _torch()
    if dt == torch.float16:
        return SLTX_F16
    if dt == torch.bfloat16:
        return SLTX_BF16
    if dt == torch.float32:
        return SLTX_F32
    raise ValueError(f"unsupported dtype {dt}")


@dataclass
class Q4Weight:
    """LinearWeight.quantized (ModelWeights.swift:7-11): weight uint32/int32
    [N, K/8], scales and biases fp16 [N, K/group_size]."""
    weight: object
    scales: object
    biases: object
    K: int
    group_size: int = 64

    @property
    def N(self) -> int:
        return int(self.weight.shape[0])

    def c(self) -> CQ4Weight:
        return CQ4Weight(self.weight.data_ptr(), self.scales.data_ptr(), self.biases.data_ptr(),
                         int(self.K), int(self.group_size))


def _new(shape, dtype, like):
    return _torch().empty(shape, dtype=dtype, device=like.device)


def _need(t, what, count, dtypes=None):
    """Checks a tensor handed to the library as a raw pointer: a contiguous
    device tensor of an accepted dtype holding at least `count` elements (the
    library reads or writes exactly that many from its start).  A strided
    view or a short buffer would otherwise be read or written out of bounds
    on the device."""
    if t is None:
        raise ValueError(f"{what} is None")
    if not getattr(t, "is_cuda", False):
        raise ValueError(f"{what} must be a device tensor")
    if dtypes is not None and t.dtype not in dtypes:
        raise ValueError(f"{what} has dtype {t.dtype}, expected one of {dtypes}")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous (got strides {tuple(t.stride())})")
    if t.numel() < count:
        raise ValueError(f"{what} holds {t.numel()} elements, {count} needed")
    return t


def _shape_ok(K, g):
    """The library's shape rules; tensors are checked only for shapes it
    accepts (it reports the others with its own status code)."""
    return K > 0 and K % 32 == 0 and g in (32, 64, 128) and K % g == 0


def _f16():
    return (_torch().float16,)


def _w_dtypes():
    torch = _torch()
    return tuple(d for d in (torch.int32, getattr(torch, "uint32", None)) if d is not None)


def _need_w(w, N, K=None, what="weight"):
    """Q4Weight operands for N rows of K (default w.K) columns."""
    K = w.K if K is None else K
    g = int(w.group_size)
    if g <= 0 or K % g != 0:
        return   # the library reports the bad shape
    _need(w.weight, what + ".weight", N * K // 8, _w_dtypes())
    _need(w.scales, what + ".scales", N * (K // g), _f16())
    _need(w.biases, what + ".biases", N * (K // g), _f16())


def _need_raw(weight, scales, biases, N, K, g):
    if g > 0 and K % g == 0:
        _need(weight, "weight", N * K // 8, _w_dtypes())
        _need(scales, "scales", N * (K // g), _f16())
        _need(biases, "biases", N * (K // g), _f16())


def matmul_q4(x, weight, scales, biases, M, K, N, group_size, out=None, stream=None):
    """matmulQ4 (Ops.swift:285-305): [M,N] fp16 = x[M,K] fp16 . dequant(W)^T."""
    out = _new((M, N), _torch().float16, x) if out is None else out
    if M > 0 and N > 0 and _shape_ok(K, group_size):
        _need(x, "x", M * K, _f16())
        _need_raw(weight, scales, biases, N, K, group_size)
        _need(out, "out", M * N, (_torch().float16,))
    check(lib().sltx_matmul_q4(_ptr(x), _ptr(weight), _ptr(scales), _ptr(biases), _ptr(out),
                               M, K, N, group_size, _stream(stream)))
    return out


def matmul_q4_fast(x, weight, scales, biases, M, K, N, group_size, out=None, stream=None):
    """matmulQ4Fast (Ops.swift:312-345): MFMA GEMM, fp16 out."""
    out = _new((M, N), _torch().float16, x) if out is None else out
    if M > 0 and N > 0 and _shape_ok(K, group_size):
        _need(x, "x", M * K, _f16())
        _need_raw(weight, scales, biases, N, K, group_size)
        _need(out, "out", M * N, (_torch().float16,))
    check(lib().sltx_matmul_q4_fast(_ptr(x), _ptr(weight), _ptr(scales), _ptr(biases), _ptr(out),
                                    M, K, N, group_size, _stream(stream)))
    return out


def matmul_q4_fast_f32(x, weight, scales, biases, M, K, N, group_size, out=None, stream=None):
    """matmulQ4FastF32 (Ops.swift:348-381): MFMA GEMM, fp32 out."""
    out = _new((M, N), _torch().float32, x) if out is None else out
    if M > 0 and N > 0 and _shape_ok(K, group_size):
        _need(x, "x", M * K, _f16())
        _need_raw(weight, scales, biases, N, K, group_size)
        _need(out, "out", M * N, (_torch().float32,))
    check(lib().sltx_matmul_q4_fast_f32(_ptr(x), _ptr(weight), _ptr(scales), _ptr(biases),
                                        _ptr(out), M, K, N, group_size, _stream(stream)))
    return out


def silu_mul(a, b, out=None, stream=None):
    """siluMul (Ops.swift:44-56): half(silu(a) * b), fp16."""
    out = _torch().empty_like(a) if out is None else out
    n = a.numel()
    if n > 0:
        _need(a, "a", n, _f16())
        _need(b, "b", n, _f16())
        _need(out, "out", n, _f16())
    check(lib().sltx_silu_mul(_ptr(a), _ptr(b), _ptr(out), n, _stream(stream)))
    return out


def linear(x, w: Q4Weight, M, K, N, fast=False, out=None, stream=None):
    """linear (Ops.swift:741-752), quantized case: fast && M>1 -> GEMM, else matmul_q4."""
    out = _new((M, N), _torch().float16, x) if out is None else out
    if M > 0 and N > 0 and _shape_ok(K, w.group_size) and w.K == K:
        _need(x, "x", M * K, _f16())
        _need_w(w, N)
        _need(out, "out", M * N, _f16())
    cw = w.c()
    check(lib().sltx_linear(_ptr(x), ctypes.byref(cw), _ptr(out), M, K, N, 1 if fast else 0,
                            _stream(stream)))
    return out


def matmul_q4_silu_mul(x, gate: Q4Weight, up: Q4Weight, M, K, N, out=None, stream=None):
    """Fused silu(x.Wg^T) * (x.Wu^T) -> fp16 [M, N]; replaces linear(gate),
    linear(up), siluMul (LlamaModel.swift:275-277, :327-329)."""
    out = _new((M, N), _torch().float16, x) if out is None else out
    if M > 0 and N > 0 and _shape_ok(K, gate.group_size):
        _need(x, "x", M * K, _f16())
        _need_w(gate, N, K, "gate")
        _need_w(up, N, K, "up")
        _need(out, "out", M * N, _f16())
    g, u = gate.c(), up.c()
    check(lib().sltx_matmul_q4_silu_mul(_ptr(x), ctypes.byref(g), ctypes.byref(u), _ptr(out), M,
                                        K, N, _stream(stream)))
    return out


def matmul_q4_ex(x, w: Q4Weight, M, N, out_dtype=None, bias=None, epilogue=SLTX_EPI_NONE,
                 out=None, stream=None):
    """epi(x . dequant(W)^T + bias) with x fp16/bf16/fp32 and out
    fp16/bf16/fp32 (DiTLinear.applyF32in q4 branch, DiTModel.swift:102-125,
    + GELU-tanh); fp32 x is cast to fp16 with the +-65504 clamp of
    cast_f32_to_f16 (Kernels.swift:816-822) inside the GEMM."""
    torch = _torch()
    if out is None:
        out = _new((M, N), out_dtype or torch.float32, x)
    if M > 0 and N > 0 and _shape_ok(w.K, w.group_size):
        _need(x, "x", M * w.K, (torch.float16, torch.bfloat16, torch.float32))
        _need_w(w, N)
        _need(out, "out", M * N, (torch.float16, torch.bfloat16, torch.float32))
        if bias is not None:
            _need(bias, "bias", N, (torch.float32,))
    cw = w.c()
    check(lib().sltx_matmul_q4_ex(_ptr(x), _dtype_code(x.dtype), ctypes.byref(cw), _ptr(bias),
                                  epilogue, _ptr(out), _dtype_code(out.dtype), M, N,
                                  _stream(stream)))
    return out


def rms_norm(x, weight, eps, rows, dim, out=None, stream=None):
    """rmsNorm (Ops.swift:8-27): fp16 [rows, dim], fp32 weight [dim]."""
    out = _new((rows, dim), _torch().float16, x) if out is None else out
    if rows > 0 and dim > 0:
        _need(x, "x", rows * dim, _f16())
        _need(weight, "weight", dim, (_torch().float32,))
        _need(out, "out", rows * dim, _f16())
    check(lib().sltx_rms_norm(_ptr(x), _ptr(weight), eps, _ptr(out), rows, dim, _stream(stream)))
    return out


def residual_rms_norm(a, b, weight, eps, rows, dim, residual_out=None, norm_out=None,
                      stream=None):
    """residualRmsNorm (Ops.swift:256-279) -> (residual, normed), fp16 [rows, dim]."""
    torch = _torch()
    residual_out = _new((rows, dim), torch.float16, a) if residual_out is None else residual_out
    norm_out = _new((rows, dim), torch.float16, a) if norm_out is None else norm_out
    if rows > 0 and dim > 0:
        for t, n in ((a, "a"), (b, "b"), (residual_out, "residual_out"), (norm_out, "norm_out")):
            _need(t, n, rows * dim, _f16())
        _need(weight, "weight", dim, (torch.float32,))
    check(lib().sltx_residual_rms_norm(_ptr(a), _ptr(b), _ptr(weight), eps, _ptr(residual_out),
                                       _ptr(norm_out), rows, dim, _stream(stream)))
    return residual_out, norm_out


def rmsnorm_matmul_q4(x, norm_weight, eps, w: Q4Weight, N, out=None, stream=None):
    """rms_norm(x) . dequant(W)^T at M = 1 (input_layernorm + q|k|v,
    LlamaModel.swift:288-292) -> fp16 [1, N]."""
    out = _new((1, N), _torch().float16, x) if out is None else out
    if N > 0 and _shape_ok(w.K, w.group_size):
        _need(x, "x", w.K, _f16())
        _need(norm_weight, "norm_weight", w.K, (_torch().float32,))
        _need_w(w, N)
        _need(out, "out", N, _f16())
    cw = w.c()
    check(lib().sltx_rmsnorm_matmul_q4(_ptr(x), _ptr(norm_weight), eps, ctypes.byref(cw),
                                       _ptr(out), N, _stream(stream)))
    return out


def residual_rmsnorm_matmul_q4_silu_mul(a, b, norm_weight, eps, gate: Q4Weight, up: Q4Weight, N,
                                        residual_out=None, out=None, stream=None):
    """residualRmsNorm + gate/up + siluMul at M = 1 (LlamaModel.swift:326-329)
    -> (residual [1, K], activated [1, N])."""
    torch = _torch()
    residual_out = _new((1, gate.K), torch.float16, a) if residual_out is None else residual_out
    out = _new((1, N), torch.float16, a) if out is None else out
    if N > 0 and _shape_ok(gate.K, gate.group_size):
        for t, n in ((a, "a"), (b, "b"), (residual_out, "residual_out")):
            _need(t, n, gate.K, _f16())
        _need(norm_weight, "norm_weight", gate.K, (torch.float32,))
        _need_w(gate, N, what="gate")
        _need_w(up, N, what="up")
        _need(out, "out", N, _f16())
    g, u = gate.c(), up.c()
    check(lib().sltx_residual_rmsnorm_matmul_q4_silu_mul(
        _ptr(a), _ptr(b), _ptr(norm_weight), eps, _ptr(residual_out), ctypes.byref(g),
        ctypes.byref(u), _ptr(out), N, _stream(stream)))
    return residual_out, out


def matmul_q4_residual(x, w: Q4Weight, residual, M, N, out=None, stream=None):
    """half(residual + half(x . dequant(W)^T)): linear + elemAdd
    (LlamaModel.swift:330-331) -> fp16 [M, N]."""
    out = _new((M, N), _torch().float16, x) if out is None else out
    if M > 0 and N > 0 and _shape_ok(w.K, w.group_size):
        _need(x, "x", M * w.K, _f16())
        _need_w(w, N)
        _need(residual, "residual", M * N, _f16())
        _need(out, "out", M * N, _f16())
    cw = w.c()
    check(lib().sltx_matmul_q4_residual(_ptr(x), ctypes.byref(cw), _ptr(residual), _ptr(out), M,
                                        N, _stream(stream)))
    return out


def matmul_q4_residual_rms_norm(x, w: Q4Weight, residual, norm_weight, eps, M, N, sum_rounded,
                                residual_out=None, norm_out=None, stream=None):
    """linear + residual add + RMSNorm for prefill rows: residual_out =
    half(residual + half(x . dequant(W)^T)), norm_out = rms_norm(residual_out)
    with the sum of squares over the unrounded sum (sum_rounded False: the o_proj
    step's residualRmsNorm, LlamaModel.swift:269-272) or over residual_out
    (True: elemAdd then the next layer's rmsNorm, LlamaModel.swift:278-279, 233)
    -> (residual_out, norm_out), fp16 [M, N]."""
    torch = _torch()
    residual_out = _new((M, N), torch.float16, x) if residual_out is None else residual_out
    norm_out = _new((M, N), torch.float16, x) if norm_out is None else norm_out
    if M > 0 and N > 0 and _shape_ok(w.K, w.group_size):
        _need(x, "x", M * w.K, _f16())
        _need_w(w, N)
        for t, n in ((residual, "residual"), (residual_out, "residual_out"),
                     (norm_out, "norm_out")):
            _need(t, n, M * N, _f16())
        _need(norm_weight, "norm_weight", N, (torch.float32,))
    cw = w.c()
    check(lib().sltx_matmul_q4_residual_rms_norm(_ptr(x), ctypes.byref(cw), _ptr(residual),
                                                 _ptr(norm_weight), eps, M, N,
                                                 1 if sum_rounded else 0, _ptr(residual_out),
                                                 _ptr(norm_out), _stream(stream)))
    return residual_out, norm_out


ROUTES = {0: "gemm", 1: "small_m", 2: "narrow", 3: "mid", 4: "wide", 5: "gemv"}


def gemm_route(M, N, K, group_size=64, gated=False, x_dtype=None):
    """The kernel family a matmul of this shape runs (sltx_gemm_route):
    "gemm", "small_m", "narrow", "mid", "wide" or "gemv" (M = 2).  No device needed."""
    code = SLTX_F16 if x_dtype is None else _dtype_code(x_dtype)
    rc = lib().sltx_gemm_route(M, N, K, group_size, 1 if gated else 0, code)
    if rc < 0:
        check(rc)
    return ROUTES[rc]


def matmul_q4_geglu(x, gate: Q4Weight, up: Q4Weight, M, K, N, out=None, stream=None):
    """gelu_tanh(x.Wg^T) * (x.Wu^T) -> fp16 [M, N]: the T5 encoder FFN's
    gate/up (T5Encoder.swift:191-199)."""
    out = _new((M, N), _torch().float16, x) if out is None else out
    if M > 0 and N > 0 and _shape_ok(K, gate.group_size):
        _need(x, "x", M * K, _f16())
        _need_w(gate, N, K, "gate")
        _need_w(up, N, K, "up")
        _need(out, "out", M * N, _f16())
    g, u = gate.c(), up.c()
    check(lib().sltx_matmul_q4_geglu(_ptr(x), ctypes.byref(g), ctypes.byref(u), _ptr(out), M, K,
                                     N, _stream(stream)))
    return out


def embedding_q4(table: Q4Weight, vocab, token_ids, out=None, stream=None):
    """embeddingQ4Batch (Ops.swift:163-187): dequantized rows [n, K] fp16 of a
    4-bit table for int32 device token ids."""
    n = int(token_ids.numel())
    out = _new((n, table.K), _torch().float16, token_ids) if out is None else out
    if n > 0 and vocab >= 0 and _shape_ok(table.K, table.group_size):
        _need(token_ids, "token_ids", n, (_torch().int32,))
        _need_w(table, vocab, what="table")
        _need(out, "out", n * table.K, _f16())
    cw = table.c()
    check(lib().sltx_embedding_q4(ctypes.byref(cw), vocab, _ptr(token_ids), n, _ptr(out),
                                  _stream(stream)))
    return out


def _logits_dtype(logits):
    torch = _torch()
    if logits.dtype == torch.float16:
        return SLTX_F16
    if logits.dtype == torch.float32:
        return SLTX_F32
    raise TypeError(f"logits must be float16 or float32, not {logits.dtype}")


def argmax(logits, out=None, stream=None):
    """argmax (Ops.swift:757-781) on the device: int32 [1] tensor holding the
    first index of the maximum of a contiguous fp16/fp32 vector."""
    out = _new((1,), _torch().int32, logits) if out is None else out
    _need(logits, "logits", logits.numel())
    _need(out, "out", 1, (_torch().int32,))
    check(lib().sltx_argmax(_ptr(logits), _logits_dtype(logits), int(logits.numel()), _ptr(out),
                            _stream(stream)))
    return out


def sample(logits, temperature=0.7, top_p=0.9, repetition_penalty=1.1, seen_tokens=None,
           u=None, out=None, stream=None):
    """sample(_:temperature:topP:repetitionPenalty:seenTokens:) (Ops.swift:785-806)
    on the device -> int32 [1] tensor.  seen_tokens: int32 device tensor (or
    None); u: uniform draw in [0, 1) (drawn here with Python's random when
    None, as the reference draws Float.random)."""
    import random
    if u is None:
        u = random.random()
    out = _new((1,), _torch().int32, logits) if out is None else out
    n_seen = 0 if seen_tokens is None else int(seen_tokens.numel())
    _need(logits, "logits", logits.numel())
    _need(out, "out", 1, (_torch().int32,))
    if n_seen:
        _need(seen_tokens, "seen_tokens", n_seen, (_torch().int32,))
    check(lib().sltx_sample_top_p(_ptr(logits), _logits_dtype(logits), int(logits.numel()),
                                  temperature, top_p, repetition_penalty,
                                  _ptr(seen_tokens) if n_seen else None, n_seen, u, _ptr(out),
                                  _stream(stream)))
    return out


def sample_noalloc(logits, temperature, top_p, repetition_penalty, seen_tokens, u, out=None,
                   stream=None):
    """sample(...) through sltx_sample_top_p_noalloc: the same result as
    sample() with the library allocating nothing (a fixed per-GPU scratch,
    at most 262144 logits; calls that overlap on one GPU race on it)."""
    out = _new((1,), _torch().int32, logits) if out is None else out
    n_seen = 0 if seen_tokens is None else int(seen_tokens.numel())
    _need(logits, "logits", logits.numel())
    _need(out, "out", 1, (_torch().int32,))
    if n_seen:
        _need(seen_tokens, "seen_tokens", n_seen, (_torch().int32,))
    check(lib().sltx_sample_top_p_noalloc(_ptr(logits), _logits_dtype(logits),
                                          int(logits.numel()), temperature, top_p,
                                          repetition_penalty,
                                          _ptr(seen_tokens) if n_seen else None, n_seen, u,
                                          _ptr(out), _stream(stream)))
    return out


class SamplerState:
    """sltx_sample_state: the sampler's token history and uniform draws in
    device memory, so a sampled step takes no per-token host argument (the
    reference keeps both on the host: seenTokens = prompt + generated,
    LlamaModel.swift:150-161, and Float.random, Ops.swift:2092).

    history: token ids already seen (the prompt); capacity: history entries
    (the chosen tokens are appended until it is full); draws: uniform draws in
    [0, 1) used one per call, cyclically (a float32 sequence or a count, in
    which case they are drawn here with torch's generator).

    Setup (the constructor, set_history, set_draws) runs on torch's current
    stream and waits for it, so a call on any other stream sees the new
    state."""

    def __init__(self, capacity, draws=4096, history=(), device="cuda", generator=None):
        torch = _torch()
        if capacity < 0:
            raise ValueError("capacity must be >= 0")
        self.history = torch.zeros(max(1, capacity), dtype=torch.int32, device=device)
        self.history_len = torch.zeros(1, dtype=torch.int32, device=device)
        self.capacity = int(capacity)
        if isinstance(draws, int):
            draws = torch.rand(draws, generator=generator, device=device)
        self.draws = torch.as_tensor(draws, dtype=torch.float32, device=device).contiguous()
        if self.draws.numel() < 1:
            raise ValueError("at least one draw")
        self.next_draw = torch.zeros(1, dtype=torch.int32, device=device)
        self.set_history(history)   # waits for the stream
        self.c = CSampleState(_ptr(self.history), _ptr(self.history_len), self.capacity,
                              _ptr(self.draws), _ptr(self.next_draw), int(self.draws.numel()))

    def set_history(self, tokens):
        """Replace the history (e.g. with a new prompt); keeps at most
        `capacity` ids.  Host-side copy: call outside graph capture."""
        torch = _torch()
        t = torch.as_tensor(list(tokens), dtype=torch.int32)[: self.capacity]
        if t.numel():
            self.history[: t.numel()].copy_(t)
        self.history_len.fill_(int(t.numel()))
        torch.cuda.current_stream(self.history.device).synchronize()

    def set_draws(self, draws, start=0):
        """Overwrite the draws in place (same count) and the next index."""
        torch = _torch()
        self.draws.copy_(torch.as_tensor(draws, dtype=torch.float32))
        self.next_draw.fill_(int(start))
        torch.cuda.current_stream(self.draws.device).synchronize()

    def tokens(self):
        """The history as a host list."""
        n = int(self.history_len.item())
        return self.history[:n].tolist()


def sample_with_state(logits, temperature, top_p, repetition_penalty, state, out=None,
                      stream=None):
    """sample(...) with seen tokens and the draw taken from `state` (a
    SamplerState) in device memory; appends the chosen token to the history
    and advances the draw.  Capturable in a HIP graph (after one eager call
    on the same stream, which sizes the workspace)."""
    out = _new((1,), _torch().int32, logits) if out is None else out
    _need(logits, "logits", logits.numel())
    _need(out, "out", 1, (_torch().int32,))
    check(lib().sltx_sample_top_p_state(_ptr(logits), _logits_dtype(logits), int(logits.numel()),
                                        temperature, top_p, repetition_penalty,
                                        ctypes.byref(state.c), _ptr(out), _stream(stream)))
    return out


# ------------------------------------------------------------ safetensors ---
# sltx_st_dtype codes -> (safetensors name, numpy dtype)
ST_DTYPES = {0: ("F32", "float32"), 1: ("F16", "float16"), 2: ("BF16", "uint16"),
             3: ("I8", "int8"), 4: ("U8", "uint8"), 5: ("I32", "int32"), 6: ("U32", "uint32")}


class TensorInfo:
    """TensorInfo (SafeTensors.swift:7-13)."""

    def __init__(self, name, c):
        self.name = name
        self.dtype = ST_DTYPES[c.dtype][0]
        self.code = c.dtype
        self.shape = tuple(int(c.shape[i]) for i in range(c.ndim))
        self.offset = int(c.offset)
        self.byte_count = int(c.nbytes)

    def __repr__(self):
        return f"TensorInfo({self.name!r}, {self.dtype}, {self.shape}, {self.byte_count} B)"


class SafeTensorsFile:
    """SafeTensorsFile (SafeTensors.swift:41-118) over the native reader:
    header parsed at open; tensors read to host (numpy) or straight into a
    device tensor."""

    def __init__(self, path):
        self.path = os.fspath(path)
        h = ctypes.c_void_p()
        check(lib().sltx_st_open(self.path.encode(), ctypes.byref(h)))
        self._h = h
        L = lib()
        self.tensors = {}
        for i in range(L.sltx_st_num_tensors(h)):
            name = L.sltx_st_name(h, i).decode()
            c = CStInfo()
            check(L.sltx_st_info_of(h, name.encode(), ctypes.byref(c)))
            self.tensors[name] = TensorInfo(name, c)

    def close(self):
        if self._h:
            lib().sltx_st_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def read_host(self, name):
        """readTensorRaw (SafeTensors.swift:205-214) -> numpy array (BF16 as uint16 bits)."""
        import numpy as np
        info = self.tensors[name]
        out = np.empty(info.shape, dtype=ST_DTYPES[info.code][1])
        check(lib().sltx_st_read_host(self._h, name.encode(), out.ctypes.data, out.nbytes))
        return out

    def read_device(self, name, out, byte_offset=0, stream=None):
        """Raw bytes of `name` into device tensor `out` at byte_offset."""
        cap = out.numel() * out.element_size() - byte_offset
        check(lib().sltx_st_read_device(self._h, name.encode(), out.data_ptr() + byte_offset, cap,
                                        _stream(stream)))
        return out

    def read_device_f32(self, name, out, stream=None):
        """loadFloat (ModelWeights.swift:96-108): F32/F16/BF16 widened to fp32."""
        check(lib().sltx_st_read_device_f32(self._h, name.encode(), out.data_ptr(), out.numel(),
                                            _stream(stream)))
        return out


def load_safetensors(directory):
    """loadSafeTensors(from:) (SafeTensors.swift:256-262): every *.safetensors
    file in the directory, sorted by file name."""
    names = sorted(f for f in os.listdir(directory) if f.endswith(".safetensors"))
    return [SafeTensorsFile(os.path.join(directory, f)) for f in names]
