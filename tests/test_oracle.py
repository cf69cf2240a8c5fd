"""Pins the CPU oracle (oracle/q4_oracle.{c,py}) independently of itself.

The reference holds no golden vectors for the 4-bit matmul (its tests never
call it), so each oracle function is checked against what the mathematics or
a library routine fixes, chosen so that a dropped term, a wrong sign, a
wrong index or a transposed operand fails at least one check:
  * fp16 conversions: bit-exact against numpy's float16 casts.
  * nibble order: known-answer words, and MLX's pack convention round trip.
  * matmul: brute-force pure-Python loops, exact integer products (s=1, b=0),
    b=-8s with all-8 codes giving exactly 0, linearity in x, group
    permutation invariance, and a scale/bias transposition trap (N != K/g).
  * silu_mul / gelu: closed forms through math.exp / math.tanh.
"""
import math

import numpy as np
import pytest


# ------------------------------------------------------------------ fp16 ---

def test_f16_to_f32_all_patterns(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = oracle.c_f16_to_f32(bits)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne_matches_numpy(oracle):
    rng = np.random.default_rng(0)
    # random bit patterns over the whole float range plus targeted edge cases
    pats = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    vals = pats.view(np.float32)
    edge = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 65536.0, -65520.0, 1e-8, 2.0**-24,
                     2.0**-25, 2.0**-25 * 1.0000001, 3 * 2.0**-25, 2.0**-14, 2.0**-14 * 0.99999,
                     1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, 2048.0 + 1.0, 2048.0 + 3.0,
                     np.inf, -np.inf], dtype=np.float32)
    # exact ties in the normal and subnormal ranges
    ties = (np.arange(1, 2000, dtype=np.float32) + 0.5) * np.float32(2.0**-24)
    vals = np.concatenate([vals, edge, ties, rng.standard_normal(50_000).astype(np.float32) * 100])
    L = oracle.lib()
    got = np.array([L.oracle_f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    nan = np.isnan(vals)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all(np.isnan(got[nan].view(np.float16)))


# ---------------------------------------------------------------- nibbles ---

def test_unpack_known_words(oracle):
    w = np.array([[0x76543210, 0xFEDCBA98, 0x0000000F, 0xF0000000]], dtype=np.uint32)
    want = np.array([list(range(8)) + list(range(8, 16)) + [15] + [0] * 7 + [0] * 7 + [15]],
                    dtype=np.uint8)
    assert np.array_equal(oracle.unpack_q4(w), want)
    assert np.array_equal(oracle.c_unpack_q4(w, 32), want)


def test_pack_unpack_roundtrip(oracle):
    rng = np.random.default_rng(1)
    q = rng.integers(0, 16, size=(37, 256), dtype=np.uint8)
    w = oracle.pack_q4(q)
    assert w.dtype == np.uint32 and w.shape == (37, 32)
    assert np.array_equal(oracle.unpack_q4(w), q)
    assert np.array_equal(oracle.c_unpack_q4(w, 256), q)
    # low nibble first: code k sits at bits 4*(k%8) of word k/8
    k = 13
    assert ((w[:, k // 8] >> (4 * (k % 8))) & 0xF).astype(np.uint8).tolist() == q[:, k].tolist()


# ----------------------------------------------------------------- matmul ---

def _brute(x, w, s, b, g):
    """Pure-Python loops straight from the formula, tiny shapes only."""
    M, K = x.shape
    N = w.shape[0]
    y = [[0.0] * N for _ in range(M)]
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                q = (int(w[n, k // 8]) >> (4 * (k % 8))) & 0xF
                wk = float(s[n, k // g]) * q + float(b[n, k // g])
                acc += float(x[m, k]) * wk
            y[m][n] = acc
    return np.array(y)


@pytest.mark.parametrize("M,N,K,g", [(2, 3, 64, 32), (1, 5, 128, 64), (3, 4, 256, 128)])
def test_matmul_brute_force(oracle, M, N, K, g):
    x, [(w, s, b)] = oracle.make_inputs(M, N, K, g, seed=K + N)
    # non-uniform biases so a dropped or misplaced bias term shows
    rng = np.random.default_rng(7)
    b = (rng.standard_normal(b.shape) * 0.1).astype(np.float16)
    ref = _brute(x, w, s, b, g)
    assert np.allclose(oracle.matmul_q4_f64(x, w, s, b, g), ref, rtol=1e-12, atol=1e-12)
    assert np.allclose(oracle.c_matmul_q4_f64(x, w, s, b, g), ref, rtol=1e-12, atol=1e-12)


def test_exact_integer_matmul(oracle):
    rng = np.random.default_rng(2)
    M, N, K, g = 4, 24, 192, 64
    q = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    xi = rng.integers(-8, 9, size=(M, K))
    w = oracle.pack_q4(q)
    s = np.ones((N, K // g), np.float16)
    b = np.zeros((N, K // g), np.float16)
    want = xi @ q.astype(np.int64).T
    x = xi.astype(np.float16)
    assert np.array_equal(oracle.matmul_q4_f64(x, w, s, b, g), want.astype(np.float64))
    assert np.array_equal(oracle.c_matmul_q4_f64(x, w, s, b, g), want.astype(np.float64))
    # emulator and CPU baseline are exact here too (integers < 2048 in fp16)
    assert np.array_equal(oracle.c_matmul_q4_emu(x, w, s, b, g).astype(np.int64), want)
    assert np.array_equal(oracle.c_cpu_matmul_q4(x, w, s, b, g, 2).astype(np.int64), want)


def test_all_eight_codes_with_minus8s_bias_is_zero(oracle):
    M, N, K, g = 3, 16, 128, 64
    x, [(w, s, b)] = oracle.make_inputs(M, N, K, g, seed=3)
    w8 = oracle.pack_q4(np.full((N, K), 8, np.uint8))
    assert np.all(oracle.matmul_q4_f64(x, w8, s, b, g) == 0.0)
    assert np.all(oracle.c_matmul_q4_f64(x, w8, s, b, g) == 0.0)
    # matmul_q4 keeps q*s*x and b*sum(x) in separate fp32 accumulators
    # (Kernels.swift:547-600), so its cancellation is only to fp32 rounding.
    emu = oracle.c_matmul_q4_emu(x, w8, s, b, g).astype(np.float32)
    assert np.all(np.abs(emu) < 1e-5) and np.any(emu != 0.0)


def test_linearity_in_x(oracle):
    M, N, K, g = 2, 32, 256, 64
    x1, [(w, s, b)] = oracle.make_inputs(M, N, K, g, seed=4)
    x2, _ = oracle.make_inputs(M, N, K, g, seed=5)
    a = 0.37
    lhs = oracle.matmul_q4_f64(a * x1.astype(np.float64) + x2.astype(np.float64), w, s, b, g)
    rhs = a * oracle.matmul_q4_f64(x1, w, s, b, g) + oracle.matmul_q4_f64(x2, w, s, b, g)
    assert np.allclose(lhs, rhs, rtol=1e-10, atol=1e-10)


def test_group_permutation_invariance(oracle):
    M, N, K, g = 2, 16, 256, 64
    x, [(w, s, b)] = oracle.make_inputs(M, N, K, g, seed=6)
    rng = np.random.default_rng(9)
    b = (rng.standard_normal(b.shape) * 0.05).astype(np.float16)
    perm = np.array([2, 0, 3, 1])
    q = oracle.unpack_q4(w)
    kperm = np.concatenate([np.arange(p * g, (p + 1) * g) for p in perm])
    y0 = oracle.c_matmul_q4_f64(x, w, s, b, g)
    y1 = oracle.c_matmul_q4_f64(np.ascontiguousarray(x[:, kperm]), oracle.pack_q4(q[:, kperm]),
                                np.ascontiguousarray(s[:, perm]), np.ascontiguousarray(b[:, perm]),
                                g)
    assert np.allclose(y0, y1, rtol=1e-12, atol=1e-12)


def test_scale_bias_index_trap(oracle):
    """N == K/g with row-distinct scales: reading s[g, n] instead of s[n, g]
    (or dropping the bias) changes the result."""
    M, N, K, g = 1, 4, 256, 64
    x, [(w, s, b)] = oracle.make_inputs(M, N, K, g, seed=10)
    s = (np.arange(16, dtype=np.float32).reshape(4, 4) * 0.01 + 0.01).astype(np.float16)
    b = (-np.arange(16, dtype=np.float32).reshape(4, 4) * 0.02).astype(np.float16)
    y = oracle.c_matmul_q4_f64(x, w, s, b, g)
    assert np.allclose(y, _brute(x, w, s, b, g), rtol=1e-12, atol=1e-12)
    assert not np.allclose(y, oracle.matmul_q4_f64(x, w, np.ascontiguousarray(s.T),
                                                   np.ascontiguousarray(b.T), g))
    assert not np.allclose(y, oracle.matmul_q4_f64(x, w, s, np.zeros_like(b), g))


def test_emulator_within_two_ulp(oracle):
    M, N, K, g = 1, 256, 3072, 64
    x, [(w, s, b)] = oracle.make_inputs(M, N, K, g, seed=11)
    ref = oracle.matmul_q4_f64(x, w, s, b, g)
    emu = oracle.c_matmul_q4_emu(x, w, s, b, g).astype(np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(emu - ref) <= 2 * ulp + 1e-6)


def test_cpu_baseline_matches_f64(oracle):
    M, N, K, g = 3, 100, 512, 64
    x, [(w, s, b)] = oracle.make_inputs(M, N, K, g, seed=12)
    ref = oracle.matmul_q4_f64(x, w, s, b, g)
    for th in (1, 3):
        y = oracle.c_cpu_matmul_q4(x, w, s, b, g, th)
        ok, worst = oracle.elementwise_ok(y, ref, rtol=6e-4, atol_rms=1e-4)
        assert ok, worst


def test_baseline_distribution(oracle):
    """The benchmark's synthetic inputs: |y| has std ~5 at K=3072, bias == -8*scale exactly."""
    x, [(w, s, b)] = oracle.make_inputs(64, 256, 3072, 64, seed=0)
    assert np.array_equal(b.astype(np.float32), -8.0 * s.astype(np.float32))
    std = oracle.matmul_q4_f64(x, w, s, b, 64).std()
    assert 4.0 < std < 6.5


# ------------------------------------------------------------ activations ---

def test_silu_mul_closed_form(oracle):
    rng = np.random.default_rng(13)
    a = (rng.standard_normal(4096) * 4).astype(np.float16)
    bb = rng.standard_normal(4096).astype(np.float16)
    got = oracle.c_silu_mul(a, bb).astype(np.float64)
    ref = np.array([float(u) / (1.0 + math.exp(-float(u))) * float(v) for u, v in zip(a, bb)])
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - ref) <= ulp)
    assert np.allclose(oracle.silu_mul_f64(a, bb), ref, rtol=1e-12, atol=0)


def test_silu_mul_special_values(oracle):
    a = np.array([0.0, 20.0, -30.0, 1.0], np.float16)
    b = np.array([3.0, 2.0, 1.0, 0.0], np.float16)
    out = oracle.c_silu_mul(a, b)
    assert out[0] == 0.0
    assert out[1] == np.float16(40.0)
    assert out[2] == 0.0 and np.signbit(out[2])
    assert out[3] == 0.0


def test_gelu_tanh_closed_form_and_clamp(oracle):
    v = np.concatenate([np.linspace(-12, 12, 2001), [0.0, 50.0, -50.0]]).astype(np.float32)
    got = oracle.c_gelu_tanh_f32(v).astype(np.float64)

    def ref1(t):
        inner = 0.7978845608 * (t + 0.044715 * t ** 3)
        inner = min(max(inner, -10.0), 10.0)
        return 0.5 * t * (1.0 + math.tanh(inner))

    ref = np.array([ref1(float(t)) for t in v])
    assert np.allclose(got, ref, rtol=2e-6, atol=2e-6)
    assert np.allclose(oracle.gelu_tanh_f64(v), ref, rtol=1e-12, atol=1e-12)
    # clamp: for large |v| the inner term saturates at +-10, not at +-inf
    big = oracle.gelu_tanh_f64(np.array([-50.0]))[0]
    assert big == pytest.approx(0.5 * -50.0 * (1.0 + math.tanh(-10.0)), rel=1e-12)


def test_bf16_rounding(oracle):
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 3.0e38], np.float32)
    bits = oracle.f32_to_bf16_bits(vals)
    back = oracle.bf16_bits_to_f32(bits)
    assert back[0] == 1.0
    assert back[1] == 1.0          # tie to even
    assert back[2] == 1.0 + 2 ** -6  # tie to even (up)
    assert back[3] == -2.5
    L = oracle.lib()
    L.oracle_f32_to_bf16.argtypes = [__import__("ctypes").c_float]
    L.oracle_f32_to_bf16.restype = __import__("ctypes").c_uint16
    assert [L.oracle_f32_to_bf16(float(v)) for v in vals] == bits.tolist()


# ------------------------------------------------ norms and residual add ---
# rms_norm / residual_rms_norm (Kernels.swift:40-86, :238-290) are pinned by
# what the definition fixes: a constant vector maps to sign(c) * w, the output
# of a unit-weight norm has RMS 1 and points along x, power-of-two scaling of x
# leaves it bit-identical (eps = 0), b = 0 reduces the residual form to the
# plain one, and the residual equals numpy's own fp16 addition.

def test_cast_f32_to_f16_clamp_known_values(oracle):
    """cast_f32_to_f16 (Kernels.swift:816-822) on values whose fp16 results
    are fixed by hand: the clamp holds the finite range at the largest fp16,
    65504 (without it 65520 and beyond round to infinity), NaN takes the
    lower bound (Metal's fmax returns the non-NaN operand), and inside the
    range the cast is round-to-nearest-even: 1 + 2^-11 is a tie that stays
    at 1, 1 + 3 * 2^-11 rounds up to 1 + 2^-9, 2^-24 is the smallest fp16
    subnormal and 2^-26 rounds to zero."""
    x = np.array([1e6, -1e6, 65520.0, -65520.0, 65519.0, 70000.0, np.inf, -np.inf, np.nan,
                  1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 2.0 ** -24, 2.0 ** -26, -2.5, 0.0],
                 dtype=np.float32)
    want = [65504.0, -65504.0, 65504.0, -65504.0, 65504.0, 65504.0, 65504.0, -65504.0, -65504.0,
            1.0, 1.0 + 2.0 ** -9, 2.0 ** -24, 0.0, -2.5, 0.0]
    got = oracle.cast_f32_to_f16_ref(x)
    assert got.dtype == np.float16
    assert got.astype(np.float64).tolist() == want
    # without the clamp the same inputs overflow: the clamp is what keeps them finite
    assert np.isinf(np.float32(65520.0).astype(np.float16))


def test_rms_norm_constant_vector():
    from oracle import q4_oracle as o
    w = np.array([0.5, 1.25, -2.0, 3.0] * 16, dtype=np.float32)
    for c in (0.75, -3.0, 0.001):
        x = np.full((1, 64), c, dtype=np.float16)
        out = o.rms_norm_ref(x, w, 0.0)
        assert np.array_equal(out[0], (np.sign(c) * w).astype(np.float16))


def test_rms_norm_unit_rms_and_direction():
    from oracle import q4_oracle as o
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 3072)).astype(np.float16) * np.float16(7)
    out = o.rms_norm_ref(x, np.ones(3072, np.float32), 1e-6).astype(np.float64)
    rms = np.sqrt(np.mean(out ** 2, axis=1))
    assert np.all(np.abs(rms - 1.0) < 1e-3)
    xf = x.astype(np.float64)
    cos = np.sum(out * xf, axis=1) / (np.linalg.norm(out, axis=1) * np.linalg.norm(xf, axis=1))
    assert np.all(cos > 1 - 1e-6)


def test_rms_norm_power_of_two_scaling_exact():
    from oracle import q4_oracle as o
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 256)).astype(np.float16)
    w = rng.standard_normal(256).astype(np.float32)
    base = o.rms_norm_ref(x, w, 0.0)
    for k in (-3, 2, 5):
        xs = (x.astype(np.float32) * 2.0 ** k).astype(np.float16)
        assert np.array_equal(xs.astype(np.float32), x.astype(np.float32) * 2.0 ** k)
        assert np.array_equal(o.rms_norm_ref(xs, w, 0.0), base)


def test_rms_norm_eps_dominates_zero_vector():
    from oracle import q4_oracle as o
    out = o.rms_norm_ref(np.zeros((1, 32), np.float16), np.ones(32, np.float32), 1e-5)
    assert np.array_equal(out, np.zeros((1, 32), np.float16))


def test_residual_rms_norm_reductions():
    from oracle import q4_oracle as o
    rng = np.random.default_rng(5)
    a = rng.standard_normal((2, 512)).astype(np.float16)
    b = rng.standard_normal((2, 512)).astype(np.float16)
    w = rng.standard_normal(512).astype(np.float32)
    res, nrm = o.residual_rms_norm_ref(a, b, w, 1e-5)
    assert np.array_equal(res, a + b)                       # numpy's fp16 add
    r2, n2 = o.residual_rms_norm_ref(b, a, w, 1e-5)
    assert np.array_equal(res, r2) and np.array_equal(nrm, n2)
    r0, n0 = o.residual_rms_norm_ref(a, np.zeros_like(a), w, 1e-5)
    assert np.array_equal(r0, a)
    assert np.array_equal(n0, o.rms_norm_ref(a, w, 1e-5))


def test_residual_add_ref():
    from oracle import q4_oracle as o
    rng = np.random.default_rng(6)
    r = rng.standard_normal(64).astype(np.float16)
    y = rng.standard_normal(64) * 3
    assert np.array_equal(o.residual_add_ref(np.zeros(64, np.float16), y), y.astype(np.float16))
    assert np.array_equal(o.residual_add_ref(r, np.zeros(64)), r)
    assert np.array_equal(o.residual_add_ref(r, y), r + y.astype(np.float16))


def test_embedding_q4_ref_exact_and_closed_form(oracle):
    """Rows match the fp64 closed form exactly when every value is
    representable (power-of-two scales, integer biases) and to 1 fp16 ulp
    otherwise; bad ids give zero rows; row order follows the ids."""
    from oracle import q4_oracle as o
    rng = np.random.default_rng(9)
    V, K, g = 40, 256, 64
    q = rng.integers(0, 16, (V, K))
    w = o.pack_q4(q)
    s = (2.0 ** -rng.integers(0, 6, (V, K // g))).astype(np.float16)
    b = rng.integers(-8, 8, (V, K // g)).astype(np.float16)
    ids = [3, 0, 39, 3, -1, 40]
    out = o.embedding_q4_ref(w, s, b, ids, g)
    ref = o.dequant_f64(w, s, b, g)
    assert np.array_equal(out[:4].astype(np.float64), ref[[3, 0, 39, 3]])
    assert not out[4:].any()
    s2 = (np.abs(rng.standard_normal((V, K // g))) * 0.02).astype(np.float16)
    b2 = (-8 * s2.astype(np.float32)).astype(np.float16)
    out2 = o.embedding_q4_ref(w, s2, b2, [5, 17], g).astype(np.float64)
    ref2 = o.dequant_f64(w, s2, b2, g)[[5, 17]]
    assert np.all(np.abs(out2 - ref2) <= np.spacing(np.abs(ref2).astype(np.float16)))


# -------------------------------------------------------- token selection --
# argmax_ref: a pure-Python transcription of the scan on small vectors, and
# numpy's argmax (first occurrence) wherever no NaN is present.
# sample_ref: a hand-worked nucleus, the closed forms that a vanishing top_p
# reduces sampling to argmax of the penalised logits and u = 0 to the most
# probable token, penalties applied once per distinct id, and an inverse-CDF
# count over a grid of u that reproduces the fp64 softmax of logits / T.

def _scan_argmax(v):
    best, bv = 0, float(v[0])
    for i in range(1, len(v)):
        if float(v[i]) > bv:
            best, bv = i, float(v[i])
    return best


def test_argmax_ref_scan_and_numpy():
    from oracle import q4_oracle as o
    rng = np.random.default_rng(20)
    for n in (1, 2, 17, 300):
        for dt in (np.float16, np.float32):
            v = rng.standard_normal(n).astype(dt)
            assert o.argmax_ref(v) == int(np.argmax(v)) == _scan_argmax(v)
            v = rng.integers(-3, 3, n).astype(dt)            # many ties: first wins
            assert o.argmax_ref(v) == int(np.argmax(v)) == _scan_argmax(v)
    nan, inf = np.nan, np.inf
    for v in ([nan, 5.0, 7.0], [1.0, nan, 7.0, 7.0], [-inf, -inf], [-inf, nan], [2.0, inf, inf, nan],
              [nan], [0.0, -0.0]):
        a = np.array(v, dtype=np.float32)
        assert o.argmax_ref(a) == _scan_argmax(a), v
    assert o.argmax_ref(np.array([nan, 5.0], np.float32)) == 0
    assert o.argmax_ref(np.array([1.0, nan, 7.0, 7.0], np.float32)) == 2


def test_sample_ref_hand_worked_nucleus():
    """p = [0.1, 0.2, 0.3, 0.4]: order 3, 2, 1, 0; top_p 0.65 keeps {3, 2}
    (running sums 0.4, 0.7) and r = u * 0.7 picks 3 below r = 0.4, else 2."""
    from oracle import q4_oracle as o
    lg = np.log(np.array([1.0, 2.0, 3.0, 4.0])).astype(np.float32)
    for u, tok in ((0.0, 3), (0.5, 3), (0.6, 2), (0.9, 2), (0.999, 2)):
        assert o.sample_ref(lg, 1.0, 0.65, 1.0, [], u) == tok, u
    for u, tok in ((0.05, 3), (0.5, 2), (0.8, 1), (0.95, 0)):   # top_p 0.95: all four
        assert o.sample_ref(lg, 1.0, 0.95, 1.0, [], u) == tok, u
    t, info = o.sample_ref(lg, 1.0, 0.65, 1.0, [], 0.5, detail=True)
    assert info["cutoff"] == 2 and list(info["order"]) == [3, 2, 1, 0]
    assert abs(info["cum"] - 0.7) < 1e-6


def test_sample_ref_tiny_top_p_is_penalised_argmax():
    from oracle import q4_oracle as o
    rng = np.random.default_rng(21)
    for n in (5, 64, 1000):
        lg = (rng.standard_normal(n) * 3).astype(np.float32)
        seen = rng.integers(0, n, 7)
        pen = lg.copy()
        for t in set(seen.tolist()):
            pen[t] = pen[t] / np.float32(1.3) if pen[t] > 0 else pen[t] * np.float32(1.3)
        for u in (0.0, 0.37, 0.999):
            for T in (0.5, 1.0, 2.0):
                assert o.sample_ref(lg, T, 1e-9, 1.3, seen, u) == int(np.argmax(pen))


def test_sample_ref_penalty_once_per_token_and_sign():
    from oracle import q4_oracle as o
    a = np.array([2.0, 1.7], np.float32)            # once: 1.818 > 1.7; twice: 1.653 < 1.7
    assert o.sample_ref(a, 1.0, 1e-9, 1.1, [0, 0, 0], 0.5) == 0
    b = np.array([-1.0, -1.05], np.float32)         # non-positive logits are multiplied
    assert o.sample_ref(b, 1.0, 1e-9, 1.1, [0], 0.5) == 1
    c = np.array([0.0, -0.01], np.float32)          # zero counts as non-positive: stays 0
    assert o.sample_ref(c, 1.0, 1e-9, 5.0, [0], 0.5) == 0
    assert o.sample_ref(a, 1.0, 1e-9, 1.1, [2, 99, -1], 0.5) == 0   # ids >= n are ignored


def test_sample_ref_u_grid_reproduces_softmax():
    """top_p above 1 keeps every token; over u = (j + 1/2) / G the walk is
    the inverse CDF of the sorted probabilities, so token t is drawn
    G * p_t times (within one count per token boundary), p = fp64
    softmax(logits / T)."""
    from oracle import q4_oracle as o
    rng = np.random.default_rng(22)
    lg = rng.standard_normal(12).astype(np.float32)
    for T in (0.7, 1.0, 1.9):
        G = 20000
        counts = np.zeros(12, np.int64)
        for j in range(G):
            counts[o.sample_ref(lg, T, 1.5, 1.0, [], (j + 0.5) / G)] += 1
        z = lg.astype(np.float64) / np.float64(np.float32(T))
        p = np.exp(z - z.max())
        p /= p.sum()
        assert np.all(np.abs(counts - G * p) <= 2.0), (T, counts, G * p)


def test_sample_ref_nucleus_support_and_renormalisation():
    """For top_p < 1 only the shortest most-probable prefix reaching top_p is
    drawn, in proportion to its renormalised probabilities."""
    from oracle import q4_oracle as o
    p = np.array([0.05, 0.3, 0.1, 0.25, 0.2, 0.1])
    lg = np.log(p).astype(np.float32)
    G = 10000
    counts = np.zeros(6, np.int64)
    for j in range(G):
        counts[o.sample_ref(lg, 1.0, 0.7, 1.0, [], (j + 0.5) / G)] += 1
    keep = [1, 3, 4]                                 # 0.3 + 0.25 + 0.2 = 0.75 >= 0.7
    assert set(np.nonzero(counts)[0]) == set(keep)
    assert np.all(np.abs(counts[keep] - G * p[keep] / 0.75) <= 2.0)


def test_sample_ref_gpu_sums_agree_with_reference_sums():
    """The exact-mass form differs from the reference's sequential fp32 sums
    only by rounding: on the hand-worked nucleus and grids far from token
    boundaries both give the same token."""
    from oracle import q4_oracle as o
    lg = np.log(np.array([1.0, 2.0, 3.0, 4.0])).astype(np.float32)
    for top_p, u in ((0.65, 0.0), (0.65, 0.5), (0.65, 0.6), (0.95, 0.05), (0.95, 0.5),
                     (0.95, 0.8), (0.95, 0.95), (1e-9, 0.7), (2.0, 0.3)):
        assert o.sample_ref(lg, 1.0, top_p, 1.0, [], u, gpu_sums=True) == \
            o.sample_ref(lg, 1.0, top_p, 1.0, [], u), (top_p, u)
    rng = np.random.default_rng(23)
    agree = 0
    for k in range(200):
        x = (rng.standard_normal(3000) * 2).astype(np.float32)
        u = float(rng.random())
        a = o.sample_ref(x, 0.8, 0.9, 1.1, [1, 2, 2], u, gpu_sums=True)
        b, info = o.sample_ref(x, 0.8, 0.9, 1.1, [1, 2, 2], u, detail=True)
        agree += a == b
        pos = list(info["order"]).index(a)
        c = np.cumsum(info["probs"].astype(np.float64))
        assert c[pos] >= info["r"] - 1e-5 and (pos == 0 or c[pos - 1] <= info["r"] + 1e-5)
    assert agree >= 190


@pytest.mark.parametrize("M,N,K,g", [(1, 96, 256, 64), (3, 40, 512, 32), (5, 64, 1024, 128),
                                     (1, 257, 3072, 64)])
def test_cpu_baselines_match_the_closed_form(oracle, M, N, K, g):
    """The CPU baselines timed beside the GPU (q4_cpu_baseline.c: scalar in
    matmulCPU's loop shape, 8-wide SIMD over threads) compute the reference
    semantics: within the GEMV bound of the fp64 closed form, the SIMD result
    independent of the thread count, and both exactly 0 for all-8 codes with
    b = -8s."""
    x, [(w, s, b)] = oracle.make_inputs(M, N, K, g, seed=M * 7 + N)
    ref = oracle.matmul_q4_f64(x, w, s, b, g)
    ys = oracle.cpu_q4_scalar(x, w, s, b, g).astype(np.float64)
    y1 = oracle.cpu_q4_simd(x, w, s, b, g, 1)
    y3 = oracle.cpu_q4_simd(x, w, s, b, g, 3)
    for y, what in ((ys, "scalar"), (y1.astype(np.float64), "simd")):
        ok, worst = oracle.elementwise_ok(y, ref, rtol=6e-4, atol_rms=1e-4)
        assert ok, (what, worst)
    assert np.array_equal(y1, y3)
    w8 = np.full_like(w, 0x88888888)
    b8 = (-8.0 * s.astype(np.float32)).astype(np.float16)
    assert not np.any(oracle.cpu_q4_scalar(x, w8, s, b8, g).astype(np.float64))
    assert not np.any(oracle.cpu_q4_simd(x, w8, s, b8, g, 2).astype(np.float64))
