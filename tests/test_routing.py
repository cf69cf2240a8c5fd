"""Which kernel family a matmul runs, through sltx_gemm_route (no device
needed): the rules run_gemm applies between the MFMA GEMM, the mid-M, small-M
and narrow weight streams, on the Llama-3.2-3B, T5-XXL and vocabulary-head
shapes they were measured on, and the routes the GPU parity tests of each
small-M kernel rely on.
"""
import pytest

import test_gpu_mid
import test_gpu_narrow
import test_gpu_skinny

LLAMA_PAIR = dict(N=8192, K=3072, gated=True)
T5_WI_PAIR = dict(N=10240, K=4096, gated=True)


@pytest.mark.parametrize("M", [2, 4, 8, 16])
def test_gated_pairs_stream_on_the_small_m_route(pkg, M):
    assert pkg.gemm_route(M, **LLAMA_PAIR) == "small_m"
    assert pkg.gemm_route(M, **T5_WI_PAIR) == "small_m"


@pytest.mark.parametrize("M", [17, 20, 24, 32])
def test_mid_m_route_above_16_rows(pkg, M):
    """17..32 rows at K = 2048 / 3072 take the mid-M route (Llama gate/up pair
    11.9 against 15.3 us at M = 32, q|k|v 6.7 against 14.9, o 6.4 against 8.8,
    a single 8192-row set 7.6 against 10.4), and at K = 8192 / 10240, where
    the small-M route does not run (Llama down 15.4 against the GEMM's 23.0,
    T5 wo 14.9 against 26.9; with K in two halves now 11.5 and 11.2).  At
    K = 4096 a single set of at most 4096 rows, which it splits over K, takes
    it above 16 rows (T5 q/k/v/o 8.0 against 8.9 at M = 20), any other above
    24 rows (the T5 GeGLU pair 31.5 against 36.7 at M = 32); a gated pair at
    group size 32 fits the LDS at K = 2048 only."""
    assert pkg.gemm_route(M, **LLAMA_PAIR) == "mid"
    for N in (5120, 3072, 8192, 64, 33):
        assert pkg.gemm_route(M, N, 3072) == "mid", N
    assert pkg.gemm_route(M, 3072, 3072, group_size=32) == "mid"
    assert pkg.gemm_route(M, 3072, 8192) == "mid"
    assert pkg.gemm_route(M, 4096, 10240) == "mid"
    assert pkg.gemm_route(M, **T5_WI_PAIR) == ("mid" if M > 24 else "small_m")
    assert pkg.gemm_route(M, 4096, 4096) == "mid"
    assert pkg.gemm_route(M, 5120, 4096) == ("mid" if M > 24 else "small_m")   # no split
    assert pkg.gemm_route(M, 8192, 3072, group_size=32, gated=True) == "small_m"   # LDS
    assert pkg.gemm_route(M, 8192, 2048, group_size=32, gated=True) == "mid"   # 160 KB


@pytest.mark.parametrize("M", [9, 12, 16])
def test_mid_m_route_for_one_set_above_8_rows(pkg, M):
    """9..16 rows: one weight set of 4096..16384 rows at K <= 3072 takes the
    mid-M route (q|k|v 6.5 against 8.5 us at M = 12), and so does a set of at
    most 4096 rows that it splits over K, at K = 10240 (T5 wo 10.9-11.1
    against 12.6 / 14.3 / 16.0 us at M = 9 / 12 / 16; from M = 6) and above 12 rows at
    K = 8192 (Llama down 11.4 against 12.6 at M = 16, 11.4 against 11.2 at
    M = 12); o (3072 rows), the vocabulary head, T5 q/k/v/o (K = 4096: 8.0
    against 7.3 at M = 16) and gated pairs stay on the small-M route."""
    assert pkg.gemm_route(M, 5120, 3072) == "mid"
    assert pkg.gemm_route(M, 8192, 3072) == "mid"
    assert pkg.gemm_route(M, 16384, 2048) == "mid"
    assert pkg.gemm_route(M, 4096, 10240) == "mid"
    assert pkg.gemm_route(M, 3072, 8192) == ("mid" if M > 12 else "small_m")
    assert pkg.gemm_route(M, 3072, 3072) == "small_m"
    assert pkg.gemm_route(M, 4096, 4096) == "small_m"
    assert pkg.gemm_route(M, 128256, 3072) == "small_m"
    assert pkg.gemm_route(M, **LLAMA_PAIR) == "small_m"


@pytest.mark.parametrize("N,K", [(5120, 3072), (3072, 3072), (3072, 8192), (4096, 4096),
                                 (4096, 10240)])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_one_weight_set_at_m_le_4_is_narrow(pkg, N, K, M):
    """M = 2 through a set of at most 5120 x 4096 takes the two-row GEMV
    (Llama o 3.48 against 4.11 us on the narrow route, q|k|v 5.18 / 5.35,
    T5 q/k/v/o 4.54 / 4.78); the rest of M <= 4 the narrow route."""
    if M == 2 and K <= 4096 and N <= 5120:
        assert pkg.gemm_route(M, N, K) == "gemv"
    elif K == 10240 and M > 3:   # X = M * K * 2 bytes over the route's 78 KB of LDS
        assert pkg.gemm_route(M, N, K) == "small_m"
    else:
        assert pkg.gemm_route(M, N, K) == "narrow"


def test_t5_wo_takes_the_split_mid_route_from_6_rows(pkg):
    """T5 wo (4096 x 10240) splits K in halves on the mid-M route from M = 6
    (11.1 against 11.5 / 12.5 us on the small-M route at M = 6 / 8; even at
    M = 5)."""
    assert pkg.gemm_route(5, 4096, 10240) == "small_m"
    for M in (6, 7, 8, 16, 32):
        assert pkg.gemm_route(M, 4096, 10240) == "mid", M
    assert pkg.gemm_route(8, 4200, 10240) == "small_m"   # 132 blocks: no split


@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_vocabulary_head_takes_two_row_tiles(pkg, M):
    """128256 x 3072: the small-M route's two-tile block fits two per CU, and
    is faster than the narrow route (44 vs 47 us at M = 2)."""
    assert pkg.gemm_route(M, 128256, 3072) == "small_m"


@pytest.mark.parametrize("N,K", [(5120, 3072), (3072, 8192), (4096, 4096), (8192, 3072)])
def test_m_above_4_leaves_the_narrow_route(pkg, N, K):
    for M in (5, 8, 16, 32):
        # 17..32 activation rows take at most 4 steps of 1024 k per wave
        want = "gemm" if M > 16 and K > 4096 else "small_m"
        if K in (2048, 3072) and (M > 16 or (M > 8 and 4096 <= N <= 16384)):
            want = "mid"
        if M > 24 or (M > 16 and K > 4096):   # K = 4096 / 8192 above the small-M route
            want = "mid"
        if N <= 4096 and K in (4096, 8192) and M > (12 if K == 8192 else 16):   # K halves
            want = "mid"
        assert pkg.gemm_route(M, N, K) == want, (M, N, K)


def test_large_m_and_unsupported_shapes_take_the_gemm(pkg):
    import torch
    assert pkg.gemm_route(750, **LLAMA_PAIR) == "gemm"
    assert pkg.gemm_route(257, 8192, 3072) == "gemm"
    assert pkg.gemm_route(128, 8192, 3072, x_dtype=torch.bfloat16) == "gemm"
    assert pkg.gemm_route(2, 3072, 8192, x_dtype=torch.bfloat16) == "gemm"
    assert pkg.gemm_route(9, 24, 14336, group_size=32) == "gemm"   # past both step counts
    assert pkg.gemm_route(100, 64, 192) == "gemm"                  # K not a multiple of 128


@pytest.mark.parametrize("M", [33, 64, 100, 128, 200, 256])
def test_wide_m_routing(pkg, M):
    """33..256 rows (T5Encoder.swift:72-78, short prompts): the wide-M route
    when its grid (64 weight rows per block, at most 128 activation rows per
    block, K split until the grid fills the GPU) is one round of 256 blocks,
    or two at M <= 64; else the GEMM (measured: a second round repeats the
    whole per-block time)."""
    one = lambda N, K, gated=False: pkg.gemm_route(M, N, K, gated=gated)
    pair = lambda d: pkg.gemm_route(M, d["N"], d["K"], gated=True)
    # one round at every M: Llama q|k|v, o, down; T5 q/k/v/o
    assert one(5120, 3072) == "wide"
    assert one(3072, 3072) == "wide"
    assert one(3072, 8192) == "wide"
    assert one(4096, 4096) == "wide"
    # Llama gate/up pair: 256 blocks per 128-row block of M
    assert pair(LLAMA_PAIR) == ("wide" if M <= 128 else "gemm")
    # T5 GeGLU pair: 320 blocks; T5 wo: 64 blocks x 4 K splits per 128-row block
    assert pair(T5_WI_PAIR) == ("wide" if M <= 64 else "gemm")
    assert one(4096, 10240) == ("wide" if M <= 128 else "gemm")


def test_invalid_arguments_raise(pkg):
    for args in ((0, 64, 1024), (2, 0, 1024), (2, 64, 100)):
        with pytest.raises(pkg.SltxError):
            pkg.gemm_route(*args)
    with pytest.raises(pkg.SltxError):
        pkg.gemm_route(2, 64, 1024, group_size=16)


def test_narrow_parity_shapes_run_the_narrow_route(pkg):
    for M, N, K, g in test_gpu_narrow.SHAPES:
        assert pkg.gemm_route(M, N, K, group_size=g) == "narrow", (M, N, K, g)


def test_small_m_parity_shapes_run_the_small_m_route(pkg):
    for M, N, K, g in test_gpu_skinny.SHAPES:
        want = "gemm" if K == 14336 else "small_m"
        assert pkg.gemm_route(M, N, K, group_size=g) == want, (M, N, K, g)
    for M, N, K, g in test_gpu_skinny.PAIR_SHAPES:
        assert pkg.gemm_route(M, N, K, group_size=g, gated=True) == "small_m", (M, N, K, g)


def test_mid_parity_shapes_run_the_mid_route(pkg):
    for M, N, K, g in test_gpu_mid.SHAPES:
        assert pkg.gemm_route(M, N, K, group_size=g) == "mid", (M, N, K, g)
