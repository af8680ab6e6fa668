"""Stream layouts of the oracle, pinned by their inverse pairs and by the reference's scalar index formulas
(redline/npu_layouts.py:11-59, redline/forward.py:64-80)."""

import numpy as np
import pytest

from oracle import bfp16 as F


def test_b_layout_inverse_and_scalar_formula():
    K, N = 128, 256
    B = np.arange(K * N, dtype=np.float32).reshape(K, N)
    s = F.b_layout(B)
    np.testing.assert_array_equal(F.b_unlayout(s, K, N), B)
    rng = np.random.default_rng(0)
    for r, c in zip(rng.integers(0, K, 300), rng.integers(0, N, 300)):
        assert s[F.b_index(int(r), int(c), K)] == B[r, c]


def test_b_unlayout_fast_equals_position_map():
    K, N = 192, 384
    s = np.arange(K * N, dtype=np.float64)
    np.testing.assert_array_equal(F.b_unlayout_fast(s, K, N), F.b_unlayout(s, K, N))


def test_b_layout_tile_is_contiguous():
    """A (64 K x 128 N) tile is 1024 consecutive blocks; block l of a 16-column group at fixed K half holds column
    l % 16 and K rows 8 (l / 16) .. +7 (the MFMA operand the GEMM reads per lane)."""
    K, N = 192, 256
    B = np.arange(K * N, dtype=np.float32).reshape(K, N)
    s = F.b_layout(B).reshape(-1, 8)
    KT = K // 64
    for nt, kt, sbc, h in ((1, 2, 3, 1), (0, 0, 0, 0), (1, 1, 7, 0)):
        tile = (nt * KT + kt) * 1024
        for lane in (0, 5, 17, 63):
            blk = s[tile + sbc * 128 + 64 * h + lane]
            col = nt * 128 + sbc * 16 + lane % 16
            k0 = kt * 64 + 32 * h + 8 * (lane // 16)
            np.testing.assert_array_equal(blk, B[k0:k0 + 8, col])


def test_a_layout_inverse_and_scalar_formula():
    M, K = 256, 128
    A = np.arange(M * K, dtype=np.float32).reshape(M, K)
    s = F.a_layout(A)
    np.testing.assert_array_equal(F.a_unlayout(s, M, K), A)
    rng = np.random.default_rng(1)
    for r, c in zip(rng.integers(0, M, 300), rng.integers(0, K, 300)):
        assert s[F.a_index(int(r), int(c), K)] == A[r, c]


def test_c_atb_inverse_and_scalar_formula():
    M, N = 1024, 2048
    Cm = np.arange(M * N, dtype=np.float64).reshape(M, N)
    s = F.c_layout_atb(Cm)
    np.testing.assert_array_equal(F.c_unlayout_atb(s, M, N), Cm)
    rng = np.random.default_rng(2)
    for r, c in zip(rng.integers(0, M, 300), rng.integers(0, N, 300)):
        assert s[F.atb_index(int(r), int(c), N)] == Cm[r, c]


def test_c_atb_small_tiles_and_upstream_order_differ():
    """rows=cols=1 with 64x128 tiles (redline/run_glue.py:48-49) is a valid instance; upstream's c_unlayout order
    (redline/npu_layouts.py:25-28) is a different permutation (the reference's note at :32)."""
    M, N = 128, 256
    Cm = np.arange(M * N, dtype=np.float64).reshape(M, N)
    s = F.c_layout_atb(Cm, 64, 128, rows=1, cols=1)
    np.testing.assert_array_equal(F.c_unlayout_atb(s, M, N, 64, 128, rows=1, cols=1), Cm)
    big = np.arange(1024 * 2048, dtype=np.float64).reshape(1024, 2048)
    assert not np.array_equal(F.c_unlayout(F.c_layout_atb(big), 1024, 2048, 128, 128), big)


@pytest.mark.parametrize("K,F_", [(64, 128), (128, 192)])
def test_interleave_up(K, F_):
    rng = np.random.default_rng(3)
    wg = rng.standard_normal((F_, K)).astype(np.float32)
    wp = rng.standard_normal((F_, K)).astype(np.float32)
    B = F.interleave_up(wg, wp)
    for j in range(2 * F_):
        t, h, u = j // 128, (j % 128) // 64, j % 64
        src = wg if h == 0 else wp
        np.testing.assert_array_equal(B[:, j], src[64 * t + u])


def test_pack_b_is_blockwise_encode_of_layout():
    rng = np.random.default_rng(4)
    K, N = 128, 256
    B = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    packed = F.pack_b(B)
    assert packed.size == K * N // 8 * 9
    np.testing.assert_array_equal(F.decode_b(packed, K, N), F.b_unlayout(F.from_bfp16(F.to_bfp16(F.b_layout(B))),
                                                                          K, N))
    # blocks run along K: quantizing W (= B.T) along its rows gives the same values
    np.testing.assert_array_equal(F.decode_b(packed, K, N), F.quantize_rows(B.T).T)
