"""The oracle's QKV post pass (oracle/qkv.py) and the host-side index maps of the run_qkv mirror, pinned without the
reference: RoPE closed forms (angle 0, a quarter turn, norm preservation), RMSNorm against torch's float64 rms_norm,
the vectorised table against the reference's own scalar loop (redline/run_glue.py:56-63), tile encodings against the
layouts' inverse maps, and the torch block-index maps against the oracle's position maps."""

import numpy as np
import pytest
import torch

from oracle import bfp16 as F
from oracle import qkv as QK
from rlbfp import layouts as LY
from rlbfp import run_qkv as RQ


def test_rope_closed_forms():
    rng = np.random.default_rng(0)
    y = rng.standard_normal((5, 128))
    ones, zeros = np.ones((5, 64)), np.zeros((5, 64))
    np.testing.assert_array_equal(QK.rope(y, ones, zeros), y)
    q = QK.rope(y, zeros, ones)  # a quarter turn: (a, b) -> (-b, a)
    np.testing.assert_array_equal(q[:, 0::2], -y[:, 1::2])
    np.testing.assert_array_equal(q[:, 1::2], y[:, 0::2])
    ang = rng.uniform(-np.pi, np.pi, (5, 64))
    r = QK.rope(y, np.cos(ang), np.sin(ang))
    np.testing.assert_allclose(r[:, 0::2] ** 2 + r[:, 1::2] ** 2, y[:, 0::2] ** 2 + y[:, 1::2] ** 2, rtol=1e-12)
    # the rotation composes: angle a then angle b = angle a + b
    b = rng.uniform(-np.pi, np.pi, (5, 64))
    np.testing.assert_allclose(QK.rope(r, np.cos(b), np.sin(b)), QK.rope(y, np.cos(ang + b), np.sin(ang + b)),
                               atol=1e-12)


def test_rms_rope_matches_torch():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((7, 128)) * 3
    w = 1 + 0.1 * rng.standard_normal(128)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x), (128,), eps=1e-6).numpy() * w
    ones, zeros = np.ones((7, 64)), np.zeros((7, 64))
    np.testing.assert_allclose(QK.rms_rope(x, w, ones, zeros), ref, rtol=1e-12)


def test_tables_match_scalar_loop():
    rng = np.random.default_rng(2)
    M = 192
    ang = rng.uniform(-np.pi, np.pi, (M, 64))
    cos, sin = F.bf16_round(np.cos(ang).astype(np.float32)), F.bf16_round(np.sin(ang).astype(np.float32))
    wqc = F.bf16_round((1 + 0.1 * rng.standard_normal(128)) * QK.C_LOG2)
    wk = F.bf16_round(1 + 0.1 * rng.standard_normal(128))
    tab = QK.qkv_tables(cos, sin, wqc, wk)
    for t in range(M // 64):
        np.testing.assert_array_equal(tab[t], QK.qkv_table_loop(cos, sin, wqc, wk, 64 * t))
    # the mirror's torch version (CPU tensors) builds the same buffer, and its inverse recovers the rows
    tt = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16)
    tab_t = RQ.qkv_tables(tt(cos), tt(sin), tt(wqc), tt(wk))
    np.testing.assert_array_equal(tab_t.float().numpy(), tab)
    c, s, wq2, wk2 = RQ.tables_rows(tab_t)
    for got, want in ((c, cos), (s, sin), (wq2, wqc), (wk2, wk)):
        np.testing.assert_array_equal(got.float().numpy(), want)


def test_tiles_round_trip_through_unpack_head():
    rng = np.random.default_rng(3)
    M, H = 128, 2
    C = F.bf16_round(rng.standard_normal((M, 3 * H * 128)).astype(np.float32))
    ang = rng.uniform(-np.pi, np.pi, (M, 64))
    Q, K, V = QK.qkv_post_ref(C, np.cos(ang), np.sin(ang), np.ones(128), np.ones(128), H)
    q, kv = QK.tiles(Q, K, V)
    Qq, Kq, Vq = QK.quantize_qkv(Q, K, V)
    for h in range(H):
        a, b, c = QK.unpack_head(q, kv, h)
        np.testing.assert_array_equal(a, Qq[h])
        np.testing.assert_array_equal(b, Kq[h])
        np.testing.assert_array_equal(c, Vq[h])
    np.testing.assert_array_equal(Vq, F.bf16_round(Vq))  # V of bf16 inputs quantizes to values exact in bf16


@pytest.mark.parametrize("M", [4096, 8704, 4608])
def test_positions(M):
    pos = QK.positions(M)
    np.testing.assert_array_equal(pos, RQ.positions(M))
    assert len(pos) == M
    valid = pos[pos >= 0]
    assert (valid[-4096:] == QK.PREFIX + np.arange(4096)).all()  # the target's 4096 tokens come last in position
    if M != 4096:
        row0 = 4224 if M == 8704 else 512
        assert (pos[:QK.PREFIX] == np.arange(QK.PREFIX)).all() if M == 8704 else True
        assert (pos[row0:row0 + 4096] == QK.PREFIX + np.arange(4096)).all()
    with pytest.raises(ValueError):
        QK.positions(1000)


@pytest.mark.parametrize("R,C,m,k", [(64, 128, 64, 128), (256, 192, 128, 64)])
def test_a_block_index(R, C, m, k):
    rr, cc = np.meshgrid(np.arange(R), np.arange(C // 8), indexing="ij")
    np.testing.assert_array_equal(LY.a_block_index(R, C, m, k, "cpu").numpy(), (F.a_pos(rr, 8 * cc, R, C, m, k) // 8)
                                  .reshape(-1))


@pytest.mark.parametrize("K,N,k,n", [(128, 64, 128, 64), (64, 128, 64, 128), (128, 256, 64, 128)])
def test_b_block_index(K, N, k, n):
    kb, cc = np.meshgrid(np.arange(K // 8), np.arange(N), indexing="ij")
    np.testing.assert_array_equal(LY.b_block_index(K, N, k, n, "cpu").numpy(), (F.b_pos(8 * kb, cc, K, N, k, n) // 8)
                                  .reshape(-1))
