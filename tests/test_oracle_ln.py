"""The oracle's residual + LayerNorm/RMSNorm + modulate pass (oracle/ln.py), pinned without the reference:
torch's float64 layer_norm / rms_norm (library routines), hand-derived answers for the bf16 rounding of x' and for a
row with a closed-form mean and variance, and the row split of the parameters."""

import numpy as np
import pytest
import torch

from oracle import bfp16 as F
from oracle import ln as LN


def rand_case(rng, M, D):
    x = F.bf16_round((rng.standard_normal((M, D)) * 3).astype(np.float32))
    x[:, rng.integers(0, D, 4)] *= 40  # outlier channels, as redline/run_ln.py:93 draws them
    x = F.bf16_round(x)
    br = F.quantize_rows(rng.standard_normal((M, D)).astype(np.float32))
    g = np.tanh(rng.standard_normal((2, D))).astype(np.float32)
    sc = (1 + 0.3 * rng.standard_normal((2, D))).astype(np.float32)
    return x, br, LN.ln_params(g, sc)


def test_layer_norm_matches_torch():
    rng = np.random.default_rng(0)
    M, D, split = 300, 256, 128
    x, br, p = rand_case(rng, M, D)
    xp, y = LN.ln_mod_ref(x, br, p, split_row=split)
    g = LN.rows_param(p[:, :D], M, split)
    sc = LN.rows_param(p[:, D:], M, split)
    xt = torch.from_numpy(xp.astype(np.float64))
    ref = torch.nn.functional.layer_norm(xt, (D,), eps=1e-6).numpy() * sc
    np.testing.assert_allclose(y, ref, rtol=1e-9, atol=1e-9)
    # x' itself: float32 add of the exact product, then RNE to bf16, checked through torch's bf16 cast
    xr = (torch.from_numpy(x) + torch.from_numpy(g) * torch.from_numpy(br)).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(xp, xr)


def test_rms_norm_matches_torch():
    rng = np.random.default_rng(1)
    M, D = 64, 512
    x, br, _ = rand_case(rng, M, D)
    w = (1 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    p = LN.rms_params(w)
    xp, y = LN.ln_mod_ref(x, br, p, norm="rms")
    ref = torch.nn.functional.rms_norm(torch.from_numpy(xp.astype(np.float64)), (D,), eps=1e-6).numpy()
    np.testing.assert_allclose(y, ref * p[0, D:], rtol=1e-9, atol=1e-9)
    # redline/vlm_run.py:68-70 form: g = 1, x' = bf(x + br)
    np.testing.assert_array_equal(xp, F.bf16_round(x + br))


def test_closed_form_row():
    """x = 0..63, no branch, sc = 1: mean 31.5, variance (64^2 - 1) / 12."""
    D = 64
    x = np.arange(D, dtype=np.float32)[None, :]
    p = LN.ln_params(np.zeros((2, D)), np.ones((2, D)))
    xp, y = LN.ln_mod_ref(x, None, p)
    np.testing.assert_array_equal(xp, x)
    expect = (np.arange(D) - 31.5) / np.sqrt((D * D - 1) / 12 + 1e-6)
    np.testing.assert_allclose(y[0], expect, rtol=1e-12)
    _, yr = LN.ln_mod_ref(x, None, p, norm="rms")
    np.testing.assert_allclose(yr[0], np.arange(D) / np.sqrt(np.mean(np.arange(D) ** 2.0) + 1e-6), rtol=1e-12)


@pytest.mark.parametrize("br,expect", [
    (2.0 ** -8, 1.0),                  # 1 + 2^-8 is the tie between 1 and 1 + 2^-7: to even (1.0)
    (3 * 2.0 ** -8, 1.0 + 2.0 ** -6),  # tie between 1 + 2^-7 (odd) and 1 + 2^-6 (even)
    (2.0 ** -8 + 2.0 ** -20, 1.0 + 2.0 ** -7),  # just above the tie
    (-2.0 ** -9, 1.0),                 # 1 - 2^-9 is the tie between 1 - 2^-8 (odd) and 1 (even)
])
def test_residual_rounding(br, expect):
    x = np.array([[1.0]], np.float32)
    assert LN.residual(x, np.array([[br]], np.float32), np.float32(1.0))[0, 0] == np.float32(expect)


def test_rows_param_split():
    v = np.array([[0.0] * 4, [1.0] * 4], np.float32)
    out = LN.rows_param(v, 300, 128)
    assert (out[:128] == 1.0).all() and (out[128:] == 0.0).all()
    assert (LN.rows_param(v, 10, 0) == 0.0).all()
    assert (LN.rows_param(v, 10, 10) == 1.0).all()


def test_layer_norm_invariants():
    """sc = 1: every row of y has mean 0 and mean square var / (var + eps)."""
    rng = np.random.default_rng(2)
    M, D = 16, 1024
    x = F.bf16_round(rng.standard_normal((M, D)).astype(np.float32) * 0.01)
    p = LN.ln_params(np.zeros((2, D)), np.ones((2, D)))
    xp, y = LN.ln_mod_ref(x, None, p)
    var = xp.astype(np.float64).var(1)
    np.testing.assert_allclose(y.mean(1), 0, atol=1e-10)
    np.testing.assert_allclose((y * y).mean(1), var / (var + 1e-6), rtol=1e-9)
