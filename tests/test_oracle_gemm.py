"""The GEMM emulation pinned by a brute-force loop on tiny shapes and by the epilogues' closed forms."""

import numpy as np
import pytest

from oracle import bfp16 as F
from oracle import gemm as G


def brute(Aq, Bq):
    M, K = Aq.shape
    N = Bq.shape[1]
    out = np.zeros((M, N))
    for i in range(M):
        for j in range(N):
            s = 0.0
            for k in range(K):
                s += float(Aq[i, k]) * float(Bq[k, j])
            out[i, j] = s
    return out


def test_gemm_matches_brute_force():
    rng = np.random.default_rng(0)
    M, K, N = 5, 64, 128
    A = G.activations(rng, M, K)
    W = G.linear_weight(rng, N, K)
    Aq, Bq = F.quantize_rows(A), F.decode_b(F.pack_b(W.T), K, N)
    got = G.gemm_ref(Aq, Bq)
    np.testing.assert_array_equal(got, F.bf16_round_f64(brute(Aq, Bq)))


def test_quantized_operands_are_bf16_exact():
    rng = np.random.default_rng(1)
    A = G.activations(rng, 16, 64, outliers=0.05)
    Aq = F.quantize_rows(A)
    np.testing.assert_array_equal(F.bf16_round(Aq), Aq)


def test_swiglu_pairs_columns_64_apart():
    v = np.zeros((1, 256))
    v[0, 3], v[0, 67] = 2.0, 5.0          # gate unit 3, proj unit 3 of tile 0
    v[0, 128 + 10], v[0, 128 + 74] = -1.0, 4.0  # tile 1, unit 10 -> output column 64 + 10
    out = G.swiglu_i128(v)
    assert out.shape == (1, 128)
    assert out[0, 3] == pytest.approx(2.0 / (1 + np.exp(-2.0)) * 5.0)
    assert out[0, 74] == pytest.approx(-1.0 / (1 + np.exp(1.0)) * 4.0)
    assert np.count_nonzero(out) == 2


def test_epilogue_closed_forms():
    acc = np.array([[0.0, 1.0, -2.0, 3.5] * 2], np.float64)
    assert (G.epilogue(acc, act=G.ACT_GELU_TANH)[0, 0]) == 0.0
    g = G.gelu_tanh(np.array([1.7, -1.7]))
    assert g[0] - g[1] == pytest.approx(1.7)            # gelu(x) - gelu(-x) = x
    res = np.full((1, 8), 0.5, np.float32)
    out = G.epilogue(acc, gate=np.zeros(8), residual=res)
    np.testing.assert_array_equal(out, res)              # gate 0 -> residual only
    two = np.stack([np.full(8, 2.0), np.full(8, 3.0)])
    out2 = G.epilogue(np.ones((4, 8)), gate=two, gate_split_row=2)
    np.testing.assert_array_equal(out2[:, 0], [3.0, 3.0, 2.0, 2.0])   # rows < split use gate row 1
    b = np.arange(8, dtype=np.float64)
    np.testing.assert_array_equal(G.epilogue(np.zeros((1, 8)), bias=b)[0], b)


def test_quantize_out_is_blockwise():
    rng = np.random.default_rng(2)
    acc = rng.standard_normal((3, 64)) * 3
    out = G.epilogue(acc, quantize_out=True)
    np.testing.assert_array_equal(out, F.quantize_rows(F.bf16_round_f64(acc)))


def test_gemv_matches_loop():
    rng = np.random.default_rng(3)
    K, N = 64, 128
    x = F.bf16_round(rng.standard_normal((2, K)).astype(np.float32))
    Bq = F.decode_b(F.pack_b(G.linear_weight(rng, N, K).T), K, N)
    got = G.gemv_ref(x, Bq)
    a = F.quantize_rows(G.silu(x).astype(np.float32))     # the activation is quantized like the GEMM's A
    want = F.bf16_round_f64(brute(a, Bq))
    np.testing.assert_array_equal(got, want)
    assert not np.array_equal(got, F.bf16_round_f64(brute(G.silu(x), Bq)))   # and that quantization matters


# ---- silu / gelu_tanh pinned by library routines (torch's and scipy's float64 implementations) --------------------

def _grid():
    """|x| up to 30 (both exponential tails), a dense core, and the SwiGLU gate / GELU input range of the FFN shapes
    (accumulators of K = 3072 products of N(0,1) activations and N(0, 0.02) weights: |v| < ~6)."""
    rng = np.random.default_rng(7)
    return np.concatenate([np.linspace(-30.0, 30.0, 6001), np.linspace(-6.0, 6.0, 4001),
                           rng.standard_normal(4000) * 1.1, [0.0, -0.0, 1e-30, -1e-30, 5e-8]])


def _pinned(f, ref, x):
    """f agrees with the library routine to float64 rounding: 1e-13 absolute plus 1e-13 relative."""
    got = np.asarray(f(x), np.float64)
    return bool(np.all(np.abs(got - ref) <= 1e-13 + 1e-13 * np.abs(ref)))


def _torch_ref(name, x):
    import torch
    t = torch.as_tensor(x, dtype=torch.float64)
    if name == "silu":
        return torch.nn.functional.silu(t).numpy()
    return torch.nn.functional.gelu(t, approximate="tanh").numpy()


def test_silu_matches_library_float64():
    from scipy.special import expit
    x = _grid()
    assert _pinned(G.silu, _torch_ref("silu", x), x)
    assert _pinned(G.silu, x * expit(x), x)


def test_gelu_tanh_matches_library_float64():
    x = _grid()
    assert _pinned(G.gelu_tanh, _torch_ref("gelu_tanh", x), x)


def test_activation_pins_reject_plausible_mistakes():
    """Each mutant (a rounded constant, a sign, the erf form, a missing term) must fail the same check that the
    oracle passes."""
    from scipy.special import erf
    x = _grid()
    g_ref, s_ref = _torch_ref("gelu_tanh", x), _torch_ref("silu", x)

    def gelu_c(c=0.044715, k=np.sqrt(2.0 / np.pi)):
        return lambda v: 0.5 * v * (1.0 + np.tanh(k * (v + c * v ** 3)))

    gelu_mutants = [gelu_c(c=0.0447), gelu_c(k=0.7978), gelu_c(k=np.sqrt(np.pi / 2.0)), gelu_c(c=0.0),
                    lambda v: 0.5 * v * (1.0 + erf(v / np.sqrt(2.0))),
                    lambda v: v / (1.0 + np.exp(-1.702 * v))]
    for m in gelu_mutants:
        assert not _pinned(m, g_ref, x)
    silu_mutants = [lambda v: v / (1.0 + np.exp(v)), lambda v: 1.0 / (1.0 + np.exp(-v)),
                    lambda v: v / (1.0 + np.exp2(-v)), lambda v: v / (1.0 + np.exp(-v.astype(np.float32)))]
    for m in silu_mutants:
        assert not _pinned(m, s_ref, x)
    assert _pinned(gelu_c(), g_ref, x)   # the check itself accepts a faithful restatement
