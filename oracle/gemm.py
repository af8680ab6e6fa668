"""CPU emulation of the bfp16-weight GEMM path (oracle; test infrastructure only).

The contract the HIP path is checked against (redline/vlm_run.py:95-110 is the reference's own GEMM check: a float64
matmul of the dequantized bfp16 operands):

  A_q  = decoded bfp16 of the activations, blocks = 8 consecutive K of a row (to_bfp16 on the row-major rows)
  B_q  = decoded packed weights (b_layout of W.T, redline/pack_weights.py:72-79)
  acc  = A_q @ B_q in float64 (the products are exact; only summation order differs from the GPU's fp32 MFMA)
  out  = bf16( epilogue(acc) ), the epilogue evaluated in float64:
           v = acc (+ bias[n])
           act: none | gelu_tanh (redline/host_glue.py:55, kernels/vlm/gelu_bfp.cc:1-8)
                | swiglu on the [gate 64 | proj 64] per-128-column interleave (redline/pack_weights.py:82-89,
                  redline/run_glue.py:145): out[:, 64t+u] = silu(v[:, 128t+u]) * v[:, 128t+64+u]
           gate/residual: v = residual + gate[n] * v (redline/run_ln.py:65-67 "x' = x + g * branch"; the gate row is
                  row 1 of a 2-row gate for rows < gate_split_row, redline/run_ln.py:82-86)
         then rounded to bf16 (RNE), and optionally re-quantized to bfp16 along rows (quantize_out).

The adaLN modulation GEMV (redline/host_glue.py:26-28,43-44: ``linear(silu(te), W)``) is emulated with the same
decoded weights: y = bf16( Q(act(x)) @ B_q ) with act = silu or identity evaluated on the bf16 input, rounded to
float32 and quantized to bfp16 blocks of 8 along K (Q, the same encoder as the activations of the GEMM), i.e. both
GEMV operands are bfp16 as in the reference's NPU GEMMs. The GPU evaluates silu in float32 with the hardware exp2 and
reciprocal; where that moves a value across a bfp16 rounding boundary the results differ by one quantization step of
one product, far inside the tolerance.
"""

import numpy as np

from . import bfp16 as F

ACT_NONE, ACT_GELU_TANH, ACT_SWIGLU = "none", "gelu_tanh", "swiglu"


def silu(x):
    x = np.asarray(x, dtype=np.float64)
    return x / (1.0 + np.exp(-x))


def gelu_tanh(x):
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def swiglu_i128(v):
    """(M, 2F) with [gate 64 | proj 64] per 128-column tile -> (M, F): silu(gate) * proj, output column 64t+u."""
    M, N2 = v.shape
    assert N2 % 128 == 0
    t = v.reshape(M, N2 // 128, 2, 64)
    return (silu(t[:, :, 0, :]) * t[:, :, 1, :]).reshape(M, N2 // 2)


def epilogue(acc, act=ACT_NONE, bias=None, gate=None, gate_split_row=0, residual=None, quantize_out=False):
    """float64 accumulator (M, N) -> the bf16-rounded float32 output of the fused epilogue."""
    v = np.asarray(acc, dtype=np.float64)
    if bias is not None:
        v = v + np.asarray(bias, dtype=np.float64)[None, :]
    if act == ACT_GELU_TANH:
        v = gelu_tanh(v)
    elif act == ACT_SWIGLU:
        v = swiglu_i128(v)
    elif act != ACT_NONE:
        raise ValueError(act)
    if residual is not None or gate is not None:
        M, Nout = v.shape
        g = np.ones((2, Nout)) if gate is None else np.asarray(gate, dtype=np.float64).reshape(-1, Nout)
        rows = np.repeat(g[0:1], M, axis=0)
        if g.shape[0] > 1 and gate_split_row > 0:
            rows[:gate_split_row] = g[1]
        v = rows * v
        if residual is not None:
            v = np.asarray(residual, dtype=np.float64) + v
    out = F.bf16_round_f64(v)
    if quantize_out:
        out = F.quantize_rows(out)
    return out


def gemm_ref(Aq, Bq, **ep):
    """Decoded A (M, K) and decoded B (K, N), both float32 exact values -> bf16-rounded float32 output."""
    acc = np.asarray(Aq, dtype=np.float64) @ np.asarray(Bq, dtype=np.float64)
    return epilogue(acc, **ep)


def gemm_bf16_acts(A_bf16, packed_b, K, N, **ep):
    """bf16 activations (float32 values), packed weights -> output: quantizes A along K, decodes B, multiplies."""
    return gemm_ref(F.quantize_rows(A_bf16), F.decode_b(packed_b, K, N), **ep)


def gemv_ref(x, Bq, act="silu"):
    """x (M, K) bf16 values as float32, decoded weights (K, N) -> bf16-rounded (M, N): act(x) is evaluated in float64,
    rounded to float32 and quantized to bfp16 blocks of 8 along K (the GEMM's activation encoding), then multiplied
    with the decoded weights in float64."""
    v = np.asarray(x, dtype=np.float64)
    if act == "silu":
        v = silu(v)
    elif act != ACT_NONE:
        raise ValueError(act)
    a = F.quantize_rows(v.astype(np.float32))
    return F.bf16_round_f64(a.astype(np.float64) @ np.asarray(Bq, dtype=np.float64))


def rel_err(got, ref):
    """The reference's error metric: max |got - ref| / max |ref| (redline/run_glue.py:158-159,
    redline/vlm_run.py:34-36)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-300))


def corr(got, ref):
    return float(np.corrcoef(np.asarray(got, np.float64).ravel(), np.asarray(ref, np.float64).ravel())[0, 1])


# ---------------------------------------------------------------------------------------------------------------
# synthetic inputs (seeded like the reference's checks: np.random.default_rng(seed), redline/run_glue.py:141)
# ---------------------------------------------------------------------------------------------------------------

def activations(rng, M, K, outliers=0.0, rms_rows=False):
    """bf16 activations ~N(0,1) as float32 values; optionally round(outliers*K) channels x20 (chosen without
    replacement) or rows normalised to unit RMS before the bf16 cast."""
    a = rng.standard_normal((M, K)).astype(np.float32)
    if outliers:
        cols = rng.choice(K, int(round(outliers * K)), replace=False)
        a[:, cols] *= 20.0
    if rms_rows:
        a = (a / np.sqrt((a.astype(np.float64) ** 2).mean(1, keepdims=True))).astype(np.float32)
    return F.bf16_round(a)


def linear_weight(rng, N, K, std=0.02):
    """A Linear weight W (N, K) ~ N(0, std) in float32; the GEMM's B is W.T."""
    return (rng.standard_normal((N, K)) * std).astype(np.float32)
