"""CPU restatement of the fused residual add + LayerNorm / RMSNorm + modulate pass (oracle; test infrastructure only).

Follows redline/run_ln.py (the reference's own model of kernels/glue/ln_mod.cc):
  ln_params  (:38-40)  P = concat([g, sc], axis 1) rounded to bf16; row 0 = real t, row 1 = t = 0
  rows_param (:82-86)  per-row parameters: rows of the first S 128-row M-tiles (row < split_row) take row 1
  ln_ref     (:65-71)  x' = bf(x + bf(g) * br) in float32; y = (x' - mu) / sqrt(var + 1e-6) * bf(sc), with mu and
                       var = mean(x'^2) - mu^2 in float64
and its RMSNorm copy in redline/vlm_run.py:
  rms_params (:62-65)  rows [g = 1 | w]
  rms_ref    (:68-70)  x' = bf(x + br); y = x' / sqrt(mean(x'^2) + 1e-6) * w
Here both take g and sc from the (2, 2D) parameter buffer, as the kernels do. The GPU stores y as bfp16 blocks of 8
along the row; ``ln_mod_ref`` returns the float64 y, and ``quantize_rows`` of it is the packed A the oracle expects.
"""

import numpy as np

from . import bfp16 as F

EPS = 1e-6


def ln_params(g, sc):
    """g, sc: (2, D) rows [real t, t = 0] -> (2, 2D) float32 array of bf16 values (redline/run_ln.py:38-40)."""
    return F.bf16_round(np.concatenate([np.asarray(g, np.float32), np.asarray(sc, np.float32)], 1))


def rms_params(w, g=1.0):
    """RMSNorm parameters: both rows [g | w] (redline/vlm_run.py:62-65)."""
    D = len(w)
    row = np.concatenate([np.full(D, g, np.float32), np.asarray(w, np.float32)])
    return F.bf16_round(np.stack([row, row]))


def rows_param(v, M, split_row):
    """Per-row parameter (M, D) from 2 rows: rows < split_row use row 1, the rest row 0 (redline/run_ln.py:82-86,
    there with split_row = S * 128)."""
    v = np.asarray(v)
    out = np.repeat(v[0:1], M, 0)
    out[:split_row] = v[1]
    return out


def residual(x, br, g):
    """x' = bf16(x + g * br) in float32 (the product of a bf16 and a bfp16 value is exact in float32, so this is one
    rounding to float32 and one to bf16, as an fma followed by RNE)."""
    x = np.asarray(x, np.float32)
    return F.bf16_round(x + np.asarray(g, np.float32) * np.asarray(br, np.float32))


def ln_mod_ref(x, br, params, split_row=0, norm="layer"):
    """x (M, D) bf16 values, br (M, D) exact branch values (or None), params (2, 2D) -> (x' float32, y float64)."""
    x = np.asarray(x, np.float32)
    M, D = x.shape
    params = np.asarray(params, np.float32)
    g = rows_param(params[:, :D], M, split_row)
    sc = rows_param(params[:, D:], M, split_row).astype(np.float64)
    xp = residual(x, np.zeros_like(x) if br is None else br, g)
    x64 = xp.astype(np.float64)
    if norm == "layer":
        mu = x64.mean(1, keepdims=True)
        var = (x64 * x64).mean(1, keepdims=True) - mu * mu
        y = (x64 - mu) / np.sqrt(var + EPS) * sc
    elif norm == "rms":
        y = x64 / np.sqrt((x64 * x64).mean(1, keepdims=True) + EPS) * sc
    else:
        raise ValueError(norm)
    return xp, y
