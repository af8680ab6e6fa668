"""CPU restatement of attention over the QKV post pass's output (oracle; test infrastructure only).

Follows redline/run_attn.py:131-150 (the reference's own float64 check of the attention artifacts) with the kernel's
conventions from kernels/attn/attn_bfp.cc:1-12: Q arrives pre-multiplied by log2(e)/sqrt(128), so the scores are in
log2 units and the softmax is 2^(s - max) / sum; keys j >= nkv (zero padding) and, per query i, keys j > lim[i] are
not visible.
"""

import numpy as np

HEAD_DIM = 128
C_LOG2 = np.log2(np.e) / np.sqrt(HEAD_DIM)


def attention_ref(q, k, v, nkv=None, lim=None):
    """q (H, NQ, 128) with the score scale folded in, k and v (H, NK, 128) -> O (H, NQ, 128) float64."""
    q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
    nk = k.shape[1]
    nkv = nk if nkv is None else nkv
    s = np.einsum("hqd,hkd->hqk", q, k)
    keys = np.arange(nk)[None, None, :]
    visible = keys < nkv
    if lim is not None:
        visible = visible & (keys <= np.asarray(lim)[None, :, None])
    s = np.where(visible, s, -np.inf)
    mx = s.max(2, keepdims=True)
    w = np.where(visible, np.exp2(s - np.where(np.isfinite(mx), mx, 0.0)), 0.0)
    den = w.sum(2, keepdims=True)
    return np.einsum("hqk,hkd->hqd", w, v) / np.where(den > 0, den, 1.0)
