"""CPU restatement of the QKV post pass: the QKV GEMM's output -> attention Q / K / V tiles (oracle; test
infrastructure only).

Follows the reference's host model and helpers:
  rope      redline/run_glue.py:27-32   complex RoPE on adjacent dim pairs (2i, 2i+1) with cos/sin[:, i]
  rms_rope  redline/run_glue.py:35-37   RMSNorm over the 128 dims (eps 1e-6) * w, then RoPE
  positions redline/run_qkv.py:37-49    rotary row per GEMM row (-1 = pad row)
  qkv_tables redline/run_qkv.py:52-64   the NPU kernel's per-half-tile table (cos/sin per input 8x8 block, then
                                        w_q * log2(e)/sqrt(128) and w_k)
  checks    redline/run_qkv.py:124-136  Q = rms_rope(q cols, w_q * log2(e)/sqrt(128)), K = rms_rope(k cols, w_k),
                                        V = v cols, per head of 128 dims
and the tile formats of kernels/glue/qkv_post.cc:1-16 as unpack_head reads them (redline/run_qkv.py:85-91):
  Q tile (head h, 64 tokens t)  to_bfp16(a_layout(Q[t rows], 64, 128))      blocks = 8 dims of one token
  K tile                        to_bfp16(b_layout(K[t rows].T, 128, 64))    blocks = 8 dims of one key
  V tile                        to_bfp16(b_layout(V[t rows], 64, 128))      blocks = 8 keys of one dim
"""

import numpy as np

from . import bfp16 as F

HEAD_DIM = 128
TILE_TOKENS = 64
C_LOG2 = np.log2(np.e) / np.sqrt(128)  # the attention kernel's score scale, folded into w_q (run_qkv.py:27)
PREFIX = 4128

# per input 8x8 block blk = (sbr*8 + sbc)*4 + kk of a half-tile: its 8 token rows and 4 rotary pairs
# (redline/run_qkv.py:31-34)
_BLK = np.arange(128)
ROWS = (_BLK // 32)[:, None] * 16 + ((_BLK % 4) // 2)[:, None] * 8 + np.arange(8)[None, :]
PAIRS = ((_BLK // 4) % 8)[:, None] * 8 + ((_BLK % 4) % 2)[:, None] * 4 + np.arange(4)[None, :]


def rope(y, cos, sin):
    """Complex RoPE on adjacent dim pairs: y (n, 128), cos/sin (n, 64) (redline/run_glue.py:27-32)."""
    a, b = y[:, 0::2], y[:, 1::2]
    out = np.empty_like(y)
    out[:, 0::2], out[:, 1::2] = a * cos - b * sin, a * sin + b * cos
    return out


def rms_rope(x, w, cos, sin):
    """RMSNorm over the last dim (eps 1e-6) * w, then RoPE (redline/run_glue.py:35-37)."""
    return rope(x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6) * w, cos, sin)


def positions(M, P=None):
    """Rotary row per GEMM row, -1 = pad (redline/run_qkv.py:37-49)."""
    P = PREFIX if P is None else P
    if M == 4096:
        return P + np.arange(4096)
    if M in (8704, 4608):
        row0 = 4224 if M == 8704 else 512
        pos = np.full(M, -1)
        pos[:P] = np.arange(P)
        pos[row0:row0 + 4096] = P + np.arange(4096)
        return pos
    raise ValueError(M)


def qkv_tables(cos, sin, wqc, wk):
    """cos/sin (M, 64) and w_q * log2(e)/sqrt(128), w_k (128 each) -> the (M/64, 8448) table of bf16 values
    (redline/run_qkv.py:52-64): per half-tile, for each input block 32 cos (lane r*4 + p) then 32 sin, then wqc, wk."""
    T = cos.shape[0] // 64
    c = np.asarray(cos, np.float32).reshape(T, 64, 64)[:, ROWS[:, :, None], PAIRS[:, None, :]].reshape(T, 128, 32)
    s = np.asarray(sin, np.float32).reshape(T, 64, 64)[:, ROWS[:, :, None], PAIRS[:, None, :]].reshape(T, 128, 32)
    tab = np.empty((T, 128 * 64 + 256), np.float32)
    tab[:, :128 * 64] = np.concatenate([c, s], -1).reshape(T, -1)
    tab[:, 128 * 64:128 * 64 + 128] = wqc
    tab[:, 128 * 64 + 128:] = wk
    return F.bf16_round(tab)


def qkv_table_loop(cos, sin, wqc, wk, t0):
    """One half-tile's table by the scalar loop of redline/run_glue.py:56-63 (qkvpost1_raw.table): an independent
    statement of the same block -> (rows, pairs) map."""
    tab = np.empty((128, 64), np.float32)
    for blk in range(128):
        sbr, sbc, kk = blk // 32, (blk // 4) % 8, blk % 4
        rows = t0 + sbr * 16 + (kk // 2) * 8 + np.arange(8)
        pairs = sbc * 8 + (kk % 2) * 4 + np.arange(4)
        tab[blk, :32] = cos[np.ix_(rows, pairs)].reshape(-1)
        tab[blk, 32:] = sin[np.ix_(rows, pairs)].reshape(-1)
    return F.bf16_round(np.concatenate([tab.reshape(-1), wqc, wk]))


def qkv_post_ref(C, cos, sin, wqc, wk, heads, kv_heads=None):
    """C (M, (heads + 2 kv_heads) * 128) float values, columns [q heads | k kv_heads | v kv_heads] (kv_heads None:
    = heads; fewer for the text encoder's grouped-query attention, kernels/vlm/qkv_gqa_design.py:1-10); cos/sin
    (M, 64); wqc, wk (128). -> (Q (heads, M, 128), K, V (kv_heads, M, 128)) float64, before quantization."""
    C = np.asarray(C, np.float64)
    cos, sin = np.asarray(cos, np.float64), np.asarray(sin, np.float64)
    wqc, wk = np.asarray(wqc, np.float64), np.asarray(wk, np.float64)
    hkv = heads if kv_heads is None else kv_heads
    hd = HEAD_DIM
    dq, dk = heads * hd, hkv * hd
    Q = np.stack([rms_rope(C[:, h * hd:(h + 1) * hd], wqc, cos, sin) for h in range(heads)])
    K = np.stack([rms_rope(C[:, dq + h * hd:dq + (h + 1) * hd], wk, cos, sin) for h in range(hkv)])
    V = np.stack([C[:, dq + dk + h * hd:dq + dk + (h + 1) * hd] for h in range(hkv)])
    return Q, K, V


def quantize_qkv(Q, K, V):
    """The bfp16 values the tiles hold, as (heads, M, 128) float32: Q and K in blocks of 8 dims, V in blocks of 8
    tokens of one dim."""
    Qq = F.quantize_rows(Q.astype(np.float32).reshape(-1, HEAD_DIM)).reshape(Q.shape)
    Kq = F.quantize_rows(K.astype(np.float32).reshape(-1, HEAD_DIM)).reshape(K.shape)
    Vt = np.ascontiguousarray(V.astype(np.float32).transpose(0, 2, 1))  # (heads, 128, M): blocks along tokens
    Vq = F.quantize_rows(Vt.reshape(-1, Vt.shape[-1])).reshape(Vt.shape).transpose(0, 2, 1)
    return Qq, Kq, np.ascontiguousarray(Vq)


def tiles(Q, K, V):
    """(heads, M, 128) values before quantization (K, V: kv heads) -> the byte tiles q (heads, T, 9216), kv (kv heads,
    T, 2, 9216), each tile encoded once from its float32 values (encoding already-quantized values again is not the
    identity in the -128 corner)."""
    Q, K, V = (np.asarray(a, np.float32) for a in (Q, K, V))
    H, M, _ = Q.shape
    HKV = K.shape[0]
    T = M // TILE_TOKENS
    q = np.empty((H, T, 9216), np.uint8)
    kv = np.empty((HKV, T, 2, 9216), np.uint8)
    for t in range(T):
        r = slice(t * TILE_TOKENS, (t + 1) * TILE_TOKENS)
        for h in range(H):
            q[h, t] = F.to_bfp16(F.a_layout(Q[h, r], 64, 128))
        for h in range(HKV):
            kv[h, t, 0] = F.to_bfp16(F.b_layout(np.ascontiguousarray(K[h, r].T), 128, 64))
            kv[h, t, 1] = F.to_bfp16(F.b_layout(V[h, r], 64, 128))
    return q, kv


def unpack_head(q, kv, h):
    """Q, K, V of head h, each (T*64, 128) float32 (redline/run_qkv.py:85-91)."""
    T = q.shape[1]
    Q = F.a_unlayout(F.from_bfp16(q[h].ravel()), T * 64, 128, 64, 128)
    K = F.b_unlayout(F.from_bfp16(kv[h, :, 0].ravel()), 128, T * 64, 128, 64).T
    V = F.b_unlayout(F.from_bfp16(kv[h, :, 1].ravel()), T * 64, 128, 64, 128)
    return Q, K, V
