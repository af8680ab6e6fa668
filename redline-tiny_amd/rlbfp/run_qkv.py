"""The host helpers of redline/run_qkv.py over the HIP pass rl_qkv_post (device tensors in and out).

``positions`` / ``qkv_tables`` / ``qkv32_npu`` / ``unpack_head`` keep the reference's names and argument meanings
(redline/run_qkv.py:37-91): the input is the QKV GEMM's C stream (bfp16, c_layout_atb(., 128, 128) of
M x 3 * hidden), the rotary cos/sin and the q/k norm weights travel in the NPU kernel's table format, and the outputs
are the attention kernel's tiles, Q (heads, T, 9216 bytes) and KV (heads, T, 2, 9216 bytes), T = M / 64. On the HIP
path the pass reads cos/sin as (M, 64) rows, so ``qkv32_npu`` unpacks the table first; ``ops.qkv_post`` is the
native entry point (bf16 C from the GEMM, bf16 cos/sin rows, tiles and/or head-major bf16 Q/K/V out).
"""

import numpy as np
import torch

from . import layouts, ops

H, D, PREFIX = 32, 128, 4128  # heads, head dim and image prefix of the reference DiT (redline/run_qkv.py:24)
HALF = 64 * 128 // 8          # blocks per tile
TAB = 128 * 64 + 2 * 128      # one table: cos/sin of 128 input blocks, then w_q, w_k (bf16)
C_LOG2 = float(np.log2(np.e) / np.sqrt(128))

# per input 8x8 block blk = (sbr*8 + sbc)*4 + kk of a half-tile: its 8 token rows and 4 rotary pairs
# (redline/run_qkv.py:31-34)
_BLK = np.arange(128)
_ROWS = (_BLK // 32)[:, None] * 16 + ((_BLK % 4) // 2)[:, None] * 8 + np.arange(8)[None, :]
_PAIRS = ((_BLK // 4) % 8)[:, None] * 8 + ((_BLK % 4) % 2)[:, None] * 4 + np.arange(4)[None, :]


def positions(M, P=None):
    """Rotary row (token position) per GEMM row, -1 = pad. M=4096: cached step (target only); M=8704: step 1
    [prefix P (default 4128) | pad | target 4096 from row 4224 | pad 384]; M=4608: text-to-image step 1
    (redline/run_qkv.py:37-49)."""
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


def _gather_index(T, device):
    rows = torch.as_tensor(_ROWS, device=device)[:, :, None].expand(128, 8, 4)
    pairs = torch.as_tensor(_PAIRS, device=device)[:, None, :].expand(128, 8, 4)
    return (rows * 64 + pairs).reshape(-1)  # (128 * 32,) position in a 64 x 64 tile, lane order blk, r, p


def qkv_tables(cos, sin, wqc, wk):
    """cos/sin (M, 64) per GEMM row and w_q * log2(e)/sqrt(128), w_k (128 each) -> the TABS buffer (M/64, 8448) bf16
    (redline/run_qkv.py:52-64)."""
    T = cos.shape[0] // 64
    g = _gather_index(T, cos.device)
    c = cos.float().reshape(T, 64 * 64)[:, g].reshape(T, 128, 32)
    s = sin.float().reshape(T, 64 * 64)[:, g].reshape(T, 128, 32)
    tab = torch.empty((T, TAB), dtype=torch.float32, device=cos.device)
    tab[:, :128 * 64] = torch.cat([c, s], -1).reshape(T, -1)
    tab[:, 128 * 64:128 * 64 + 128] = wqc.float()
    tab[:, 128 * 64 + 128:] = wk.float()
    return tab.to(torch.bfloat16)


def tables_rows(tabs):
    """The inverse of qkv_tables: TABS (T, 8448) -> (cos (T*64, 64), sin (T*64, 64), wqc, wk), bf16."""
    T = tabs.shape[0]
    g = _gather_index(T, tabs.device)
    t3 = tabs[:, :128 * 64].reshape(T, 128, 64)
    cos = torch.empty((T, 64 * 64), dtype=tabs.dtype, device=tabs.device)
    sin = torch.empty_like(cos)
    cos[:, g] = t3[:, :, :32].reshape(T, -1)
    sin[:, g] = t3[:, :, 32:].reshape(T, -1)
    return (cos.reshape(T * 64, 64), sin.reshape(T * 64, 64), tabs[0, 128 * 64:128 * 64 + 128].contiguous(),
            tabs[0, 128 * 64 + 128:].contiguous())


def qkv32_npu(art, cin_pack, tabs, M, iters=0):
    """cin_pack: the QKV GEMM's C stream (bfp16 bytes, c_layout_atb 128x128 of M x 3 * hidden). Returns (Q, KV, ms):
    Q (heads, T, 9216) and KV (heads, T, 2, 9216) uint8 as the attention kernel takes them, and the median device ms
    over `iters` extra runs (None if 0) (redline/run_qkv.py:67-82). `art` is accepted for the reference's signature."""
    n_cols = cin_pack.numel() // 9 * 8 // M
    heads = n_cols // (3 * D)
    C = ops.dequantize(cin_pack.reshape(-1), M, n_cols, order="c_atb", dtype=torch.bfloat16)
    cos, sin, wqc, wk = tables_rows(tabs.reshape(M // 64, TAB))

    def run():
        return ops.qkv_post(C, cos.contiguous(), sin.contiguous(), wqc, wk, heads)[:2]

    q, kv = run()
    ms = None
    if iters:
        ts = []
        for _ in range(iters):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            run()
            e1.record()
            e1.synchronize()
            ts.append(e0.elapsed_time(e1))
        ms = float(np.median(ts))
    torch.cuda.current_stream().synchronize()
    return q, kv, ms


def unpack_head(q, kv, h):
    """Q, K, V of head h, each (T*64, 128) float32 (redline/run_qkv.py:85-91)."""
    T = q.shape[1]
    Q = torch.cat([layouts.a_unlayout(q[h, t], 64, 128, 64, 128) for t in range(T)])
    K = torch.cat([layouts.b_unlayout(kv[h, t, 0], 128, 64, 128, 64).t() for t in range(T)])
    V = torch.cat([layouts.b_unlayout(kv[h, t, 1], 64, 128, 64, 128) for t in range(T)])
    return Q, K, V


def qkv_post_run(art, cin, tabs, q_out, kv_out):
    """NPU.run("qkv_post", art, [C, TABS, Q, KV]): the QKV-post artifacts' buffer contract (redline/forward.py:246,
    :368; GQA copy: redline/vlm_run.py:433-437, kernels/vlm/qkv_gqa_design.py:1-10), written into the caller's Q
    (heads, T, 9216) and KV (kv heads, T, 2, 9216) uint8 buffers. C is the QKV GEMM's output: bfp16 in the C-stream
    order c_layout_atb(., 128, 128) (uint8), bf16 in that order (a flat bf16 tensor, the C16 GEMMs'), or the build's
    native (M, N) bf16. TABS: the qkv_tables buffer (T, 8448) bf16. The head counts follow from the buffer sizes;
    `art` is accepted for the reference's signature."""
    T = tabs.numel() // TAB
    M = 64 * T
    hq, hkv = q_out.numel() // (T * 9216), kv_out.numel() // (T * 2 * 9216)
    n_cols = 128 * (hq + 2 * hkv)
    if cin.dtype == torch.uint8:
        C = ops.dequantize(cin.reshape(-1), M, n_cols, order="c_atb", dtype=torch.bfloat16)
    elif cin.dim() == 1:
        C = layouts.c_unlayout_atb_values(cin, M, n_cols)
    else:
        C = cin
    cos, sin, wqc, wk = tables_rows(tabs.reshape(T, TAB))
    ops.qkv_post(C, cos.contiguous(), sin.contiguous(), wqc, wk, hq, kv_heads=hkv,
                 out_tiles=(q_out.reshape(-1), kv_out.reshape(-1)))
