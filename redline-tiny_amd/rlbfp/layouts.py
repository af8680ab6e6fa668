"""The bfp16 encode/decode names of redline/npu_layouts.py on the HIP kernels (device tensors in, device tensors out).

``to_bfp16(x)`` encodes a flat stream (blocks of 8 consecutive values) and is bit-exact to npu_layouts.to_bfp16
(redline/npu_layouts.py:62-73, round half to even); ``from_bfp16`` decodes exactly (:90-94). The layout permutations
are fused into the encoder instead of being separate passes: ``to_bfp16_a_layout`` = to_bfp16(a_layout(x, 128, 64)),
``pack_b`` = to_bfp16(b_layout(B, 64, 128)) for B = W.T, ``to_bfp16_c_atb`` = to_bfp16(c_layout_atb(x, 128, 128)).
"""

import torch

from . import ops


def to_bfp16(x):
    """Flat (or any-shaped) float32 / bf16 device tensor, size a multiple of 8 -> packed uint8 stream."""
    flat = x.reshape(1, -1) if x.numel() < 8 or x.numel() % 8 else x.reshape(-1, 8)
    p, _ = ops.quantize(flat.contiguous())
    return p


def from_bfp16(raw):
    """Packed uint8 stream -> flat float32 values."""
    n = raw.numel() // 9 * 8
    return ops.dequantize(raw, n // 8, 8).reshape(-1)


def to_bfp16_a_layout(x):
    return ops.quantize(x.contiguous(), order="a_layout")[0]


def to_bfp16_c_atb(x):
    return ops.quantize(x.contiguous(), order="c_atb")[0]


def pack_b(B):
    """(K, N) matrix B = W.T -> packed B stream (redline/pack_weights.py:72-79); pass W (N, K) to pack_weight."""
    return ops.pack_weight(B.t().contiguous())


def from_bfp16_a_layout(raw, M, K):
    return ops.dequantize(raw, M, K, order="a_layout")


def from_bfp16_c_atb(raw, M, N):
    return ops.dequantize(raw, M, N, order="c_atb")


def unpack_b(raw, K, N):
    """Packed B stream -> the decoded (K, N) matrix."""
    return ops.dequantize(raw, N, K, order="b_layout").t()


def c_atb_block_index(M, N, device="cuda"):
    """For each block of the C stream c_layout_atb(., 128, 128) (blocks of 8 consecutive columns, stream order), the
    index of the same block in row-major order: block (r, c / 8) -> r * (N / 8) + c / 8 (redline/npu_layouts.py:42-47;
    the same decomposition as the encoder's RL_ORDER_C_ATB). M % 512 == 0, N % 1024 == 0."""
    if M % 512 or N % 1024:
        raise ValueError("the C stream needs M % 512 == 0 and N % 1024 == 0")
    s = torch.arange(M * N // 8, device=device, dtype=torch.int64)
    rib, bc, br, sbc, sbr = s & 7, (s >> 3) & 1, (s >> 4) & 1, (s >> 5) & 7, (s >> 8) & 7
    rowg, colg, t = (s >> 11) & 3, (s >> 13) & 7, s >> 16
    cg, rg = t % (N // 1024), t // (N // 1024)
    r = rg * 512 + rowg * 128 + sbr * 16 + br * 8 + rib
    cb = cg * 128 + colg * 16 + sbc * 2 + bc
    return r * (N // 8) + cb


def c_layout_atb_values(x):
    """(M, N) device tensor -> its values as a flat C stream, c_layout_atb(x, 128, 128), in x's dtype (e.g. the bf16
    residual stream of redline/run_ln.py:28-30)."""
    M, N = x.shape
    return x.contiguous().reshape(-1, 8)[c_atb_block_index(M, N, x.device)].reshape(-1)


def c_unlayout_atb_values(s, M, N):
    """Flat C stream of values -> (M, N) row major (redline/npu_layouts.py:31-39)."""
    out = torch.empty((M * N // 8, 8), dtype=s.dtype, device=s.device)
    out[c_atb_block_index(M, N, s.device)] = s.reshape(-1, 8)
    return out.reshape(M, N)


def a_block_index(R, C, m, k, device="cuda"):
    """Stream block index, in a_layout(., m, k) (redline/npu_layouts.py:18-22), of each row-major block (r, c / 8):
    (m, k) tiles row major, then 16-row bands, 8-column blocks, the two 8-row halves, row."""
    r = torch.arange(R, device=device, dtype=torch.int64)[:, None]
    cb = torch.arange(C // 8, device=device, dtype=torch.int64)[None, :]
    c = cb * 8
    t = (r // m) * (C // k) + c // k
    return ((((t * (m // 16) + (r % m) // 16) * (k // 8) + (c % k) // 8) * 2 + (r % 16) // 8) * 8 + r % 8).reshape(-1)


def b_block_index(K, N, k, n, device="cuda"):
    """Stream block index, in b_layout(., k, n) (redline/npu_layouts.py:11-15), of each block (k-block kb, column c)
    of a (K, N) matrix, blocks = 8 consecutive rows of one column; indexed kb * N + c: (k, n) tiles column-tile major,
    then 16-column bands, 8-row blocks, the two 8-column halves, column."""
    kb = torch.arange(K // 8, device=device, dtype=torch.int64)[:, None]
    c = torch.arange(N, device=device, dtype=torch.int64)[None, :]
    r = kb * 8
    t = (c // n) * (K // k) + r // k
    return ((((t * (n // 16) + (c % n) // 16) * (k // 8) + (r % k) // 8) * 2 + (c % 16) // 8) * 8 + c % 8).reshape(-1)


def a_unlayout(raw, R, C, m, k):
    """bfp16 bytes of a_layout(x, m, k) -> x (R, C) float32."""
    blocks = from_bfp16(raw).reshape(-1, 8)
    return blocks[a_block_index(R, C, m, k, raw.device)].reshape(R, C)


def b_unlayout(raw, K, N, k, n):
    """bfp16 bytes of b_layout(b, k, n) -> b (K, N) float32."""
    blocks = from_bfp16(raw).reshape(-1, 8)[b_block_index(K, N, k, n, raw.device)]  # (K/8 * N, 8): [kb, c, e]
    return blocks.reshape(K // 8, N, 8).permute(0, 2, 1).reshape(K, N)
