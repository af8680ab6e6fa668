"""bfp16ebs8 format, NPU stream layouts and the weight packer, restated in numpy (oracle; test infrastructure only).

Format (redline/npu_layouts.py:62-73 encode, :90-94 decode): a block is 8 consecutive values of a stream, stored in 9
bytes ``[E][q0..q7]``. ``E`` is the largest biased float32 exponent field in the block (sign ignored) and
``q_i = clip(rint(x_i * 2^(133 - E)), -128, 127)`` with round-half-to-even; the value of a stored element is
``q_i * 2^(E - 133)``.

Layouts (redline/npu_layouts.py:11-59) are permutations of an (R, C) matrix into a flat stream; here each one is
written as the stream position of element (r, c), so that the scalar formulas of redline/forward.py:64-80 and the
vectorised maps below are two independent statements of the same order.
"""

import numpy as np

BLOCK_VALUES = 8
BLOCK_BYTES = 9
K_TILE, N_TILE = 64, 128            # B-stream tile of the GEMM weights (redline/pack_weights.py:34)
A_TILE_M, A_TILE_K = 128, 64        # A-stream tile (redline/forward.py:32, "a_layout(., 128, 64)")
C_TILE, C_ROWS, C_COLS = 128, 4, 8  # C-stream tile and group of the ATB designs (redline/forward.py:64-71)


# ---------------------------------------------------------------------------------------------------------------
# bfloat16 rounding (round to nearest even), float32 in and out
# ---------------------------------------------------------------------------------------------------------------

def bf16_bits(x):
    """float32 -> bfloat16 bit patterns (uint16), round half to even; NaN stays a quiet NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    r = ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)).astype(np.uint32)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    r = np.where(nan, ((u >> np.uint64(16)).astype(np.uint32) | np.uint32(0x40)), r)
    return r.astype(np.uint16)


def bf16_from_bits(b):
    """bfloat16 bit patterns (uint16) -> float32 (exact)."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_round(x):
    """float32 values rounded to the nearest bfloat16 (ties to even), returned as float32."""
    return bf16_from_bits(bf16_bits(x)).reshape(np.shape(x))


def bf16_round_f64(v):
    """float64 -> nearest bfloat16 (ties to even) with a single rounding, as float32.

    Rounding to float32 first and then to bf16 differs from one rounding only when the float32 result lands exactly
    on a bf16 tie (low 16 bits 0x8000) while v itself was not that tie; then the float32 value is moved one float32
    ulp toward v, which breaks the tie the way v does."""
    v = np.asarray(v, dtype=np.float64)
    f = np.atleast_1d(v.astype(np.float32))
    vv = np.atleast_1d(v)
    tie = (f.view(np.uint32) & np.uint32(0xFFFF)) == np.uint32(0x8000)
    off = f.astype(np.float64) != vv
    toward = np.where(vv > f, np.inf, -np.inf).astype(np.float32)
    f = np.where(tie & off, np.nextafter(f, toward), f)
    return bf16_round(f).reshape(v.shape)


# ---------------------------------------------------------------------------------------------------------------
# encode / decode
# ---------------------------------------------------------------------------------------------------------------

def block_exponent(xb):
    """(nblocks, 8) float32 -> (nblocks,) int32: the largest biased exponent field of each block."""
    return ((xb.view(np.uint32) >> np.uint32(23)) & np.uint32(0xFF)).max(axis=1).astype(np.int32)


def to_bfp16(x, truncate=False):
    """Flat float32 stream (length a multiple of 8) -> uint8 stream, 9 bytes per block of 8.

    Follows redline/npu_layouts.py:62-73. The scale 2^(133 - E) is a power of two, so ``x * scale`` is exact in
    float64 and the only rounding is the final one: ``np.rint`` (half to even) or, with ``truncate=True``, a floor
    (the upstream helper.h packer, redline/npu_layouts.py:74-87, kept only as a negative example; its handling of
    subnormal elements is not restated)."""
    xb = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, BLOCK_VALUES)
    e = block_exponent(xb)
    scaled = np.ldexp(xb.astype(np.float64), (133 - e)[:, None])
    q = np.floor(scaled) if truncate else np.rint(scaled)
    q = np.clip(q, -128, 127).astype(np.int8)
    out = np.empty((xb.shape[0], BLOCK_BYTES), dtype=np.uint8)
    out[:, 0] = e.astype(np.uint8)
    out[:, 1:] = q.view(np.uint8)
    return out.reshape(-1)


def from_bfp16(raw):
    """uint8 stream (9 bytes per block) -> flat float32 values ``q * 2^(E - 133)`` (redline/npu_layouts.py:90-94).
    Every decoded value is exact in float32 and in bfloat16, except where |q| * 2^(E - 133) >= 2^128: q = -128 with
    E = 254, and |q| >= 64 with E = 255. Those are beyond both formats' range and decode to +-inf (the reference's
    float64 result would be finite; the encoder writes such blocks only for inputs within half a step of -float32 max,
    and for infinite inputs)."""
    blk = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1, BLOCK_BYTES)
    q = blk[:, 1:].view(np.int8).astype(np.float32)
    scale = np.ldexp(np.float32(1.0), blk[:, :1].astype(np.int32) - 133).astype(np.float32)  # exact, >= 2^-133
    with np.errstate(over="ignore"):
        return (q * scale).reshape(-1)  # exact: |q| < 2^8, so q * 2^(E-133) is a float32 (subnormal for small E)


def quantize(x):
    """Round-trip of a flat stream through the format: from_bfp16(to_bfp16(x)) with the input's shape."""
    return from_bfp16(to_bfp16(x)).reshape(np.shape(x))


def quantize_rows(x):
    """(R, C) matrix, blocks = 8 consecutive columns of a row (the GEMM's K blocks): the decoded values."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    return quantize(x.reshape(-1)).reshape(x.shape)


# ---------------------------------------------------------------------------------------------------------------
# stream layouts as position maps
# ---------------------------------------------------------------------------------------------------------------

def _mix(*pairs):
    """Mixed-radix number from (digit, radix) pairs, most significant first."""
    i = 0
    for d, radix in pairs:
        i = i * radix + d
    return i


def b_pos(r, c, R, C, k=K_TILE, n=N_TILE):
    """Stream position of B[r, c] in b_layout(B, k, n) (redline/npu_layouts.py:11-15): (k, n) tiles ordered column
    tile major, then 16-column super-blocks, 8-row bands, the two 8-column halves, column, row. A block is 8
    consecutive rows (K) of one column."""
    return _mix((c // n, C // n), (r // k, R // k), ((c % n) // 16, n // 16), ((r % k) // 8, k // 8),
                ((c % 16) // 8, 2), (c % 8, 8), (r % 8, 8))


def a_pos(r, c, R, C, m=A_TILE_M, k=A_TILE_K):
    """Stream position of A[r, c] in a_layout(A, m, k) (redline/npu_layouts.py:18-22): (m, k) tiles row major, then
    16-row super-blocks, 8-column blocks, the two 8-row halves, row, column. A block is 8 consecutive columns."""
    return _mix((r // m, R // m), (c // k, C // k), ((r % m) // 16, m // 16), ((c % k) // 8, k // 8),
                ((r % 16) // 8, 2), (r % 8, 8), (c % 8, 8))


def c_pos(r, c, R, C, m, n):
    """Stream position in upstream's C order (redline/npu_layouts.py:25-28): (m, n) tiles row major, then 2x2
    super-blocks of row-major 8x8 blocks."""
    return _mix((r // m, R // m), (c // n, C // n), ((r % m) // 16, m // 16), ((c % n) // 16, n // 16),
                ((r % 16) // 8, 2), ((c % 16) // 8, 2), (r % 8, 8), (c % 8, 8))


def c_atb_pos(r, c, R, C, m=C_TILE, n=C_TILE, rows=C_ROWS, cols=C_COLS):
    """Stream position in the C order the ATB designs emit (redline/npu_layouts.py:31-47): groups of (rows M-tiles x
    cols N-tiles), row group outer; inside a group, per core column its `rows` tiles; inside a tile 2x2 super-blocks
    of row-major 8x8 blocks. A block is 8 consecutive columns."""
    return _mix((r // (rows * m), R // (rows * m)), (c // (cols * n), C // (cols * n)), ((c // n) % cols, cols),
                ((r // m) % rows, rows), ((r % m) // 16, m // 16), ((c % n) // 16, n // 16),
                ((r % 16) // 8, 2), ((c % 16) // 8, 2), (r % 8, 8), (c % 8, 8))


def _grid(R, C):
    return np.arange(R, dtype=np.int64)[:, None], np.arange(C, dtype=np.int64)[None, :]


def _to_stream(x, posfn, *tile):
    x = np.asarray(x)
    R, C = x.shape
    r, c = _grid(R, C)
    out = np.empty(R * C, dtype=x.dtype)
    out[posfn(r, c, R, C, *tile).reshape(-1)] = x.reshape(-1)
    return out


def _from_stream(s, R, C, posfn, *tile):
    r, c = _grid(R, C)
    return np.asarray(s).reshape(-1)[posfn(r, c, R, C, *tile)]


def b_layout(b, k=K_TILE, n=N_TILE):
    """(K, N) -> flat B stream (redline/npu_layouts.py:11-15). Requires K % k == 0, N % n == 0."""
    K, N = np.shape(b)
    assert K % k == 0 and N % n == 0 and k % 8 == 0 and n % 16 == 0
    return _to_stream(b, b_pos, k, n)


def b_unlayout(s, K, N, k=K_TILE, n=N_TILE):
    """Inverse of b_layout (redline/npu_layouts.py:50-53)."""
    return _from_stream(s, K, N, b_pos, k, n)


def a_layout(a, m=A_TILE_M, k=A_TILE_K):
    """(M, K) -> flat A stream (redline/npu_layouts.py:18-22). Requires M % m == 0, K % k == 0."""
    M, K = np.shape(a)
    assert M % m == 0 and K % k == 0 and m % 16 == 0 and k % 8 == 0
    return _to_stream(a, a_pos, m, k)


def a_unlayout(s, M, K, m=A_TILE_M, k=A_TILE_K):
    """Inverse of a_layout (redline/npu_layouts.py:56-59)."""
    return _from_stream(s, M, K, a_pos, m, k)


def c_unlayout(s, M, N, m, n):
    """Upstream's C stream -> (M, N) (redline/npu_layouts.py:25-28; not what the ATB designs emit)."""
    return _from_stream(s, M, N, c_pos, m, n)


def c_layout_atb(c, m=C_TILE, n=C_TILE, rows=C_ROWS, cols=C_COLS):
    """(M, N) -> the ATB C stream (redline/npu_layouts.py:42-47). Requires M % (rows m) == 0, N % (cols n) == 0."""
    M, N = np.shape(c)
    assert M % (rows * m) == 0 and N % (cols * n) == 0
    return _to_stream(c, c_atb_pos, m, n, rows, cols)


def c_unlayout_atb(s, M, N, m=C_TILE, n=C_TILE, rows=C_ROWS, cols=C_COLS):
    """Inverse of c_layout_atb (redline/npu_layouts.py:31-39)."""
    return _from_stream(s, M, N, c_atb_pos, m, n, rows, cols)


# ---------------------------------------------------------------------------------------------------------------
# scalar index formulas (redline/forward.py:64-80, and the B-stream formula); loops, for cross-checking only
# ---------------------------------------------------------------------------------------------------------------

def atb_index(r, c, N):
    """Scalar stream position of element (r, c) in the ATB C order, 128x128 tiles, groups of 4x8 tiles
    (redline/forward.py:64-71)."""
    i = (r // 512) * (N // 1024) + c // 1024
    for radix, digit in ((8, (c // 128) % 8), (4, (r // 128) % 4), (8, (r // 16) % 8), (8, (c // 16) % 8),
                         (2, (r // 8) % 2), (2, (c // 8) % 2), (8, r % 8), (8, c % 8)):
        i = i * radix + digit
    return i


def a_index(r, c, K):
    """Scalar stream position of element (r, c) in the A order, 128x64 tiles (redline/forward.py:74-80)."""
    i = (r // 128) * (K // 64) + c // 64
    for radix, digit in ((8, (r // 16) % 8), (8, (c // 8) % 8), (2, (r // 8) % 2), (8, r % 8), (8, c % 8)):
        i = i * radix + digit
    return i


def b_index(r, c, K):
    """Scalar stream position of B[r, c] in the B order, 64x128 tiles (the element formula of b_layout)."""
    i = (c // 128) * (K // 64) + r // 64
    for radix, digit in ((8, (c // 16) % 8), (8, (r // 8) % 8), (2, (c // 8) % 2), (8, c % 8), (8, r % 8)):
        i = i * radix + digit
    return i


# ---------------------------------------------------------------------------------------------------------------
# the weight packer (redline/pack_weights.py:72-89)
# ---------------------------------------------------------------------------------------------------------------

def pack_b(B):
    """(K, N) float32 -> the packed B stream bytes: to_bfp16(b_layout(B, 64, 128)) (redline/pack_weights.py:72-79).
    The reference encodes in chunks of 2^23 values only to bound memory; blocks are independent, so one pass gives
    the same bytes."""
    return to_bfp16(b_layout(np.ascontiguousarray(B, dtype=np.float32)))


def decode_b(packed, K, N):
    """Packed B stream -> the decoded (K, N) float32 matrix."""
    return b_unlayout_fast(from_bfp16(packed), K, N)


def b_unlayout_fast(s, K, N):
    """b_unlayout for 64 x 128 tiles as one strided copy: the stream's mixed-radix digits are
    (nt, kt, sbc, br, bis, col, row) with radices (N/128, K/64, 8, 8, 2, 8, 8), and element (r, c) has
    r = (kt, br, row), c = (nt, sbc, bis, col); the transpose reorders the digits from one to the other."""
    x = np.asarray(s).reshape(N // 128, K // 64, 8, 8, 2, 8, 8)
    return x.transpose(1, 3, 6, 0, 2, 4, 5).reshape(K, N)


def interleave_up(wg, wp):
    """gate / proj Linear weights, each (F, K) -> B_up (K, 2F): per 128-column tile t the columns are
    [gate units 64t..64t+63 | proj units 64t..64t+63] (redline/pack_weights.py:82-89)."""
    wg = np.asarray(wg, dtype=np.float32)
    wp = np.asarray(wp, dtype=np.float32)
    F, K = wg.shape
    assert wp.shape == (F, K) and F % 64 == 0
    B = np.empty((K, F // 64, 2, 64), dtype=np.float32)
    B[:, :, 0, :] = wg.T.reshape(K, F // 64, 64)
    B[:, :, 1, :] = wp.T.reshape(K, F // 64, 64)
    return B.reshape(K, 2 * F)
