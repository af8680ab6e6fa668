"""GPU encoder / decoder against the oracle: packed bytes bit-exact in every block order, decoded values exact."""

import json
import os
import struct

import numpy as np
import pytest
import torch

from oracle import bfp16 as F
from oracle import bfp16_c as C
from rlbfp import ops, layouts

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def to_dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def oracle_stream(x, order):
    if order == "rowblock":
        return F.to_bfp16(x.reshape(-1))
    if order == "a_layout":
        return F.to_bfp16(F.a_layout(x))
    if order == "b_layout":
        return F.pack_b(x.T)
    return F.to_bfp16(F.c_layout_atb(x))


def test_kat_vectors(dev):
    with open(os.path.join(HERE, "golden", "bfp16_kat.json")) as f:
        cases = json.load(f)["cases"]
    x = np.array([[struct.unpack("<f", bytes.fromhex(h))[0] for h in c["x_f32_hex"]] for c in cases], np.float32)
    p, q = ops.quantize(to_dev(x), deq=True)
    got = p.cpu().numpy().reshape(-1, 9)
    for i, c in enumerate(cases):
        assert got[i].tobytes().hex() == c["bytes_hex"], c["why"]
    want = np.array([np.array(c["q"], np.float64) * 2.0 ** (c["E"] - 133) for c in cases])
    np.testing.assert_array_equal(q.float().cpu().numpy().astype(np.float64), want)


@pytest.mark.parametrize("order,R,Cc", [("rowblock", 37, 72), ("rowblock", 4096, 3072), ("a_layout", 256, 192),
                                        ("b_layout", 384, 256), ("c_atb", 512, 2048)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_orders_bit_exact(dev, order, R, Cc, dtype):
    rng = np.random.default_rng(R * 7 + Cc)
    x = (rng.standard_normal((R, Cc)) * np.exp(rng.uniform(-8, 8, (R, 1)))).astype(np.float32)
    if dtype == torch.bfloat16:
        x = F.bf16_round(x)
    p, q = ops.quantize(to_dev(x, dtype), order=order, deq=True)
    want = oracle_stream(x, order) if R * Cc < 2**22 else C.to_bfp16(x)
    np.testing.assert_array_equal(p.cpu().numpy(), want)
    np.testing.assert_array_equal(q.float().cpu().numpy(), F.quantize_rows(x))
    back = ops.dequantize(p, R, Cc, order=order)
    np.testing.assert_array_equal(back.cpu().numpy(), F.quantize_rows(x))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_adversarial_blocks(dev, dtype):
    """ties at every exponent, saturation, -128, zeros, float32 subnormals, signed zeros, infinities. Block exponents
    7/8 and 237/238 bound the kernels' float fast path (8..237); the others take the integer encoder. E = 7 blocks
    hold subnormal elements in [2^-127, 2^-126), which scale into [0.5, 1): 2^-127 is a tie (q = 0), 1.5 * 2^-127
    gives q = 1 (the answer with IEEE denormals, which the integer encoder computes)."""
    rng = np.random.default_rng(11)
    rows = []
    for e in sorted(set(range(1, 255, 3)) | {6, 7, 8, 236, 237, 238, 254}):
        step = 2.0 ** (e - 133)
        rows.append((rng.integers(-127, 127, 8) + 0.5) * step)
        rows.append(np.array([127.5, -127.5, 64.5, -64.5, 0.5, -0.5, 1.5, -2.5]) * step)
    rows.append(rng.integers(-2**23 + 1, 2**23, 8) * 2.0 ** -149)      # subnormal block (E = 0)
    rows.append(np.array([2**-149, -2**-149, 0, -0.0, 2**-140, 0, 0, 0]))
    for e in (7, 8):                                                    # subnormal elements beside an E = 7 / 8 max
        rows.append(np.array([1.5 * 2.0 ** (e - 127), 2**-127, -2**-127, 1.5 * 2**-127, -1.5 * 2**-127,
                              1.75 * 2**-127, 2**-128, -1.5 * 2**-128]))
    rows.append(np.array([np.inf, -np.inf, 1.0, 0, 0, 0, 0, 0]))        # E = 255, saturates
    x = np.concatenate(rows).astype(np.float32).reshape(-1, 8)
    if dtype == torch.bfloat16:
        x = F.bf16_round(x)
    p, q = ops.quantize(to_dev(x, dtype), deq=True)
    np.testing.assert_array_equal(p.cpu().numpy(), C.to_bfp16(x))
    np.testing.assert_array_equal(p.cpu().numpy(), F.to_bfp16(x))
    np.testing.assert_array_equal(q.float().cpu().numpy(), F.quantize_rows(x))   # the E = 255 row decodes to +-inf
    e7 = F.to_bfp16(x[-3:-2]).reshape(9)                                # the E = 7 row: q = [96, 0, 0, 1, -1, 1, 0, 0]
    assert e7[0] == 7 and list(e7[1:].view(np.int8)) == [96, 0, 0, 1, -1, 1, 0, 0]


@pytest.mark.parametrize("order,R,Cc", [("rowblock", 3, 2728), ("rowblock", 1023, 8), ("rowblock", 5, 24),
                                        ("a_layout", 256, 128), ("b_layout", 256, 128), ("c_atb", 512, 1024)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_dequantize_every_exponent(dev, order, R, Cc, dtype):
    """Arbitrary streams, as a packed file may hold them: every exponent byte 0..255 under random q bytes, and the
    overflow edges (E = 254 with q = -128, E = 255 with q = +-64 / +-65 / 127 / -128), decoded as from_bfp16 decodes
    them: float32 products, subnormal for small E and +-inf where q * 2^(E - 133) >= 2^128. Both CPU decoders agree
    first. Ragged streams (3 x 2728: 1023 blocks; 1023 x 8; 5 x 24: 15 blocks) end inside a thread's run of 4."""
    rng = np.random.default_rng(R + Cc)
    nb = R * Cc // 8
    raw = rng.integers(0, 256, (nb, 9), dtype=np.uint8)
    raw[:, 0] = np.arange(nb) % 256
    edges = [(254, [-128, 127, -127, 64, -64, 65, -65, 1]), (255, [-128, 127, -127, 64, -64, 65, -65, 0]),
             (0, [1, -1, -128, 127, 0, 2, -2, 3]), (6, [1, -1, -128, 127, 0, 2, -2, 3])]
    for i, (e, q) in enumerate(edges):
        if i < nb:
            raw[i, 0] = e
            raw[i, 1:] = np.array(q, np.int8).view(np.uint8)
    flat = F.from_bfp16(raw.reshape(-1))
    np.testing.assert_array_equal(flat.view(np.uint32), C.from_bfp16(raw.reshape(-1)).view(np.uint32))
    assert np.isinf(flat).any() and ((np.abs(flat) < 2.0**-126) & (flat != 0)).any()
    if order == "rowblock":
        want = flat.reshape(R, Cc)
    elif order == "a_layout":
        want = F.a_unlayout(flat, R, Cc)
    elif order == "b_layout":
        want = F.b_unlayout(flat, Cc, R).T     # the decoded matrix is W (N rows, K columns)
    else:
        want = F.c_unlayout_atb(flat, R, Cc)
    got = ops.dequantize(to_dev(raw.reshape(-1), torch.uint8), R, Cc, order=order, dtype=dtype)
    if dtype == torch.bfloat16:
        np.testing.assert_array_equal(got.view(torch.int16).cpu().numpy().view(np.uint16),
                                      (np.ascontiguousarray(want).view(np.uint32) >> 16).astype(np.uint16))
    else:
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), np.ascontiguousarray(want).view(np.uint32))


def test_truncate_variant_differs(dev):
    x = np.array([[1.0, 2**-7, 3 * 2**-7, -2**-7, 255 / 128, -255 / 128, 5 * 2**-7, 0]], np.float32)
    p, _ = ops.quantize(to_dev(x))
    assert p.cpu().numpy().tobytes() == F.to_bfp16(x).tobytes()
    assert p.cpu().numpy().tobytes() != F.to_bfp16(x, truncate=True).tobytes()


def test_pack_weight_equals_pack_b(dev):
    """The GPU packer writes the bytes of redline/pack_weights.py: to_bfp16(b_layout(W.T, 64, 128)), including the
    SwiGLU interleave of the up weights."""
    rng = np.random.default_rng(5)
    K, Fh = 192, 128
    wg = (rng.standard_normal((Fh, K)) * 0.02).astype(np.float32)
    wp = (rng.standard_normal((Fh, K)) * 0.02).astype(np.float32)
    W = ops.interleave_up(to_dev(wg), to_dev(wp))
    got = ops.pack_weight(W.contiguous()).cpu().numpy()
    np.testing.assert_array_equal(got, F.pack_b(F.interleave_up(wg, wp)))
    np.testing.assert_array_equal(layouts.unpack_b(to_dev(got, torch.uint8), K, 2 * Fh).cpu().numpy(),
                                  F.decode_b(got, K, 2 * Fh))


def test_layout_names(dev):
    rng = np.random.default_rng(6)
    x = rng.standard_normal(8 * 1000).astype(np.float32)
    raw = layouts.to_bfp16(to_dev(x))
    np.testing.assert_array_equal(raw.cpu().numpy(), F.to_bfp16(x))
    np.testing.assert_array_equal(layouts.from_bfp16(raw).cpu().numpy(), F.from_bfp16(F.to_bfp16(x)))


def test_strided_input_and_small_stream(dev):
    rng = np.random.default_rng(7)
    big = rng.standard_normal((9, 48)).astype(np.float32)
    x = to_dev(big)[:, :40]                      # ld 48, 40 columns
    p, _ = ops.quantize(x)
    np.testing.assert_array_equal(p.cpu().numpy(), F.to_bfp16(big[:, :40].reshape(-1)))
    one = to_dev(big[:1, :8])                    # a single block: the decoder's window must not read past 9 bytes
    p1, _ = ops.quantize(one)
    np.testing.assert_array_equal(ops.dequantize(p1, 1, 8).cpu().numpy(), F.quantize_rows(big[:1, :8]))
