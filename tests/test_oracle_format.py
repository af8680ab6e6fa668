"""The oracle's bfp16 encoder/decoder pinned against hand-derived known answers, an independent C restatement, and
the format's closed-form invariants (redline/npu_layouts.py:62-94)."""

import json
import os
import struct

import numpy as np
import pytest
import torch

from oracle import bfp16 as F
from oracle import bfp16_c as C

HERE = os.path.dirname(os.path.abspath(__file__))


def kat_cases():
    with open(os.path.join(HERE, "golden", "bfp16_kat.json")) as f:
        return json.load(f)["cases"]


def kat_x(case):
    return np.array([struct.unpack("<f", bytes.fromhex(h))[0] for h in case["x_f32_hex"]], np.float32)


@pytest.mark.parametrize("case", kat_cases(), ids=lambda c: c["bytes_hex"][:6])
def test_kat_encode(case):
    x = kat_x(case)
    assert F.to_bfp16(x).tobytes().hex() == case["bytes_hex"]
    assert C.to_bfp16(x).tobytes().hex() == case["bytes_hex"]


@pytest.mark.parametrize("case", kat_cases(), ids=lambda c: c["bytes_hex"][:6])
def test_kat_decode(case):
    raw = np.frombuffer(bytes.fromhex(case["bytes_hex"]), np.uint8)
    want = np.array(case["q"], np.float64) * 2.0 ** (case["E"] - 133)
    np.testing.assert_array_equal(F.from_bfp16(raw).astype(np.float64), want)
    np.testing.assert_array_equal(C.from_bfp16(raw).astype(np.float64), want)


def test_decode_every_exponent_byte():
    """Arbitrary 9-byte blocks (every E byte 0..255, every q byte -128..127): both decoders give the float64 product
    q * 2^(E - 133) wherever it is below 2^128 (all of them exact in float32, subnormal below 2^-126), and +-inf at and
    above it (E = 254 with q = -128, E = 255 with |q| >= 64)."""
    E, q = np.meshgrid(np.arange(256), np.arange(-128, 128), indexing="ij")
    E, q = E.reshape(-1), q.reshape(-1)
    n = E.size // 8
    raw = np.zeros((n, 9), np.uint8)
    raw[:, 0] = E.reshape(n, 8)[:, 0]                 # 8 consecutive q values share one E (E changes every 32 blocks)
    raw[:, 1:] = q.reshape(n, 8).astype(np.int8).view(np.uint8)
    exact = q.astype(np.float64) * np.ldexp(1.0, E - 133)
    want = np.where(np.abs(exact) >= 2.0**128, np.copysign(np.inf, exact), exact)
    for got in (F.from_bfp16(raw), C.from_bfp16(raw)):
        np.testing.assert_array_equal(got.astype(np.float64), want)
    assert np.isinf(want).sum() == 1 + 65 + 64 and (want[(E == 0) & (q == 1)] == 2.0**-133).all()


def adversarial(rng, nblocks):
    """Blocks built to hit ties, saturation, -128, zeros, subnormals and wide exponent spreads."""
    out = []
    E = rng.integers(1, 250, nblocks)
    for e in E:
        kind = rng.integers(0, 6)
        step = 2.0 ** (int(e) - 133)
        if kind == 0:    # exact ties at every magnitude
            q = rng.integers(-127, 127, 8) + 0.5
            q[0] = 64.5 if rng.random() < 0.5 else -127.5
            v = q * step
        elif kind == 1:  # the max element right at the saturation boundary
            v = rng.uniform(-127.5, 127.5, 8) * step
            v[rng.integers(0, 8)] = (127.5 if rng.random() < 0.5 else -127.5) * step
        elif kind == 2:  # huge spread
            v = rng.standard_normal(8) * 2.0 ** rng.integers(-40, 1, 8) * step * 64
        elif kind == 3:  # zeros mixed in
            v = rng.standard_normal(8) * step * 64
            v[rng.random(8) < 0.5] = 0.0
        elif kind == 4:  # subnormal float32 values
            v = rng.integers(-2**23 + 1, 2**23, 8) * 2.0 ** -149
        else:
            v = rng.standard_normal(8) * step * 64
        out.append(np.asarray(v, np.float64))
    return np.concatenate(out).astype(np.float32)


def test_numpy_vs_c_restatement_random_and_adversarial():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(8 * 100000) * np.exp(rng.uniform(-40, 40, 8 * 100000))).astype(np.float32)
    x = np.concatenate([x, adversarial(rng, 50000)])
    a, b = F.to_bfp16(x), C.to_bfp16(x)
    assert np.array_equal(a, b)
    assert np.array_equal(F.from_bfp16(a), C.from_bfp16(a))


def test_invariants():
    """|q| of the max-exponent element is in [64, 128] (127 after saturation, 128 only as -128) for normal blocks;
    decoding is within half a step of the input except where saturation clips."""
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(8 * 20000) * np.exp(rng.uniform(-20, 20, 8 * 20000))).astype(np.float32)
    raw = F.to_bfp16(x).reshape(-1, 9)
    E = raw[:, 0].astype(np.int32)
    q = raw[:, 1:].view(np.int8).astype(np.int32)
    xb = x.reshape(-1, 8)
    e = (xb.view(np.uint32) >> 23) & 0xFF
    assert np.array_equal(E, e.max(1))
    imax = np.argmax(e, 1)
    qmax = np.abs(q[np.arange(len(q)), imax])
    assert ((qmax >= 64) & (qmax <= 128)).all()
    step = np.ldexp(1.0, E - 133)[:, None]
    err = np.abs(F.from_bfp16(raw).reshape(-1, 8).astype(np.float64) - xb)
    sat = (q == 127) & (xb > 127 * step)
    assert (err[~sat] <= 0.5 * np.broadcast_to(step, err.shape)[~sat]).all()
    assert (err[sat] < np.broadcast_to(step, err.shape)[sat]).all()   # clipped at 127: less than one step


def test_reencode_identity_except_minus_128():
    """Re-encoding decoded values with the same blocks gives the same bytes (redline/forward.py:342), except in a
    block whose max-exponent element rounded to -128: its decoded value is -2^(E-126), one exponent higher."""
    rng = np.random.default_rng(3)
    x = adversarial(rng, 30000)
    raw = F.to_bfp16(x)
    again = F.to_bfp16(F.from_bfp16(raw))
    blocks = raw.reshape(-1, 9)
    has_m128 = (blocks[:, 1:].view(np.int8) == -128).any(1)
    same = (again.reshape(-1, 9) == blocks).all(1)
    assert same[~has_m128].all()
    assert (~same[has_m128]).any()  # the corner is exercised


def test_truncate_mode_is_floor_and_differs():
    kat = kat_x(kat_cases()[2])
    assert F.to_bfp16(kat, truncate=True).tobytes() != F.to_bfp16(kat).tobytes()
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(8 * 5000) * 3).astype(np.float32)
    assert np.array_equal(F.to_bfp16(x, truncate=True), C.to_bfp16(x, truncate=True))


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(200000) * np.exp(rng.uniform(-30, 30, 200000))).astype(np.float32)
    ties = (rng.integers(0, 2**16, 20000).astype(np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, ties[np.isfinite(ties)]])
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(F.bf16_round(x), want)


def test_bf16_round_f64_single_rounding():
    """bf16_round_f64(v) equals rounding the exact value once: checked with values just off a bf16 tie, where
    rounding through float32 first would land on the tie."""
    rng = np.random.default_rng(6)
    base = (rng.integers(0x3F80, 0x4700, 5000).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    ulp_bf = np.ldexp(1.0, np.frexp(base)[1] - 8)
    tie = base + ulp_bf / 2
    for eps_sign in (+1, -1):
        v = tie + eps_sign * ulp_bf * 2.0 ** -30       # below float32 resolution around the tie
        got = F.bf16_round_f64(v).astype(np.float64)
        want = base + (ulp_bf if eps_sign > 0 else 0.0)
        np.testing.assert_array_equal(got, want)
    exact_tie = F.bf16_round_f64(tie).astype(np.float64)   # exact ties go to even
    even = (base.astype(np.float32).view(np.uint32) >> 16) & 1
    np.testing.assert_array_equal(exact_tie, np.where(even == 0, base, base + ulp_bf))
