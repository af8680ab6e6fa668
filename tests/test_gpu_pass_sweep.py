"""Seeded sweeps of the HBM-bound passes against the oracle, over shapes the fixed-shape tests do not name:
- the bfp16 encoder (rl_bfp16_quantize) in every block order, for float32 and bf16 input, bit-exact, with rows
  spread over 2^-120 .. 2^115 (block exponents on both sides of the encoder's fast-path bounds, subnormal
  elements) and zero rows, decoded values exact;
- the residual + LayerNorm/RMSNorm + modulate pass (rl_ln_modulate) over row widths 64..8192 and both norms, branch
  forms and output orders: x' bit-exact, y within one quantization step of the oracle's (the bar of
  tests/test_gpu_ln.py)."""

import numpy as np
import pytest
import torch

from oracle import bfp16 as F
from oracle import ln as LN
from rlbfp import ops

from test_gpu_ln import check_y, make

pytestmark = pytest.mark.gpu


def dev_t(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def _q_cases(n=16, seed=2029):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        order = ["rowblock", "a_layout", "b_layout", "c_atb"][i % 4]
        if order == "rowblock":
            R, C = int(rng.integers(1, 700)), 8 * int(rng.integers(1, 400))
        elif order == "c_atb":
            R, C = 512 * int(rng.integers(1, 3)), 1024 * int(rng.integers(1, 3))
        else:
            R, C = 128 * int(rng.integers(1, 8)), 64 * int(rng.integers(1, 24))
        out.append((order, R, C, "bf16" if i % 3 else "f32", 500 + i))
    return out


def _stream(x, order):
    if order == "rowblock":
        return F.to_bfp16(x.reshape(-1))
    if order == "a_layout":
        return F.to_bfp16(F.a_layout(x))
    if order == "b_layout":
        return F.pack_b(x.T)
    return F.to_bfp16(F.c_layout_atb(x))


@pytest.mark.parametrize("order,R,C,dt,seed", _q_cases())
def test_quantize_sweep(dev, order, R, C, dt, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((R, C)) * np.exp2(rng.uniform(-120, 115, (R, 1)))).astype(np.float32)
    x[rng.integers(0, R, max(1, R // 16))] = 0.0                       # zero rows: E = 0 blocks
    if dt == "bf16":
        x = F.bf16_round(x)
    p, q = ops.quantize(dev_t(x, torch.bfloat16 if dt == "bf16" else torch.float32), order=order, deq=True)
    np.testing.assert_array_equal(p.cpu().numpy(), _stream(x, order))
    np.testing.assert_array_equal(q.float().cpu().numpy(), F.quantize_rows(x))


def _ln_cases(n=12, seed=2030):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        D = 64 * int(rng.integers(1, 129))
        a_order = "a_layout" if i % 4 == 3 else "rowblock"
        M = 128 * int(rng.integers(1, 6)) if a_order == "a_layout" else int(rng.integers(1, 600))
        out.append((M, D, [None, "bf16", "packed"][i % 3], "rms" if i % 2 else "layer", a_order,
                    int(rng.integers(0, M + 1)), 600 + i))
    # every form of the kernel's first pass: one chunk (2 and 6 blocks per lane), two chunks (7 and 8), one block at
    # a time (9 and more), with the three branch formats among them; split rows at 0, inside and at M
    out += [(301, 1024, "packed", "layer", "rowblock", 100, 620), (96, 3072, None, "rms", "rowblock", 0, 621),
            (257, 3584, "packed", "layer", "rowblock", 257, 622), (128, 3584, "bf16", "rms", "a_layout", 64, 623),
            (130, 4096, None, "layer", "rowblock", 7, 624), (77, 4096, "bf16", "layer", "rowblock", 40, 625),
            (33, 4608, "packed", "rms", "rowblock", 1, 626), (2, 8192, "bf16", "layer", "rowblock", 1, 627)]
    return out


@pytest.mark.parametrize("M,D,br_kind,norm,a_order,split,seed", _ln_cases())
def test_ln_sweep(dev, M, D, br_kind, norm, a_order, split, seed):
    x, br, p = make(M, D, seed, norm)
    br_q = F.quantize_rows(br)
    if br_kind is None:
        branch, br_ref = None, None
    elif br_kind == "bf16":
        branch, br_ref = dev_t(br_q, torch.bfloat16), br_q
    else:
        branch, br_ref = dev_t(F.to_bfp16(br.reshape(-1)), torch.uint8), br_q
    xo, a_p, a_d = ops.ln_modulate(dev_t(x, torch.bfloat16), dev_t(p, torch.bfloat16), branch=branch,
                                   split_row=split, norm=norm, a_order=a_order)
    xp_ref, y_ref = LN.ln_mod_ref(x, br_ref, p, split_row=split, norm=norm)
    np.testing.assert_array_equal(xo.float().cpu().numpy(), xp_ref)
    raw = a_p.cpu().numpy()
    y_got = (F.from_bfp16(raw).reshape(M, D) if a_order == "rowblock"
             else F.a_unlayout(F.from_bfp16(raw), M, D))
    np.testing.assert_array_equal(a_d.float().cpu().numpy(), y_got)    # the bf16 A is the packed A decoded
    check_y(y_got, y_ref)
