"""GPU residual + LayerNorm/RMSNorm + modulate pass (rl_ln_modulate) against the oracle (oracle/ln.py).

x' is bit-exact. y is computed in fp32 on the GPU and in float64 by the oracle, then quantized to bfp16: at least
99.9% of the stored values equal the oracle's quantized y, every other one is within one quantization step of its
block (2^(E-133) of the oracle's block exponent, or of the GPU's where the exponents differ), and max |y - y_ref| /
max |y_ref| <= 1e-2 (the reference's metric, redline/run_glue.py:158-159) with correlation > 0.9999 (the bar of
redline/run_ln.py:125)."""

import numpy as np
import pytest
import torch

from oracle import bfp16 as F
from oracle import gemm as G
from oracle import ln as LN
from rlbfp import _lib as L
from rlbfp import ops

pytestmark = pytest.mark.gpu


def dev_t(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def make(M, D, seed, norm="layer"):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((M, D)) * 3).astype(np.float32)
    x[:, rng.integers(0, D, 8)] *= 40
    x = F.bf16_round(x)
    br = rng.standard_normal((M, D)).astype(np.float32)
    if norm == "layer":
        p = LN.ln_params(np.tanh(rng.standard_normal((2, D))), 1 + 0.3 * rng.standard_normal((2, D)))
    else:
        p = LN.rms_params((1 + 0.2 * rng.standard_normal(D)).astype(np.float32))
    return x, br, p


def check_y(y_got, y_ref):
    """y_got: decoded bfp16 values (M, D) float32; y_ref float64."""
    q_ref = F.quantize_rows(y_ref.astype(np.float32))
    eq = y_got == q_ref
    assert eq.mean() > 0.999, f"{(~eq).sum()} of {eq.size} values differ from the quantized reference"
    blocks = np.abs(np.stack([q_ref, y_got])).reshape(2, -1, 8).max(2).max(0)
    step = 2.0 ** (np.floor(np.log2(np.maximum(blocks, 1e-30))) - 6)  # one q step of the block: 2^(E - 133)
    d = np.abs(y_got - q_ref).reshape(-1, 8).max(1)
    assert (d <= step * 1.0000001).all(), f"max off {np.max(d / step)} steps"
    assert G.rel_err(y_got, y_ref) <= 1e-2
    assert G.corr(y_got, y_ref) > 0.9999


@pytest.mark.parametrize("M,D,br_kind,norm,split", [
    (4, 64, None, "layer", 0),
    (131, 192, "bf16", "layer", 100),
    (256, 640, "packed", "layer", 128),
    (64, 3072, "bf16", "rms", 0),
    (513, 4096, "packed", "rms", 0),
    (128, 8192, "bf16", "layer", 64),
])
def test_ln_modulate(dev, M, D, br_kind, norm, split):
    x, br, p = make(M, D, M + D, norm)
    br_q = F.quantize_rows(br)  # the branch the kernel sees: bfp16 values (exact in bf16)
    if br_kind is None:
        branch, br_ref = None, None
    elif br_kind == "bf16":
        branch, br_ref = dev_t(br_q, torch.bfloat16), br_q
    else:
        # pack the raw branch: its decode is br_q (re-encoding br_q itself is not the identity in the -128 corner)
        branch, br_ref = dev_t(F.to_bfp16(br.reshape(-1)), torch.uint8), br_q
    xo, a_p, a_d = ops.ln_modulate(dev_t(x, torch.bfloat16), dev_t(p, torch.bfloat16), branch=branch,
                                   split_row=split, norm=norm)
    xp_ref, y_ref = LN.ln_mod_ref(x, br_ref, p, split_row=split, norm=norm)
    np.testing.assert_array_equal(xo.float().cpu().numpy(), xp_ref)
    y_got = F.from_bfp16(a_p.cpu().numpy()).reshape(M, D)
    np.testing.assert_array_equal(a_d.float().cpu().numpy(), y_got)  # the bf16 A is the packed A decoded
    check_y(y_got, y_ref)


def test_a_layout_order_and_in_place(dev):
    """A-layout output = the row-block output re-ordered (same blocks); x' may overwrite x."""
    M, D = 256, 1024
    x, br, p = make(M, D, 11)
    br_t = dev_t(F.quantize_rows(br), torch.bfloat16)
    xt, pt = dev_t(x, torch.bfloat16), dev_t(p, torch.bfloat16)
    xo, a_row, a_d = ops.ln_modulate(xt, pt, branch=br_t, split_row=128)
    x2 = xt.clone()
    xo2, a_lay, a_d2 = ops.ln_modulate(x2, pt, branch=br_t, split_row=128, x_out=x2, a_order="a_layout")
    assert xo2.data_ptr() == x2.data_ptr()
    assert torch.equal(x2, xo) and torch.equal(a_d2, a_d)
    assert torch.equal(ops.dequantize(a_lay, M, D, order="a_layout"), ops.dequantize(a_row, M, D))
    # byte level: the same 9-byte blocks, moved to their a_layout positions (redline/npu_layouts.py:18-22)
    rows, cbs = np.meshgrid(np.arange(M), np.arange(D // 8), indexing="ij")
    pos = F.a_pos(rows, 8 * cbs, M, D) // 8
    want = np.empty((M * D // 8, 9), np.uint8)
    want[pos.reshape(-1)] = a_row.cpu().numpy().reshape(-1, 9)
    np.testing.assert_array_equal(a_lay.cpu().numpy(), want.reshape(-1))


def test_single_outputs(dev):
    """Each output alone equals the same output of a full call."""
    M, D = 96, 512
    x, br, p = make(M, D, 12)
    xt, pt, bt = dev_t(x, torch.bfloat16), dev_t(p, torch.bfloat16), dev_t(F.quantize_rows(br), torch.bfloat16)
    xo, a_p, a_d = ops.ln_modulate(xt, pt, branch=bt)
    _, a_p1, none1 = ops.ln_modulate(xt, pt, branch=bt, deq=False)
    _, none2, a_d1 = ops.ln_modulate(xt, pt, branch=bt, packed=False)
    assert none1 is None and none2 is None
    assert torch.equal(a_p1, a_p) and torch.equal(a_d1, a_d)


def test_full_size_dit_rows(dev):
    """The DiT hidden size at the benchmark's M (4352 x 3072, LayerNorm, bf16 branch): every row checked."""
    M, D = 4352, 3072
    x, br, p = make(M, D, 0)
    br_q = F.quantize_rows(br)
    xo, a_p, a_d = ops.ln_modulate(dev_t(x, torch.bfloat16), dev_t(p, torch.bfloat16),
                                   branch=dev_t(br_q, torch.bfloat16), split_row=4096)
    xp_ref, y_ref = LN.ln_mod_ref(x, br_q, p, split_row=4096)
    np.testing.assert_array_equal(xo.float().cpu().numpy(), xp_ref)
    check_y(F.from_bfp16(a_p.cpu().numpy()).reshape(M, D), y_ref)


def test_feeds_gemm(dev):
    """The bf16 A is a valid RL_A_BF16 operand: the GEMM on it matches the float64 product of the decoded values."""
    M, D, N = 256, 512, 256
    x, br, p = make(M, D, 13)
    _, a_p, a_d = ops.ln_modulate(dev_t(x, torch.bfloat16), dev_t(p, torch.bfloat16))
    rng = np.random.default_rng(5)
    b = ops.pack_weight(dev_t(G.linear_weight(rng, N, D), torch.float32))
    out = ops.gemm(a_d, b, N, D).float().cpu().numpy()
    ref = G.gemm_ref(F.from_bfp16(a_p.cpu().numpy()).reshape(M, D), F.decode_b(b.cpu().numpy(), D, N))
    assert G.rel_err(out, ref) <= 1e-2
    bound = 2 * np.abs(ref) * 2.0 ** -8 + 1e-4 * np.abs(ref).max()
    assert (np.abs(out - ref) <= bound).mean() > 0.999


def test_errors(dev):
    x = torch.zeros((4, 96), dtype=torch.bfloat16, device="cuda")
    p = torch.zeros((2, 192), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(L.RLError) as e:
        ops.ln_modulate(x, p)
    assert e.value.code == L.RL_ERR_SHAPE  # D % 64 != 0
    x = torch.zeros((100, 64), dtype=torch.bfloat16, device="cuda")
    p = torch.zeros((2, 128), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(L.RLError) as e:
        ops.ln_modulate(x, p, a_order="a_layout")
    assert e.value.code == L.RL_ERR_SHAPE  # A layout needs M % 128 == 0
