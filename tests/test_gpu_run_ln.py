"""The run_ln call surface on the GPU (redline-tiny_amd/rlbfp/run_ln.py), exercised the way redline/run_ln.py:89-114
(check_random) and redline/vlm_run.py:73-92 (check_rms) exercise the NPU artifacts: x and the branch in config3's
C-stream order, A back in the A layout, checked against the oracle (oracle/ln.py)."""

import numpy as np
import pytest
import torch

from oracle import bfp16 as F
from oracle import gemm as G
from oracle import ln as LN
from rlbfp import forward, run_ln

pytestmark = pytest.mark.gpu


def tt(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def check(xp, y, xr, yr):
    np.testing.assert_array_equal(xp, xr)
    assert G.rel_err(y, yr) <= 1e-2 and G.corr(y, yr) > 0.9999
    assert (y == F.quantize_rows(yr.astype(np.float32))).mean() > 0.999


@pytest.mark.parametrize("M,S", [(512, 0), (1024, 3)])
def test_check_random(dev, M, S):
    Dm = 4096
    rng = np.random.default_rng(0)
    x = rng.standard_normal((M, Dm)).astype(np.float32) * 3
    x[:, rng.integers(0, Dm, 8)] *= 40
    br = rng.standard_normal((M, Dm)).astype(np.float32)
    g = np.tanh(rng.standard_normal((2, Dm))).astype(np.float32)
    sc = (1 + 0.3 * rng.standard_normal((2, Dm))).astype(np.float32)
    xc, brc, p = run_ln.ln_pack_x(tt(x)), run_ln.ln_pack_br(tt(br)), run_ln.ln_params(tt(g), tt(sc))
    # the packed streams are the oracle's bytes
    np.testing.assert_array_equal(brc.cpu().numpy(), F.to_bfp16(F.c_layout_atb(br)))
    np.testing.assert_array_equal(xc.float().cpu().numpy(), F.c_layout_atb(F.bf16_round(x)))
    art = f"glue-ln-m{M}-s{S}"
    xo, ao, us = run_ln.ln_run(art, xc, brc, p, iters=3, warmup=1)
    assert len(us) == 3 and all(u > 0 for u in us)
    xp, y = run_ln.ln_unpack(xo, ao, M)
    xr, yr = LN.ln_mod_ref(F.bf16_round(x), F.quantize_rows(br), LN.ln_params(g, sc), split_row=S * 128)
    check(xp.cpu().numpy(), y.cpu().numpy(), xr, yr)
    # the same op through NPU.run, into caller-allocated buffers
    npu = forward.NPU()
    xo2, ao2 = torch.zeros_like(xc), forward.v9(M * Dm)
    npu.run("ln_mod", art, [xc, brc, p, xo2, ao2])
    npu.sync()
    assert torch.equal(xo2, xo) and torch.equal(ao2, ao)
    assert npu.calls["ln_mod"] == 1


def test_check_rms(dev):
    """RMSNorm with a massive-activation channel and g = 1 (rms_params), as check_rms draws it."""
    M, Dm = 512, 4096
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((M, Dm)) * 3).astype(np.float32)
    x[:, 7] += 40
    br = rng.standard_normal((M, Dm)).astype(np.float32)
    w = (1 + 0.2 * rng.standard_normal(Dm)).astype(np.float32)
    p = LN.rms_params(w)
    xo, ao, _ = run_ln.ln_run("vlm-rms-m512", run_ln.ln_pack_x(tt(x)), run_ln.ln_pack_br(tt(br)),
                              tt(p, torch.bfloat16).reshape(-1))
    xp, y = run_ln.ln_unpack(xo, ao, M)
    xr, yr = LN.ln_mod_ref(F.bf16_round(x), F.quantize_rows(br), p, norm="rms")
    check(xp.cpu().numpy(), y.cpu().numpy(), xr, yr)


def test_native_forms(dev):
    """Row-major bf16 X / XO / branch and a bf16 AO (the next GEMM's operand) give the same values."""
    M, Dm = 512, 1024
    rng = np.random.default_rng(3)
    x = tt(rng.standard_normal((M, Dm)) * 2, torch.bfloat16)
    br_raw = rng.standard_normal((M, Dm)).astype(np.float32)
    br = tt(F.quantize_rows(br_raw), torch.bfloat16)  # the values the packed C-stream branch decodes to
    p = run_ln.ln_params(tt(np.tanh(rng.standard_normal((2, Dm)))), tt(1 + 0.1 * rng.standard_normal((2, Dm))))
    xo, ao = torch.empty_like(x), torch.empty_like(x)
    run_ln.ln_fused("glue-ln-m512-s1", x, br, p, xo, ao)
    xo_s, ao_s, _ = run_ln.ln_run("glue-ln-m512-s1", run_ln.ln_pack_x(x), run_ln.ln_pack_br(tt(br_raw)), p)
    xp, y = run_ln.ln_unpack(xo_s, ao_s, M)
    assert torch.equal(xo.float(), xp) and torch.equal(ao.float(), y)
