"""GPU GEMV (adaLN modulation) against the emulation, M = 1..8."""

import numpy as np
import pytest
import torch

from oracle import bfp16 as F
from oracle import gemm as G
from rlbfp import host_glue, ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,K,N,act", [(1, 3072, 18432, "silu"), (2, 4096, 16384, "silu"), (8, 192, 384, None),
                                       (3, 640, 1024, "silu"), (1, 64, 128, None), (4, 1536, 2048, "silu"),
                                       (5, 5120, 256, None), (6, 704, 512, "silu"), (7, 2560, 384, None)])
def test_gemv(dev, M, K, N, act):
    rng = np.random.default_rng(M + K)
    x = F.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    W = G.linear_weight(rng, N, K)
    packed = F.pack_b(W.T)
    got = ops.gemv(torch.from_numpy(x).cuda().bfloat16(), torch.from_numpy(packed).cuda(), N, act=act)
    ref = G.gemv_ref(x, F.decode_b(packed, K, N), act=act or "none")
    err = G.rel_err(got.float().cpu().numpy(), ref)
    assert err <= 1e-2, err
    d = np.abs(got.float().cpu().numpy() - ref)
    assert (d <= 2 * np.abs(ref) * 2.0 ** -8 + 1e-5 * np.abs(ref).max()).mean() > 0.999


def test_modulation_names(dev):
    rng = np.random.default_rng(1)
    K, N = 3072, 18432
    W = G.linear_weight(rng, N, K)
    wp = host_glue.pack_linear(torch.from_numpy(W))
    te = F.bf16_round(rng.standard_normal((2, K)).astype(np.float32))
    te[1] = 0.0                                   # rows [t, 0] as the reference's temb
    y = host_glue.modulation({"modulation.1.weight": wp, "modulation.N": N}, torch.from_numpy(te))
    ref = G.gemv_ref(te, F.decode_b(wp.cpu().numpy(), K, N))
    assert G.rel_err(y.float().cpu().numpy(), ref) <= 1e-2
    assert (y[1] == 0).all()                      # silu(0) = 0
