"""The forward.py call surface on the HIP path: one DiT block's GEMM sequence through NPU.run / gemm, checked
against the emulation; the V9 (NPU stream) output adapters; run_glue's SwiGLU stream adapters."""

import numpy as np
import pytest
import torch

from oracle import bfp16 as F
from oracle import gemm as G
from rlbfp import forward as FW
from rlbfp import ops, run_glue

pytestmark = pytest.mark.gpu


def test_block_sequence(dev):
    rng = np.random.default_rng(0)
    M, H, FF = 512, 256, 512
    x = G.activations(rng, M, H)
    mats = {"qkv": G.linear_weight(rng, 3 * H, H), "o": G.linear_weight(rng, H, H),
            "down": G.linear_weight(rng, H, FF)}
    wg, wp = G.linear_weight(rng, FF, H), G.linear_weight(rng, FF, H)
    packed = {(0, k): F.pack_b(v.T) for k, v in mats.items()}
    packed[0, "up"] = F.pack_b(F.interleave_up(wg, wp))
    w = FW.Weights.from_tensors({k: torch.from_numpy(v).cuda() for k, v in packed.items()})
    npu = FW.NPU(kn={"qkv": (H, 3 * H), "o": (H, H), "up": (H, 2 * FF), "down": (FF, H)})
    xq = F.quantize_rows(x)
    a = torch.from_numpy(xq).cuda().bfloat16()
    c_qkv = torch.empty((M, 3 * H), dtype=torch.bfloat16, device="cuda")
    FW.gemm(npu, w, "qkv", M, a, c_qkv, block=0)
    h = torch.empty((M, FF), dtype=torch.bfloat16, device="cuda")
    npu.run("up_swiglu", "atb3sw2-m4096", [a, w.b[0, "up"], h])
    npu.sync()
    dec = lambda k, K, N: F.decode_b(packed[0, k], K, N)
    check = lambda got, ref: G.rel_err(got.float().cpu().numpy(), ref)
    assert check(c_qkv, G.gemm_ref(xq, dec("qkv", H, 3 * H))) <= 1e-2
    assert check(h, G.gemm_ref(xq, dec("up", H, 2 * FF), act=G.ACT_SWIGLU)) <= 1e-2
    # the down GEMM takes H quantized along K, with NPU.a_fmt = "bf16_quantize"
    npu.a_fmt = "bf16_quantize"
    c = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    FW.gemm(npu, w, "down", M, h, c, block=0)
    npu.sync()
    hq = F.quantize_rows(h.float().cpu().numpy())
    assert check(c, G.gemm_ref(hq, dec("down", FF, H))) <= 1e-2
    assert npu.calls["qkv"] == 1 and npu.t_npu["down"] > 0


def test_v9_outputs(dev):
    """A V9 C receives the reference's stream order: ATB C order for a GEMM, the A layout for up_swiglu."""
    rng = np.random.default_rng(1)
    M, K, N = 512, 128, 1024
    A = G.activations(rng, M, K)
    W = G.linear_weight(rng, N, K)
    packed = F.pack_b(W.T)
    npu = FW.NPU()
    Aq = F.quantize_rows(A)
    a_v9 = torch.from_numpy(F.to_bfp16(F.a_layout(A))).cuda()      # the NPU's A operand
    c = FW.v9(M * N)
    npu.kn["o"] = (K, N)
    npu.run("o", "atb3d2-4096", [a_v9, torch.from_numpy(packed).cuda(), c])
    npu.sync()
    got = F.c_unlayout_atb(F.from_bfp16(c.cpu().numpy()), M, N)
    ref = G.gemm_ref(Aq, F.decode_b(packed, K, N))
    assert G.rel_err(got, ref) <= 2e-2


def test_swiglu_stream_adapters(dev):
    rng = np.random.default_rng(2)
    M, Fh = 512, 512
    gate = (rng.standard_normal((M, Fh)) * 2).astype(np.float32)
    proj = rng.standard_normal((M, Fh)).astype(np.float32)
    c_pack, gq, pq = run_glue.swiglu_pack(torch.from_numpy(gate).cuda(), torch.from_numpy(proj).cuda())
    c = np.empty((M, 2 * Fh), np.float32)
    c.reshape(M, Fh // 64, 2, 64)[:, :, 0] = gate.reshape(M, Fh // 64, 64)
    c.reshape(M, Fh // 64, 2, 64)[:, :, 1] = proj.reshape(M, Fh // 64, 64)
    np.testing.assert_array_equal(c_pack.cpu().numpy(), F.to_bfp16(F.c_layout_atb(c)))
    h = F.bf16_round(rng.standard_normal((M, Fh)).astype(np.float32))
    a_t, _ = ops.quantize(torch.from_numpy(h).cuda(), order="a_layout")
    np.testing.assert_array_equal(run_glue.swiglu_unpack(a_t, M, Fh).cpu().numpy(), F.quantize_rows(h))
