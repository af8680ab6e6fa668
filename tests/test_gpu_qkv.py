"""GPU QKV post pass (rl_qkv_post) against the oracle (oracle/qkv.py).

V is pure re-blocking and quantization of bf16 inputs: its tiles are bit-exact. Q and K are computed in fp32 on the
GPU and in float64 by the oracle, then quantized: at least 99.9% of the stored values equal the oracle's quantized
values and every other one is within one quantization step of its block; per head the correlation exceeds 0.999,
the bar of redline/run_qkv.py:137. The head-major bf16 outputs (V transposed) equal the tiles' decoded values bit for
bit."""

import numpy as np
import pytest
import torch

from oracle import bfp16 as F
from oracle import gemm as G
from oracle import qkv as QK
from rlbfp import ops, run_qkv

pytestmark = pytest.mark.gpu


def tt(a, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to("cuda").to(dtype)


def make(M, H, seed):
    rng = np.random.default_rng(seed)
    C = F.bf16_round((rng.standard_normal((M, 3 * H * 128)) * 2).astype(np.float32))
    C[:, rng.integers(0, 3 * H * 128, 6)] *= 30  # a few large channels
    C = F.bf16_round(C)
    ang = rng.uniform(-np.pi, np.pi, (M, 64))
    cos, sin = F.bf16_round(np.cos(ang).astype(np.float32)), F.bf16_round(np.sin(ang).astype(np.float32))
    wqc = F.bf16_round(((1 + 0.1 * rng.standard_normal(128)) * QK.C_LOG2).astype(np.float32))
    wk = F.bf16_round((1 + 0.1 * rng.standard_normal(128)).astype(np.float32))
    return C, cos, sin, wqc, wk


def close_values(got, ref_q):
    """got / ref_q: quantized values of the same blocks (last axis = 8-value blocks' axis already flattened)."""
    eq = got == ref_q
    assert eq.mean() > 0.999, f"{(~eq).sum()} of {eq.size} differ"
    m = np.abs(np.stack([got, ref_q])).reshape(2, -1, 8).max(2).max(0)
    step = 2.0 ** (np.floor(np.log2(np.maximum(m, 1e-30))) - 6)
    assert (np.abs(got - ref_q).reshape(-1, 8).max(1) <= step * 1.0000001).all()


def check_heads(qt, kvt, C, cos, sin, wqc, wk, H, heads):
    Q, K, V = QK.qkv_post_ref(C, cos, sin, wqc, wk, H)
    Qq, Kq, Vq = QK.quantize_qkv(Q, K, V)
    q_np, kv_np = qt.cpu().numpy(), kvt.cpu().numpy()
    _, kv_ref = QK.tiles(Q[heads], K[heads], V[heads])
    for i, h in enumerate(heads):
        a, b, c = QK.unpack_head(q_np, kv_np, h)
        close_values(a, Qq[h])
        close_values(b, Kq[h])
        np.testing.assert_array_equal(kv_np[h, :, 1], kv_ref[i, :, 1])  # V tiles bit-exact
        assert G.corr(a, Q[h]) > 0.999 and G.corr(b, K[h]) > 0.999
    return Qq, Kq, Vq


@pytest.mark.parametrize("M,H", [(64, 1), (128, 2), (640, 5)])
def test_qkv_post(dev, M, H):
    C, cos, sin, wqc, wk = make(M, H, M + H)
    qt, kvt, q, k, v = ops.qkv_post(tt(C), tt(cos), tt(sin), tt(wqc), tt(wk), H, tiles=True, native=True)
    Qq, Kq, Vq = check_heads(qt, kvt, C, cos, sin, wqc, wk, H, list(range(H)))
    # native outputs are the tiles' decoded values
    q_np, kv_np = qt.cpu().numpy(), kvt.cpu().numpy()
    for h in range(H):
        a, b, c = QK.unpack_head(q_np, kv_np, h)
        np.testing.assert_array_equal(q[h].float().cpu().numpy(), a)
        np.testing.assert_array_equal(k[h].float().cpu().numpy(), b)
        np.testing.assert_array_equal(v[h].float().cpu().numpy(), c.T)  # V^T
    np.testing.assert_array_equal(v.float().cpu().numpy(), Vq.transpose(0, 2, 1))


def test_outputs_alone_and_pad_rows(dev):
    """Tiles alone and native alone give the same values as together; zero (pad) rows give zero Q, K, V."""
    M, H = 256, 3
    C, cos, sin, wqc, wk = make(M, H, 9)
    C[64:80] = 0.0
    args = (tt(C), tt(cos), tt(sin), tt(wqc), tt(wk), H)
    qt, kvt, q, k, v = ops.qkv_post(*args, tiles=True, native=True)
    qt2, kvt2, n1, n2, n3 = ops.qkv_post(*args, tiles=True, native=False)
    n4, n5, q3, k3, v3 = ops.qkv_post(*args, tiles=False, native=True)
    assert n1 is None and n2 is None and n3 is None and n4 is None and n5 is None
    assert torch.equal(qt, qt2) and torch.equal(kvt, kvt2)
    assert torch.equal(q, q3) and torch.equal(k, k3) and torch.equal(v, v3)
    for x in (q, k):
        assert (x[:, 64:80] == 0).all()
    assert (v[:, :, 64:80] == 0).all()


def test_full_size_qkv_config(dev):
    """The QKV GEMM output of the 4352-token, 24-head (hidden 3072) configuration; heads 0, 11 and 23 checked in
    full, V of every head bit-exact."""
    M, H = 4352, 24
    C, cos, sin, wqc, wk = make(M, H, 0)
    qt, kvt, q, k, v = ops.qkv_post(tt(C), tt(cos), tt(sin), tt(wqc), tt(wk), H, tiles=True, native=True)
    check_heads(qt, kvt, C, cos, sin, wqc, wk, H, [0, 11, 23])
    V = np.stack([C[:, 2 * H * 128 + h * 128:2 * H * 128 + (h + 1) * 128] for h in range(H)])
    Vt = np.ascontiguousarray(V.transpose(0, 2, 1))
    Vq = F.quantize_rows(Vt.reshape(-1, M)).reshape(Vt.shape).transpose(0, 2, 1)
    np.testing.assert_array_equal(v.float().cpu().numpy(), Vq.transpose(0, 2, 1))


def test_qkv32_npu_reference_formats(dev):
    """run_qkv's random check (redline/run_qkv.py:111-140) through the mirror: the C stream in, the table format for
    cos/sin and the weights, Q and KV tiles out, unpack_head; 32 heads of the reference's hidden 4096."""
    M, H = 512, 32
    rng = np.random.default_rng(0)
    ang = rng.uniform(-np.pi, np.pi, (M, 64))
    cos, sin = F.bf16_round(np.cos(ang).astype(np.float32)), F.bf16_round(np.sin(ang).astype(np.float32))
    wq, wk = 1 + 0.1 * rng.standard_normal(128), 1 + 0.1 * rng.standard_normal(128)
    C = rng.standard_normal((M, 3 * 4096)).astype(np.float32)
    C[100:164] = 0  # pad rows
    wqc = F.bf16_round((wq * QK.C_LOG2).astype(np.float32))
    wk = F.bf16_round(wk.astype(np.float32))
    cin = ops.quantize(tt(C, torch.float32), order="c_atb")[0]
    tabs = run_qkv.qkv_tables(tt(cos), tt(sin), tt(wqc), tt(wk))
    q, kv, ms = run_qkv.qkv32_npu("glue-qkv32-m512", cin, tabs, M, iters=3)
    assert ms is not None and ms > 0
    assert q.shape == (H, M // 64, 9216) and kv.shape == (H, M // 64, 2, 9216)
    cq = F.quantize_rows(C)  # the C stream's values (blocks of 8 columns of a row)
    for h in (0, 17, 31):
        Qg, Kg, Vg = (x.cpu().numpy() for x in run_qkv.unpack_head(q, kv, h))
        refs = (QK.rms_rope(cq[:, h * 128:(h + 1) * 128].astype(np.float64), wqc, cos, sin),
                QK.rms_rope(cq[:, 4096 + h * 128:4096 + (h + 1) * 128].astype(np.float64), wk, cos, sin),
                cq[:, 8192 + h * 128:8192 + (h + 1) * 128])
        for got, ref in zip((Qg, Kg, Vg), refs):
            assert G.corr(got, ref) > 0.999
            assert np.abs(got[100:164]).max() == 0.0
        close_values(Qg, F.quantize_rows(refs[0].astype(np.float32)))
