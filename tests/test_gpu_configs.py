"""The configurations of the reference's GEMM path at their full sizes (seed 0, the draw order activations,
weights, epilogue vectors): the GPU result against the emulation (decoded operands, float64 products, the fused
epilogue, bf16) on every row for the headline FFN pair and on sampled rows elsewhere, the grouped launch
bit-identical to single launches, and the packed H of the FFN pair re-encoding to itself (but for the -128 corner).
Weights are packed on the GPU (byte-identical to the CPU packer, checked in test_gpu_quantize.py) and decoded on the
CPU for the reference."""

import numpy as np
import pytest
import torch

from oracle import bfp16 as F
from oracle import gemm as G
from rlbfp import ops

pytestmark = pytest.mark.gpu
TOL = 1e-2


def cuda(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda().to(dtype)


def sample_rows(rng, M, n=48):
    """Rows at both ends, around the 128/224/256-row tile boundaries and the 4096-row launch split, and random."""
    edges = [0, 1, 127, 128, 223, 224, 255, 256, 4095, 4096, M - 129, M - 128, M - 1]
    rows = np.concatenate([np.array([r for r in edges if 0 <= r < M]), rng.integers(0, M, n)])
    return np.unique(rows)


def check_rows(out, rows, ref):
    got = out[torch.from_numpy(rows).cuda()].float().cpu().numpy()
    err = G.rel_err(got, ref)
    assert err <= TOL, f"rel err {err}"
    d = np.abs(got.astype(np.float64) - ref)
    assert (d <= 2 * np.abs(ref) * 2.0 ** -8 + 1e-4 * np.abs(ref).max()).mean() > 0.999


def packed_weight(rng, N, K):
    W = G.linear_weight(rng, N, K)
    p = ops.pack_weight(cuda(W, torch.float32))
    return p, F.decode_b(p.cpu().numpy(), K, N)


def packed_up(rng, F_, K):
    wg, wp = G.linear_weight(rng, F_, K), G.linear_weight(rng, F_, K)
    p = ops.pack_weight(ops.interleave_up(cuda(wg, torch.float32), cuda(wp, torch.float32)))
    return p, F.decode_b(p.cpu().numpy(), K, 2 * F_)


def test_config2_qkv_bias_outliers(dev):
    """DiT joint-attention QKV: M=4352, K=3072, N=9216, 1% of channels x20, bias epilogue; quantize-on-load and the
    separate quantize pass give identical results."""
    rng = np.random.default_rng(0)
    M, K, N = 4352, 3072, 9216
    A = G.activations(rng, M, K, outliers=0.01)
    bw, Bq = packed_weight(rng, N, K)
    bias = (rng.standard_normal(N) * 0.02).astype(np.float32)
    a = cuda(A, torch.bfloat16)
    _, aq = ops.quantize(a, deq=True)
    out = ops.gemm(aq, bw, N, K, bias=cuda(bias, torch.float32))
    out_q = ops.gemm(a, bw, N, K, a_fmt="bf16_quantize", bias=cuda(bias, torch.float32))
    assert torch.equal(out, out_q)
    rows = sample_rows(rng, M)
    check_rows(out, rows, G.gemm_ref(F.quantize_rows(A[rows]), Bq, bias=bias))


def check_all_rows(out, ref_fn, M, chunk=256):
    """Every row of a GPU output against the emulation, computed on the host chunk by chunk (ref_fn(r0, r1) -> the
    emulated rows r0..r1-1): max |got - ref| / max |ref| <= 1e-2 over the whole output, and >= 99.9% of the elements
    within 2 bf16 ulps (plus the fp32 summation difference). Returns (rel err, fraction within the element bound)."""
    worst, scale, n_ok, n = 0.0, 0.0, 0, 0
    refs = []
    for r0 in range(0, M, chunk):
        r1 = min(M, r0 + chunk)
        ref = ref_fn(r0, r1)
        got = out[r0:r1].float().cpu().numpy().astype(np.float64)
        d = np.abs(got - ref)
        worst, scale = max(worst, d.max()), max(scale, np.abs(ref).max())
        refs.append((d, np.abs(ref)))
    for d, aref in refs:
        n_ok += int((d <= 2 * aref * 2.0 ** -8 + 1e-4 * scale).sum())
        n += d.size
    err, frac = worst / scale, n_ok / n
    assert err <= TOL, f"rel err {err}"
    assert frac > 0.999, f"{n - n_ok} of {n} elements off"
    return err, frac


def test_config3_ffn_pair(dev):
    """DiT FFN pair: up 4352x3072x(2x12288) SwiGLU with re-quantized H, then down 4352x12288x3072 with gate and
    residual. Every row of both outputs is compared with the emulation (float64 products on the host, chunked by
    rows); the down GEMM is checked on the GPU's own H."""
    rng = np.random.default_rng(0)
    M, K, FF = 4352, 3072, 12288
    X = G.activations(rng, M, K)
    up, Bup = packed_up(rng, FF, K)
    down, Bdown = packed_weight(rng, K, FF)
    res = F.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    gate = rng.standard_normal(K).astype(np.float32)
    _, xq = ops.quantize(cuda(X, torch.bfloat16), deq=True)
    h = ops.gemm(xq, up, 2 * FF, K, act="swiglu", quantize_out=True)
    out = ops.gemm(h, down, K, FF, gate=cuda(gate, torch.float32), residual=cuda(res, torch.bfloat16))
    Xq = F.quantize_rows(X).astype(np.float64)
    Bup, Bdown = np.asarray(Bup, np.float64), np.asarray(Bdown, np.float64)
    check_all_rows(h, lambda r0, r1: G.gemm_ref(Xq[r0:r1], Bup, act=G.ACT_SWIGLU, quantize_out=True), M)
    H = h.float().cpu().numpy()
    # H is made of bfp16 blocks: re-encoding changes nothing but the -128 corner (a block whose largest magnitude
    # is -2^k re-encodes one exponent up)
    blocks = H.reshape(-1, 8).astype(np.float64)
    same = (F.quantize_rows(H).reshape(-1, 8) == blocks).all(1)
    vmax = blocks[np.arange(len(blocks)), np.abs(blocks).argmax(1)]
    corner = (vmax < 0) & (np.frexp(-vmax)[0] == 0.5)
    assert same[~corner].all()
    H64 = H.astype(np.float64)
    check_all_rows(out, lambda r0, r1: G.gemm_ref(H64[r0:r1], Bdown, gate=gate, residual=res[r0:r1]), M)


def test_config4_text_encoder_mlp(dev):
    """Text-encoder prefill MLP: M=512 RMS-normalised rows, up K=4096 N=2x12288 SwiGLU, down K=12288 N=4096."""
    rng = np.random.default_rng(0)
    M, K, FF = 512, 4096, 12288
    X = G.activations(rng, M, K, rms_rows=True)
    up, Bup = packed_up(rng, FF, K)
    down, Bdown = packed_weight(rng, K, FF)
    _, xq = ops.quantize(cuda(X, torch.bfloat16), deq=True)
    h = ops.gemm(xq, up, 2 * FF, K, act="swiglu", quantize_out=True)
    out = ops.gemm(h, down, K, FF)
    rows = sample_rows(rng, M, n=24)
    check_rows(h, rows, G.gemm_ref(F.quantize_rows(X[rows]), Bup, act=G.ACT_SWIGLU, quantize_out=True))
    check_rows(out, rows, G.gemm_ref(h[torch.from_numpy(rows).cuda()].float().cpu().numpy(), Bdown))


def test_config5_grouped_streams(dev):
    """One DiT block at 1024x1024: the image (M=4096) and text (M=256) streams' QKV projections with separate
    weights as one grouped launch, identical to two single launches; the modulation GEMV at M=1, K=3072, N=18432."""
    rng = np.random.default_rng(0)
    K, N = 3072, 9216
    streams = []
    for M in (4096, 256):
        A = G.activations(rng, M, K)
        bw, Bq = packed_weight(rng, N, K)
        _, aq = ops.quantize(cuda(A, torch.bfloat16), deq=True)
        streams.append((M, A, bw, Bq, aq))
    outs = ops.gemm_grouped([ops.GemmSpec(aq, bw, N, K) for (_, _, bw, _, aq) in streams])
    for (M, A, bw, Bq, aq), o in zip(streams, outs):
        assert torch.equal(o, ops.gemm(aq, bw, N, K))
        rows = sample_rows(rng, M, n=16)
        check_rows(o, rows, G.gemm_ref(F.quantize_rows(A[rows]), Bq))
    temb = F.bf16_round(rng.standard_normal((1, K)).astype(np.float32))
    wm, Bm = packed_weight(rng, 6 * K, K)
    y = ops.gemv(cuda(temb, torch.bfloat16), wm, 6 * K, act="silu")
    assert G.rel_err(y.float().cpu().numpy(), G.gemv_ref(temb, Bm)) <= TOL


@pytest.mark.parametrize("op", ["out_proj", "up_swiglu", "down"])
def test_config5_grouped_launches(dev, op):
    """Config 5's other grouped launches at full size, image (M=4096) and text (M=256) streams with separate weights:
    the out-projection (K = N = 3072), the SwiGLU up GEMM with re-quantized H (K = 3072, N = 2 x 12288) and the down
    GEMM (K = 12288, N = 3072), each checked on sampled rows against the emulation and bit-identical to single
    launches."""
    rng = np.random.default_rng({"out_proj": 1, "up_swiglu": 2, "down": 3}[op])
    K, FF = 3072, 12288
    Kop, N = {"out_proj": (K, K), "up_swiglu": (K, 2 * FF), "down": (FF, K)}[op]
    kind = "swiglu" if op == "up_swiglu" else None
    streams = []
    for M in (4096, 256):
        A = G.activations(rng, M, Kop)
        bw, Bq = packed_up(rng, FF, K) if kind else packed_weight(rng, N, Kop)
        _, aq = ops.quantize(cuda(A, torch.bfloat16), deq=True)
        streams.append((M, A, bw, Bq, aq))
    specs = [ops.GemmSpec(aq, bw, N, Kop, act=kind, quantize_out=kind is not None) for (_, _, bw, _, aq) in streams]
    outs = ops.gemm_grouped(specs)
    for (M, A, bw, Bq, aq), o in zip(streams, outs):
        assert torch.equal(o, ops.gemm(aq, bw, N, Kop, act=kind, quantize_out=kind is not None, split=False))
        rows = sample_rows(rng, M, n=16)
        ref = G.gemm_ref(F.quantize_rows(A[rows]), Bq, act=G.ACT_SWIGLU if kind else G.ACT_NONE,
                         quantize_out=kind is not None)
        check_rows(o, rows, ref)


def test_packer_full_size_against_c_restatement(dev):
    """The GPU weight packer at config 3's up-projection size (W_up 2 x 12288 x 3072 interleaved, 84.9 MB packed)
    against the oracle's integer C encoder applied to the b_layout of B = W.T, compared 2048 columns (16 N tiles) at a
    time: every byte equal."""
    from oracle import bfp16_c as C
    rng = np.random.default_rng(0)
    K, FF = 3072, 12288
    wg, wp = G.linear_weight(rng, FF, K), G.linear_weight(rng, FF, K)
    W = F.interleave_up(wg, wp).T.copy()          # the Linear weight (2 FF, K) whose B = W.T is interleave_up's
    got = ops.pack_weight(cuda(W, torch.float32)).cpu().numpy()
    per = K * 2048 // 8 * 9                        # bytes of 2048 columns: N tiles are contiguous in the stream
    for c0 in range(0, 2 * FF, 2048):
        want = C.to_bfp16(F.b_layout(np.ascontiguousarray(W[c0:c0 + 2048].T)))
        np.testing.assert_array_equal(got[c0 // 2048 * per:(c0 // 2048 + 1) * per], want)


def test_gemv_against_unquantized_reference_math(dev):
    """The modulation GEMV at config 5's size against the reference's own math, linear(silu(te), W) with an
    unquantized activation in float64 (redline/host_glue.py:26-28, :43-44) on the packed weights' values: the
    activation encoding the GPU applies (bfp16 blocks of 8) stays within the 1e-2 bar."""
    rng = np.random.default_rng(5)
    K, N = 3072, 18432
    temb = F.bf16_round(rng.standard_normal((1, K)).astype(np.float32))
    wm, Bm = packed_weight(rng, N, K)
    y = ops.gemv(cuda(temb, torch.bfloat16), wm, N, act="silu").float().cpu().numpy()
    ref = G.silu(temb.astype(np.float64)) @ Bm.astype(np.float64)
    assert G.rel_err(y, ref) <= TOL
    assert G.corr(y, ref) > 0.999
