"""GPU GEMM against the CPU emulation (decoded operands, float64 matmul, epilogue, bf16): max |got - ref| /
max |ref| <= 1e-2 (the reference's error metric, redline/run_glue.py:158-159), and element-wise within a bf16 ulp
plus the fp32 summation difference."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import bfp16 as F
from oracle import gemm as G
from rlbfp import ops

pytestmark = pytest.mark.gpu
TOL = 1e-2


def dev_t(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def setup(M, K, N, seed, outliers=0.0):
    rng = np.random.default_rng(seed)
    A = G.activations(rng, M, K, outliers=outliers)
    W = G.linear_weight(rng, N, K)
    packed = F.pack_b(W.T)
    return rng, A, packed, F.quantize_rows(A), F.decode_b(packed, K, N)


def check(got, ref, tol=TOL):
    got = got.float().cpu().numpy()
    assert got.shape == ref.shape
    err = G.rel_err(got, ref)
    assert err <= tol, f"rel err {err}"
    # element-wise: within 2 bf16 ulps of the reference value, or tiny relative to the output scale
    d = np.abs(got.astype(np.float64) - ref)
    bound = 2 * np.abs(ref) * 2.0 ** -8 + 1e-4 * np.abs(ref).max()
    assert (d <= bound).mean() > 0.999, f"{(d > bound).sum()} elements off"
    return err


@pytest.mark.parametrize("M,K,N", [(256, 64, 256), (1, 64, 128), (100, 128, 384), (257, 192, 256),
                                   (512, 512, 640), (4352, 256, 256)])
def test_plain_shapes(dev, M, K, N):
    rng, A, packed, Aq, Bq = setup(M, K, N, M + K + N)
    a = dev_t(Aq, torch.bfloat16)
    out = ops.gemm(a, dev_t(packed, torch.uint8), N, K)
    check(out, G.gemm_ref(Aq, Bq))


def test_output_canary_and_ldc(dev):
    """Writes stay inside the (M, N) window of a wider output; rows past M are not written."""
    M, K, N = 130, 128, 256
    rng, A, packed, Aq, Bq = setup(M, K, N, 3)
    big = torch.full((M + 5, N + 64), 7.0, dtype=torch.bfloat16, device="cuda")
    ops.gemm(dev_t(Aq, torch.bfloat16), dev_t(packed, torch.uint8), N, K, out=big[:M, :N])
    check(big[:M, :N], G.gemm_ref(Aq, Bq))
    assert (big[:, N:] == 7.0).all() and (big[M:, :] == 7.0).all()


@pytest.mark.parametrize("M,K,N", [(256, 192, 256), (128, 4096, 384)])
@pytest.mark.parametrize("workspace", [True, False])
@pytest.mark.parametrize("a_fmt", ["bf16_quantize", "packed_rowblock", "packed_a_layout"])
def test_a_formats_agree(dev, a_fmt, workspace, M, K, N):
    """Every A format computes on the same bfp16 values: results identical to the bf16 (pre-quantized) path, whether
    the staged bf16 copy of A lives in the caller's workspace or in the library's own stream-ordered allocation.
    128 x 4096 x 384 is a shape the planner splits along K when given a workspace: with one, every format runs the
    split (the bf16 path's split bits); without one (rl_bfp16_gemm), every format runs whole K (its whole-K bits)."""
    rng, A, packed, Aq, Bq = setup(M, K, N, 4, outliers=0.01)
    b = dev_t(packed, torch.uint8)
    if K == 4096:
        assert ops.gemm_workspace_bytes(M, N, K) > 0, "the case is meant to split"
    ref = ops.gemm(dev_t(Aq, torch.bfloat16), b, N, K, split=workspace)
    if a_fmt == "bf16_quantize":
        a = dev_t(A, torch.bfloat16)
    elif a_fmt == "packed_rowblock":
        a = dev_t(F.to_bfp16(A.reshape(-1)), torch.uint8)
    else:
        a = dev_t(F.to_bfp16(F.a_layout(A)), torch.uint8)
    got = ops.gemm(a, b, N, K, M=M, a_fmt=a_fmt, workspace=workspace)
    assert torch.equal(got, ref)
    check(got, G.gemm_ref(Aq, Bq))


def test_bias_gelu(dev):
    M, K, N = 200, 128, 384
    rng, A, packed, Aq, Bq = setup(M, K, N, 5)
    bias = (rng.standard_normal(N) * 0.5).astype(np.float32)
    out = ops.gemm(dev_t(Aq, torch.bfloat16), dev_t(packed, torch.uint8), N, K, bias=dev_t(bias, torch.float32),
                   act="gelu_tanh")
    check(out, G.gemm_ref(Aq, Bq, bias=bias, act=G.ACT_GELU_TANH))


def test_swiglu_interleaved(dev):
    M, K, Fh = 300, 128, 256
    rng = np.random.default_rng(6)
    A = G.activations(rng, M, K)
    wg, wp = G.linear_weight(rng, Fh, K), G.linear_weight(rng, Fh, K)
    packed = F.pack_b(F.interleave_up(wg, wp))
    Aq, Bq = F.quantize_rows(A), F.decode_b(packed, K, 2 * Fh)
    bias = (rng.standard_normal(2 * Fh) * 0.1).astype(np.float32)
    for kw in ({}, {"bias": bias}):
        out = ops.gemm(dev_t(Aq, torch.bfloat16), dev_t(packed, torch.uint8), 2 * Fh, K, act="swiglu",
                       **{k: dev_t(v, torch.float32) for k, v in kw.items()})
        assert out.shape == (M, Fh)
        check(out, G.gemm_ref(Aq, Bq, act=G.ACT_SWIGLU, **kw))


@pytest.mark.parametrize("M,K,N,quant,scale", [
    (300, 128, 2 * 256, False, 1.0),        # rows past M in the last tile
    (1000, 256, 2 * 1024, True, 1.0),       # re-quantized output
    (512, 128, 2 * 512, True, 2.0 ** 62),   # output blocks past the float fast path (E > 237: the integer encoder)
])
def test_register_epilogue_matches_staged(dev, M, K, N, quant, scale):
    """The FFN up GEMMs (SwiGLU without bias, gate or residual, row-major C) run the 4-wave kernel's register epilogue
    (transposed accumulators, 8-column blocks assembled by row swaps); a zero bias sends the same GEMM through the
    LDS-staged epilogue (acc + 0 is acc bit for bit: an MFMA sum started from +0 is never -0). Bit-identical, and both
    against the emulation."""
    rng = np.random.default_rng(M + N)
    A = G.activations(rng, M, K) * np.float32(scale)
    Fh = N // 2
    packed = F.pack_b(F.interleave_up(G.linear_weight(rng, Fh, K), G.linear_weight(rng, Fh, K)))
    Aq = F.quantize_rows(A)
    a, b = dev_t(Aq, torch.bfloat16), dev_t(packed, torch.uint8)
    reg = ops.gemm(a, b, N, K, act="swiglu", quantize_out=quant)
    staged = ops.gemm(a, b, N, K, act="swiglu", quantize_out=quant, bias=torch.zeros(N, device="cuda"))
    assert torch.equal(reg, staged)
    assert torch.isfinite(reg.float()).all()
    if scale == 1.0:
        check(reg, G.gemm_ref(Aq, F.decode_b(packed, K, N), act=G.ACT_SWIGLU, quantize_out=quant), tol=2e-2)
    else:
        o = reg.float().cpu().numpy()
        assert np.abs(o).max() >= 2.0 ** 111  # the blocks the integer encoder serves
        assert (F.quantize_rows(o) == o).mean() > 0.999


def test_register_epilogue_ffn_up_full(dev):
    """The FFN up GEMM at full size (4352 x 3072 x 2 x 12288: 512-row tiles over rows 0..4095, then 256-row tiles)
    through the register epilogue, bit-identical to the LDS-staged one (zero bias)."""
    M, K, N = 4352, 3072, 2 * 12288
    g = torch.Generator(device="cuda").manual_seed(11)
    x = ops.quantize(torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16), deq=True)[1]
    w = ops.pack_weight(ops.interleave_up(torch.randn((N // 2, K), generator=g, device="cuda") * 0.02,
                                          torch.randn((N // 2, K), generator=g, device="cuda") * 0.02).contiguous())
    reg = ops.gemm(x, w, N, K, act="swiglu", quantize_out=True)
    staged = ops.gemm(x, w, N, K, act="swiglu", quantize_out=True, bias=torch.zeros(N, device="cuda"))
    assert torch.equal(reg, staged)


def test_gate_residual_split(dev):
    M, K, N = 384, 256, 256
    rng, A, packed, Aq, Bq = setup(M, K, N, 7)
    res = F.bf16_round(rng.standard_normal((M, N)).astype(np.float32))
    gate = rng.standard_normal((2, N)).astype(np.float32)
    out = ops.gemm(dev_t(Aq, torch.bfloat16), dev_t(packed, torch.uint8), N, K, gate=dev_t(gate, torch.float32),
                   gate_split_row=128, residual=dev_t(res, torch.bfloat16))
    check(out, G.gemm_ref(Aq, Bq, gate=gate, gate_split_row=128, residual=res))


def test_quantize_out(dev):
    """Re-quantized output: every 8-column block is an exact bfp16 block (re-encoding it changes nothing except in
    the -128 corner) and the values match the emulation."""
    M, K, N = 256, 128, 256
    rng, A, packed, Aq, Bq = setup(M, K, N, 8)
    out = ops.gemm(dev_t(Aq, torch.bfloat16), dev_t(packed, torch.uint8), N, K, quantize_out=True).float()
    o = out.cpu().numpy()
    check(out, G.gemm_ref(Aq, Bq, quantize_out=True), tol=2e-2)
    blocks = o.reshape(-1, 8).astype(np.float64)
    raw = F.to_bfp16(o.reshape(-1))
    same = (F.from_bfp16(raw).reshape(-1, 8) == blocks).all(1)
    # the only blocks a re-encode may change: a -128 element, i.e. the largest magnitude is -2^k and
    # the re-encode moves it to exponent field k + 127 with q = -64
    i = np.abs(blocks).argmax(1)
    vmax = blocks[np.arange(len(blocks)), i]
    m, e = np.frexp(-vmax)
    corner = (vmax < 0) & (m == 0.5)
    q_new = raw.reshape(-1, 9)[:, 1:].view(np.int8)[np.arange(len(blocks)), i]
    assert same[~corner].all()
    assert (q_new[~same] == -64).all()


def test_requantize_exponent_bounds(dev):
    """The epilogue's re-quantize on blocks at and around the float fast path's bounds (block exponents 7/8 and
    237/238), with bf16 subnormal elements beside an E = 7 maximum: gate 0 makes the output the residual itself, so
    the result must equal the encoder's blocks of the residual exactly."""
    M, K, N = 128, 64, 128
    rng, A, packed, Aq, Bq = setup(M, K, N, 21)
    rows = []
    for e in (1, 6, 7, 8, 9, 120, 236, 237, 238, 250):
        step = 2.0 ** (e - 133)
        rows.append((rng.integers(-127, 127, 8) + 0.5) * step)
        rows.append(np.array([127.5, -127.5, 64.5, -64.5, 0.5, -0.5, 1.5, -2.5]) * step)
    for e in (7, 8):
        rows.append(np.array([1.5 * 2.0 ** (e - 127), 2**-127, -2**-127, 1.5 * 2**-127, -1.5 * 2**-127,
                              1.75 * 2**-127, 2**-128, -1.5 * 2**-128]))
    blocks = F.bf16_round(np.concatenate(rows).astype(np.float32).reshape(-1, 8))
    res = np.tile(blocks, (M * N // 8 // len(blocks) + 1, 1))[: M * N // 8].reshape(M, N)
    out = ops.gemm(dev_t(Aq, torch.bfloat16), dev_t(packed, torch.uint8), N, K, gate=dev_t(np.zeros(N), torch.float32),
                   residual=dev_t(res, torch.bfloat16), quantize_out=True)
    np.testing.assert_array_equal(out.float().cpu().numpy(), F.quantize_rows(res))


def test_grouped_matches_single(dev):
    rng = np.random.default_rng(9)
    specs, refs = [], []
    for M, K, N, act in ((4096 // 8, 128, 384, None), (256 // 4, 128, 256, "swiglu"), (130, 192, 128, None)):
        A = G.activations(rng, M, K)
        W = G.linear_weight(rng, N, K)
        packed = F.pack_b(W.T)
        Aq = F.quantize_rows(A)
        a, b = dev_t(Aq, torch.bfloat16), dev_t(packed, torch.uint8)
        specs.append(ops.GemmSpec(a, b, N, K, act=act))
        refs.append(ops.gemm(a, b, N, K, act=act))
    outs = ops.gemm_grouped(specs)
    for o, r in zip(outs, refs):
        assert torch.equal(o, r)


def test_grouped_deep_k(dev):
    """A group of deep-K members (K = 8192, as config 5's down projection; a SwiGLU member among them): bit-identical
    to each member's own whole-K launch, and against the emulation."""
    rng = np.random.default_rng(12)
    specs, refs, emu = [], [], []
    for M, K, N, act in ((512, 8192, 384, None), (256, 8192, 256, "swiglu"), (100, 8192, 128, None)):
        A = G.activations(rng, M, K)
        if act:
            packed = F.pack_b(F.interleave_up(G.linear_weight(rng, N // 2, K), G.linear_weight(rng, N // 2, K)))
        else:
            packed = F.pack_b(G.linear_weight(rng, N, K).T)
        Aq = F.quantize_rows(A)
        a, b = dev_t(Aq, torch.bfloat16), dev_t(packed, torch.uint8)
        specs.append(ops.GemmSpec(a, b, N, K, act=act))
        refs.append(ops.gemm(a, b, N, K, act=act, split=False))
        emu.append(G.gemm_ref(Aq, F.decode_b(packed, K, N), act=G.ACT_SWIGLU if act else G.ACT_NONE))
    outs = ops.gemm_grouped(specs)
    for o, r, e in zip(outs, refs, emu):
        assert torch.equal(o, r)
        check(o, e)


@pytest.mark.parametrize("a_fmt", ["packed_a_layout", "bf16_quantize"])
def test_grouped_non_bf16_a(dev, a_fmt):
    """A grouped launch with A in another format (every member's A staged as bf16 in one allocation first) gives the
    bits of the bf16-A group on the quantized values."""
    rng = np.random.default_rng(10)
    specs, specs16 = [], []
    for M, K, N, act in ((256, 128, 384, None), (128, 192, 256, "swiglu")):
        A = G.activations(rng, M, K)
        b = dev_t(F.pack_b(G.linear_weight(rng, N, K).T), torch.uint8)
        a = dev_t(F.to_bfp16(F.a_layout(A)), torch.uint8) if a_fmt == "packed_a_layout" else dev_t(A, torch.bfloat16)
        specs.append(ops.GemmSpec(a, b, N, K, act=act, M=M))
        specs16.append(ops.GemmSpec(dev_t(F.quantize_rows(A), torch.bfloat16), b, N, K, act=act))
    for o, r in zip(ops.gemm_grouped(specs, a_fmt=a_fmt), ops.gemm_grouped(specs16)):
        assert torch.equal(o, r)


def test_config1_full_size_rows(dev):
    """The 4096 x 3072 x 3072 configuration at full size (A ~N(0,1), W 3072x3072 ~N(0,0.02), seed 0): the GPU
    quantize pass feeds the GEMM; 256 sampled rows are checked against the emulation, and the quantized A bit-exact."""
    rng = np.random.default_rng(0)
    M = K = 4096
    K, N = 3072, 3072
    A = G.activations(rng, M, K)
    W = G.linear_weight(rng, N, K)
    a = dev_t(A, torch.bfloat16)
    w = dev_t(W, torch.float32)
    packed = ops.pack_weight(w)
    p, aq = ops.quantize(a, deq=True)
    out = ops.gemm(aq, packed, N, K)
    rows = np.sort(rng.choice(M, 256, replace=False))
    Aq = F.quantize_rows(A[rows])
    np.testing.assert_array_equal(aq[torch.from_numpy(rows).cuda()].float().cpu().numpy(), Aq)
    Bq = F.decode_b(packed.cpu().numpy(), K, N)
    check(out[torch.from_numpy(rows).cuda()], G.gemm_ref(Aq, Bq))


# Shapes that the launch planner of the bf16 path (256 CUs) runs as one launch of the 4-wave kernel with 6, 7 and 8
# fragment rows per wave (384-, 448- and 512-row tiles) or of the 8-wave kernel (1100 x 24576: 224-row tiles), and as
# a first 4-wave launch followed by a second launch over the remaining rows: of 256-row 4-wave tiles (4352 and 4296 x
# 24576, the latter with a partial last tile) or of the 8-wave kernel (4200 x 9216). Checked on sampled rows (the
# first and last tiles and both sides of every tile boundary near the split), with the gate-row split inside the
# second launch.
@pytest.mark.parametrize("M,N", [(3072, 4096), (4352, 3072), (4096, 4096), (4352, 24576), (4296, 24576),
                                 (4200, 9216), (1100, 24576)])
def test_tile_plans(dev, M, N):
    K = 64
    rng, A, packed, Aq, Bq = setup(M, K, N, M + N)
    res = F.bf16_round(rng.standard_normal((M, N)).astype(np.float32))
    gate = rng.standard_normal((2, N)).astype(np.float32)
    split = 4100  # gate row 1 for rows below; lies in the second launch for M = 4352, N = 24576
    out = ops.gemm(dev_t(Aq, torch.bfloat16), dev_t(packed, torch.uint8), N, K, gate=dev_t(gate, torch.float32),
                   gate_split_row=split, residual=dev_t(res, torch.bfloat16))
    rows = np.unique(np.concatenate([np.arange(0, 20), np.arange(M - 20, M), np.arange(4090, min(M, 4110)),
                                     np.arange(180, 200), np.arange(215, 235), np.arange(250, 262),
                                     rng.integers(0, M, 64)]))
    rows = rows[rows < M]
    # gate row 1 applies to global rows below the split: evaluate the sampled rows with each gate row and select
    ref = np.where((rows < split)[:, None], G.gemm_ref(Aq[rows], Bq, gate=gate[[1, 1]], residual=res[rows]),
                   G.gemm_ref(Aq[rows], Bq, gate=gate[[0, 0]], residual=res[rows]))
    check(out[torch.from_numpy(rows).cuda()], ref)


def _split_case(M, K, N, seed, act=None):
    rng = np.random.default_rng(seed)
    A = G.activations(rng, M, K)
    if act == "swiglu":
        packed = F.pack_b(F.interleave_up(G.linear_weight(rng, N // 2, K), G.linear_weight(rng, N // 2, K)))
    else:
        packed = F.pack_b(G.linear_weight(rng, N, K).T)
    return rng, F.quantize_rows(A), packed, F.decode_b(packed, K, N)


@pytest.mark.parametrize("M,K,N", [(256, 8192, 512), (100, 4096, 384), (512, 3072, 3072), (16, 8192, 3072)])
def test_k_split_plain(dev, M, K, N):
    """Small-M, deep-K shapes split K into pieces (fp32 partials in a workspace, summed in piece order): against the
    emulation, and against the whole-K kernel to within the fp32 summation difference. The first three split on the
    4-wave kernel (64-row fragments, 128 columns); 16 x 3072 x 8192 splits 16 ways on the 8-wave kernel (a 128-row
    tile holding 16 rows, 256 columns)."""
    assert ops.gemm_workspace_bytes(M, N, K) > 0
    rng, Aq, packed, Bq = _split_case(M, K, N, M + K)
    a, b = dev_t(Aq, torch.bfloat16), dev_t(packed, torch.uint8)
    out = ops.gemm(a, b, N, K)
    whole = ops.gemm(a, b, N, K, split=False)
    ref = G.gemm_ref(Aq, Bq)
    check(out, ref)
    d = (out.float() - whole.float()).abs().cpu().numpy()
    assert (d <= np.abs(ref) * 2.0 ** -7 + 1e-5 * np.abs(ref).max()).all()


def test_k_split_epilogues(dev):
    """Every epilogue after the piece reduction: bias + GELU, SwiGLU with bias and re-quantize, gate rows split
    with residual."""
    M, K, N = 256, 8192, 512
    rng, Aq, packed, Bq = _split_case(M, K, N, 21)
    a, b = dev_t(Aq, torch.bfloat16), dev_t(packed, torch.uint8)
    bias = (rng.standard_normal(N) * 0.5).astype(np.float32)
    out = ops.gemm(a, b, N, K, bias=dev_t(bias, torch.float32), act="gelu_tanh")
    check(out, G.gemm_ref(Aq, Bq, bias=bias, act=G.ACT_GELU_TANH))
    res = F.bf16_round(rng.standard_normal((M, N)).astype(np.float32))
    gate = rng.standard_normal((2, N)).astype(np.float32)
    out = ops.gemm(a, b, N, K, gate=dev_t(gate, torch.float32), gate_split_row=100, residual=dev_t(res, torch.bfloat16))
    check(out, G.gemm_ref(Aq, Bq, gate=gate, gate_split_row=100, residual=res))
    rng, Aq, packed, Bq = _split_case(M, K, N, 22, act="swiglu")
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    out = ops.gemm(dev_t(Aq, torch.bfloat16), dev_t(packed, torch.uint8), N, K, act="swiglu",
                   bias=dev_t(bias, torch.float32), quantize_out=True)
    assert out.shape == (M, N // 2)
    check(out, G.gemm_ref(Aq, Bq, act=G.ACT_SWIGLU, bias=bias, quantize_out=True), tol=2e-2)
    o = out.float().cpu().numpy()
    assert (F.quantize_rows(o) == o).mean() > 0.999  # exact bfp16 blocks (the -128 corner aside)


def test_k_split_workspace(dev):
    """The workspace contract: a shape the planner keeps whole needs none; too small a workspace is RL_ERR_WORKSPACE;
    a NULL workspace runs the whole-K kernel (same bits as rl_bfp16_gemm)."""
    from rlbfp import _lib as L
    assert ops.gemm_workspace_bytes(4352, 24576, 3072) == 0
    M, K, N = 100, 4096, 384
    need = ops.gemm_workspace_bytes(M, N, K)
    assert need == L.lib().rl_bfp16_gemm_workspace_bytes(M, N, K) > 0
    rng, Aq, packed, Bq = _split_case(M, K, N, 23)
    a, b = dev_t(Aq, torch.bfloat16), dev_t(packed, torch.uint8)
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    ep = ops._epilogue(None, None, None, 0, None, False)
    st = torch.cuda.current_stream().cuda_stream
    args = (a.data_ptr(), 0, K, b.data_ptr(), out.data_ptr(), N, M, N, K, ctypes.byref(ep))
    assert L.lib().rl_bfp16_gemm_ws(*args, ws.data_ptr(), need - 16, st) == L.RL_ERR_WORKSPACE
    assert L.lib().rl_bfp16_gemm_ws(*args, None, 0, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, ops.gemm(a, b, N, K, split=False))


def test_workspace_checked_before_staging(dev):
    """A non-bf16 A with a workspace that holds the staged bf16 copy but not the K-split partials: RL_ERR_WORKSPACE,
    returned before anything is enqueued, so neither the workspace nor C is written (both keep their canary bytes);
    the same call with rl_bfp16_gemm_workspace_size bytes then runs (the bf16 path's split bits)."""
    from rlbfp import _lib as L
    M, K, N = 100, 4096, 384
    rng = np.random.default_rng(29)
    A = G.activations(rng, M, K)
    packed = F.pack_b(G.linear_weight(rng, N, K).T)
    Aq, Bq = F.quantize_rows(A), F.decode_b(packed, K, N)
    a = dev_t(F.to_bfp16(A.reshape(-1)), torch.uint8)  # packed row blocks: the values of Aq
    b = dev_t(packed, torch.uint8)
    lib = L.lib()
    need = lib.rl_bfp16_gemm_workspace_size(L.RL_A_PACKED_ROWBLOCK, M, N, K)
    staged = ops.staged_a_bytes(M, K)
    assert need > staged + 16 and lib.rl_bfp16_gemm_workspace_bytes(M, N, K) == need - staged
    ws = torch.full((need,), 0xA5, dtype=torch.uint8, device="cuda")
    out = torch.full((M, N), 3.0, dtype=torch.bfloat16, device="cuda")
    ep = ops._epilogue(None, None, None, 0, None, False)
    st = torch.cuda.current_stream().cuda_stream
    args = (a.data_ptr(), L.RL_A_PACKED_ROWBLOCK, K, b.data_ptr(), out.data_ptr(), N, M, N, K, ctypes.byref(ep))
    for short in (need - 16, staged, staged - 256):
        assert lib.rl_bfp16_gemm_ws(*args, ws.data_ptr(), short, st) == L.RL_ERR_WORKSPACE, short
    torch.cuda.synchronize()
    assert bool((ws == 0xA5).all()), "the refused call wrote to the workspace"
    assert bool((out == 3.0).all()), "the refused call wrote to C"
    assert lib.rl_bfp16_gemm_ws(*args, ws.data_ptr(), need, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, ops.gemm(dev_t(Aq, torch.bfloat16), b, N, K))
    check(out, G.gemm_ref(Aq, Bq))


def _exponent_class_weight(rng, N, K, classes):
    """Linear weight (N, K) whose column n of B = W.T holds blocks of exponent class classes[n % len(classes)]: E (all
    8 values in the binade [2^(E-127), 2^(E-126)), so every q is in 64..127 and every decoded value is a normal
    number), None (all-zero blocks) or "ordinary" (the usual ~N(0, 0.02) weights)."""
    W = G.linear_weight(rng, N, K)
    for n in range(N):
        E = classes[n % len(classes)]
        if E == "ordinary":
            continue
        if E is None:
            W[n] = 0.0
            continue
        mag = rng.uniform(1.0, 1.49, K)
        mag[::8] = 1.5  # one block maximum per block
        W[n] = mag * rng.choice([-1.0, 1.0], K) * 2.0 ** (E - 127)
    return W.astype(np.float32)


@pytest.mark.parametrize("classes,a_scale", [((1, 3, 6, 7, 8, None, "ordinary"), 2.0 ** 100),
                                             ((133, 134, 200, 220, None, "ordinary"), 1.0)])
def test_weight_block_exponents(dev, classes, a_scale):
    """Weight blocks at the edges of the decoder's fast exponent range (E = 7..133, by a packed exponent subtract)
    and past them (E = 1, 3, 6, 134, 200, 220, and all-zero blocks, which the float path re-decodes). Columns of one
    class sit next to columns of others, so a decoding lane covers several classes; A is scaled by a power of two so
    that every product is a normal number; each column is checked against the emulation at its own scale."""
    M, K, N = 256, 512, 256
    rng = np.random.default_rng(31)
    Aq = F.quantize_rows(G.activations(rng, M, K)) * np.float32(a_scale)
    W = _exponent_class_weight(rng, N, K, classes)
    packed = F.pack_b(W.T)
    want_E = {c for c in classes if isinstance(c, int)} | ({0} if None in classes else set())
    assert want_E <= set(packed.reshape(-1, 9)[:, 0].tolist())
    Bq = F.decode_b(packed, K, N)
    out = ops.gemm(dev_t(Aq, torch.bfloat16), dev_t(packed, torch.uint8), N, K).float().cpu().numpy()
    ref = G.gemm_ref(Aq, Bq)
    assert np.isfinite(ref).all()
    for n in range(N):
        got, want = out[:, n].astype(np.float64), ref[:, n]
        scale = np.abs(want).max()
        if scale == 0:
            assert (got == 0).all(), n  # all-zero column
            continue
        assert np.abs(got - want).max() <= TOL * scale, (n, classes[n % len(classes)])
        assert (np.abs(got - want) <= 2 * np.abs(want) * 2.0 ** -8 + 1e-4 * scale).mean() > 0.99, n


def test_packed_a_without_workspace_refused_under_capture(dev):
    """A non-bf16 A with no workspace stages into a stream-ordered allocation, which a stream under graph capture
    cannot take: the call is refused with RL_ERR_WORKSPACE before anything is enqueued, and the same call with a
    workspace is captured and replays to the eager result."""
    from rlbfp import _lib as L
    M, K, N = 128, 128, 256
    rng, A, packed, Aq, Bq = setup(M, K, N, 11)
    a = dev_t(F.to_bfp16(F.a_layout(A)), torch.uint8)
    b = dev_t(packed, torch.uint8)
    ref = ops.gemm(a, b, N, K, M=M, a_fmt="packed_a_layout", workspace=False)
    out = torch.zeros_like(ref)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        graph.capture_begin()
        try:
            with pytest.raises(L.RLError) as e:
                ops.gemm(a, b, N, K, M=M, a_fmt="packed_a_layout", workspace=False, out=out)
            ops.gemm(a, b, N, K, M=M, a_fmt="packed_a_layout", out=out)
        finally:
            graph.capture_end()
    assert e.value.code == L.RL_ERR_WORKSPACE
    torch.cuda.current_stream().wait_stream(side)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
