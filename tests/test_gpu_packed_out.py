"""The GEMM epilogue writing its output in the reference's stream orders:
  * bfp16 blocks in the ATB C order, the reference GEMM's C stream (kernels/atb3/mm_bfp_mixed.cc:153-168);
  * bfp16 blocks of the SwiGLU output H in the down GEMM's A layout (kernels/atb3/mm_bfp_swiglu.cc:73-86);
  * bf16 C in the ATB element order, the C16 artifacts' output (kernels/vlm/mm_bfp_c16.cc:1-2).
Each is checked byte for byte against the oracle's encoder and layout applied to the same call's row-major bf16
output (to_bfp16(c_layout_atb(y)), to_bfp16(a_layout(h)), c_layout_atb(y)), and against the two-pass form the
drop-in used before (row-major bf16 C, then the quantize pass in that order). Every kernel path is covered: the
4-wave kernel's whole-K tiles, its second launch over the rows past the first (the full FFN up GEMM), the 8-wave
kernel (GELU), the K-split reduce, and blocks of extreme exponents (the integer encoder)."""

import numpy as np
import pytest
import torch

from oracle import bfp16 as F
from oracle import gemm as G
from rlbfp import ops

pytestmark = pytest.mark.gpu


def dev_t(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def _case(M, K, N, seed, swiglu=False, scale=1.0):
    rng = np.random.default_rng(seed)
    A = G.activations(rng, M, K, outliers=0.01) * np.float32(scale)
    if swiglu:
        packed = F.pack_b(F.interleave_up(G.linear_weight(rng, N // 2, K), G.linear_weight(rng, N // 2, K)))
    else:
        packed = F.pack_b(G.linear_weight(rng, N, K).T)
    a = dev_t(F.quantize_rows(A), torch.bfloat16)
    return rng, a, dev_t(packed, torch.uint8)


def _check_packed(y, packed, order):
    """packed == to_bfp16(layout(y)) (the oracle) == the quantize pass over y (the two-pass form)."""
    yh = y.float().cpu().numpy()
    want = F.to_bfp16(F.c_layout_atb(yh) if order == "c_atb" else F.a_layout(yh))
    got = packed.cpu().numpy()
    assert got.shape == want.shape
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} bytes differ from the oracle, first at {bad[:4]}"
    two_pass, _ = ops.quantize(y, order=order)
    assert torch.equal(packed, two_pass)


@pytest.mark.parametrize("bias", [False, True])
def test_packed_c_atb_4wave(dev, bias):
    M, K, N = 1024, 256, 2048
    rng, a, b = _case(M, K, N, 1)
    bv = dev_t(rng.standard_normal(N).astype(np.float32) * 0.5, torch.float32) if bias else None
    y = ops.gemm(a, b, N, K, bias=bv)
    pk = torch.full((M * N // 8 * 9,), 0x5A, dtype=torch.uint8, device="cuda")
    assert ops.gemm(a, b, N, K, bias=bv, packed_out=pk, packed_order="c_atb") is pk  # no bf16 C written
    _check_packed(y, pk, "c_atb")
    # with a bf16 C beside it: C equals the plain call's; with RL_EP_QUANTIZE_OUT it holds the packed values
    pk2 = torch.empty_like(pk)
    c = ops.gemm(a, b, N, K, bias=bv, packed_out=pk2, out=torch.empty((M, N), dtype=torch.bfloat16, device="cuda"))
    assert torch.equal(c, y) and torch.equal(pk2, pk)
    cq = ops.gemm(a, b, N, K, bias=bv, packed_out=pk2, quantize_out=True,
                  out=torch.empty((M, N), dtype=torch.bfloat16, device="cuda"))
    assert torch.equal(pk2, pk)
    assert np.array_equal(cq.float().cpu().numpy(), F.c_unlayout_atb(F.from_bfp16(pk.cpu().numpy()), M, N))


def test_c_atb_bf16_elements(dev):
    """bf16 C in the ATB element order (the C16 artifacts), against the oracle's c_layout_atb of the row-major C."""
    M, K, N = 512, 192, 1024
    rng, a, b = _case(M, K, N, 2)
    y = ops.gemm(a, b, N, K)
    flat = ops.gemm(a, b, N, K, c_order="c_atb")
    assert flat.shape == (M * N,)
    want = F.c_layout_atb(y.float().cpu().numpy())
    assert np.array_equal(flat.float().cpu().numpy(), want)


def test_packed_a_layout_swiglu(dev):
    """The SwiGLU GEMM pushing H in the down GEMM's A layout; the bf16 H with RL_EP_QUANTIZE_OUT equals its decode."""
    M, K, N = 384, 256, 2 * 512
    rng, a, b = _case(M, K, N, 3, swiglu=True)
    h = ops.gemm(a, b, N, K, act="swiglu")
    pk = torch.empty(M * N // 2 // 8 * 9, dtype=torch.uint8, device="cuda")
    hq = ops.gemm(a, b, N, K, act="swiglu", quantize_out=True, packed_out=pk, packed_order="a_layout",
                  out=torch.empty((M, N // 2), dtype=torch.bfloat16, device="cuda"))
    _check_packed(h, pk, "a_layout")
    assert np.array_equal(hq.float().cpu().numpy(), F.a_unlayout(F.from_bfp16(pk.cpu().numpy()), M, N // 2))


def test_packed_full_ffn_up(dev):
    """The FFN up GEMM at full size (4352 x 3072 x 2 x 12288): two launches, the second over rows 4096..4351, both
    writing H in the A layout at their own rows."""
    M, K, N = 4352, 3072, 2 * 12288
    g = torch.Generator(device="cuda").manual_seed(5)
    x = ops.quantize(torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16), deq=True)[1]
    w = ops.pack_weight(ops.interleave_up(torch.randn((N // 2, K), generator=g, device="cuda") * 0.02,
                                          torch.randn((N // 2, K), generator=g, device="cuda") * 0.02).contiguous())
    h = ops.gemm(x, w, N, K, act="swiglu")
    pk = torch.empty(M * N // 2 // 8 * 9, dtype=torch.uint8, device="cuda")
    hq = ops.gemm(x, w, N, K, act="swiglu", quantize_out=True, packed_out=pk, packed_order="a_layout",
                  out=torch.empty_like(h))
    assert torch.equal(pk, ops.quantize(h, order="a_layout")[0])
    # the re-quantized H is the packed blocks' values (not a re-encoding of them: a block whose largest element
    # rounds to q = -128 would re-encode one exponent up)
    assert torch.equal(ops.dequantize(pk, M, N // 2, order="a_layout", dtype=torch.bfloat16), hq)


def test_packed_8wave_gelu(dev):
    """GELU runs on the 8-wave kernel (one row at a time in its epilogue)."""
    M, K, N = 512, 256, 1024
    rng, a, b = _case(M, K, N, 6)
    y = ops.gemm(a, b, N, K, act="gelu_tanh")
    pk = torch.empty(M * N // 8 * 9, dtype=torch.uint8, device="cuda")
    ops.gemm(a, b, N, K, act="gelu_tanh", packed_out=pk)
    _check_packed(y, pk, "c_atb")


@pytest.mark.parametrize("swiglu", [False, True])
def test_packed_k_split_reduce(dev, swiglu):
    """A small-M, deep-K shape split along K: the reduce launch writes the packed blocks (one block per thread)."""
    M, K, N = 512, 8192, 2048
    assert ops.gemm_workspace_bytes(M, N, K) > 0
    rng, a, b = _case(M, K, N, 7, swiglu=swiglu)
    act = "swiglu" if swiglu else None
    nout = N // 2 if swiglu else N
    order = "a_layout" if swiglu else "c_atb"
    y = ops.gemm(a, b, N, K, act=act)
    pk = torch.empty(M * nout // 8 * 9, dtype=torch.uint8, device="cuda")
    ops.gemm(a, b, N, K, act=act, packed_out=pk, packed_order=order)
    _check_packed(y, pk, order)


def test_packed_extreme_exponents(dev):
    """Outputs scaled so that their blocks' exponents fall outside the float fast path (E > 237: values of 2^111
    and more): the integer encoder writes those blocks, still equal to the oracle's."""
    M, K, N = 512, 128, 1024
    rng, a, b = _case(M, K, N, 8, scale=2.0 ** 112)
    y = ops.gemm(a, b, N, K)
    yh = y.float().cpu().numpy()
    assert np.isfinite(yh).all() and (np.abs(yh).max() >= 2.0 ** 111)
    pk = torch.empty(M * N // 8 * 9, dtype=torch.uint8, device="cuda")
    ops.gemm(a, b, N, K, packed_out=pk)
    assert (pk.cpu().numpy().reshape(-1, 9)[:, 0] > 237).any()
    _check_packed(y, pk, "c_atb")


@pytest.mark.parametrize("N", [9216, 3072])
def test_packed_tiles_past_m(dev, N):
    """M = 4608 (the DiT block's 4352 tokens padded to a multiple of 512): the planner runs these rows, or the rows
    past a first launch, on the 8-wave kernel in 224-row tiles, whose last tile reaches past M. Its row quads past M
    write nothing: the bytes after the packed stream keep their canary, and the stream equals the quantize pass."""
    M, K = 4608, 256
    rng, a, b = _case(M, K, N, 9)
    y = ops.gemm(a, b, N, K)
    n = M * N // 8 * 9
    buf = torch.full((n + 65536,), 0xC3, dtype=torch.uint8, device="cuda")
    ops.gemm(a, b, N, K, packed_out=buf[:n])
    torch.cuda.synchronize()
    assert bool((buf[n:] == 0xC3).all()), "bytes past the packed stream were written"
    assert torch.equal(buf[:n], ops.quantize(y, order="c_atb")[0])
    flat = torch.full((M * N + 32768,), 5.0, dtype=torch.bfloat16, device="cuda")
    ops.gemm(a, b, N, K, out=flat[:M * N], c_order="c_atb")
    torch.cuda.synchronize()
    assert bool((flat[M * N:] == 5.0).all()), "elements past the ATB-ordered C were written"
    assert np.array_equal(flat[:M * N].float().cpu().numpy(), F.c_layout_atb(y.float().cpu().numpy()))


def test_packed_qkv_full(dev):
    """The DiT block's QKV GEMM at full size as the reference's op list runs it (M = 4608, K = 3072, N = 9216, the C
    stream in the ATB order): the planner's two launches (4-wave tiles, then the 8-wave kernel past them) write the
    same bytes as the quantize pass over the bf16 C, and a bf16 C written beside them equals the plain call's."""
    M, K, N = 4608, 3072, 9216
    g = torch.Generator(device="cuda").manual_seed(21)
    x = ops.quantize(torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16), deq=True)[1]
    w = ops.pack_weight(torch.randn((N, K), generator=g, device="cuda") * 0.02)
    y = ops.gemm(x, w, N, K)
    pk = torch.full((M * N // 8 * 9,), 0x5A, dtype=torch.uint8, device="cuda")
    ops.gemm(x, w, N, K, packed_out=pk)
    assert torch.equal(pk, ops.quantize(y, order="c_atb")[0])
    pk2 = torch.empty_like(pk)
    c = ops.gemm(x, w, N, K, packed_out=pk2, out=torch.empty_like(y))
    assert torch.equal(c, y) and torch.equal(pk2, pk)
