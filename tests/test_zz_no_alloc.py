"""rl_bfp16_gemm_noalloc (the allocation-free GEMM: its workspace is a fixed device array inside the library) against
rl_bfp16_gemm_ws with a caller's workspace of the same size, through the C ABI: bit-identical outputs on two calls in
a row, the second with a smaller input, for a K-split shape (fp32 partials in the scratch) and a packed-A shape (A
staged as bf16 in the scratch); shapes beyond the fixed size are rejected with RL_ERR_WORKSPACE."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import bfp16 as F
from oracle import gemm as G
from rlbfp import _lib as L
from rlbfp import ops

pytestmark = pytest.mark.gpu


def _case(M, K, N, seed, a_fmt):
    rng = np.random.default_rng(seed)
    A = G.activations(rng, M, K)
    W = G.linear_weight(rng, N, K)
    b = torch.from_numpy(F.pack_b(W.T)).cuda()
    if a_fmt == L.RL_A_BF16:
        a = torch.from_numpy(F.quantize_rows(A)).cuda().to(torch.bfloat16)
        lda = K
    else:
        a = torch.from_numpy(F.to_bfp16(F.a_layout(A))).cuda()
        lda = 0
    return a, lda, b, F.quantize_rows(A), F.decode_b(b.cpu().numpy(), K, N)


def _both(a, a_fmt, lda, b, M, N, K):
    lib = L.lib()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ep = ops._epilogue(None, None, None, 0, None, False)
    need = lib.rl_bfp16_gemm_workspace_size(a_fmt, M, N, K)
    assert 0 < need <= L.RL_NOALLOC_SCRATCH_BYTES
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    ref = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    got = torch.full((M, N), 7.0, dtype=torch.bfloat16, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    L.check(lib.rl_bfp16_gemm_ws(P(a), a_fmt, lda, P(b), P(ref), N, M, N, K, ctypes.byref(ep), P(ws), need, st))
    L.check(lib.rl_bfp16_gemm_noalloc(P(a), a_fmt, lda, P(b), P(got), N, M, N, K, ctypes.byref(ep), st))
    torch.cuda.synchronize()
    return got, ref


@pytest.mark.parametrize("a_fmt,shapes", [
    (L.RL_A_BF16, [(512, 12288, 4096), (100, 4096, 384)]),             # K-split partials in the scratch
    (L.RL_A_PACKED_A_LAYOUT, [(1024, 3072, 2048), (256, 1024, 512)]),  # A staged as bf16 in the scratch
])
def test_noalloc_matches_workspace_entry_point(dev, a_fmt, shapes):
    for i, (M, K, N) in enumerate(shapes):
        a, lda, b, Aq, Bq = _case(M, K, N, 40 + i, a_fmt)
        got, ref = _both(a, a_fmt, lda, b, M, N, K)
        assert torch.equal(got, ref), (M, K, N)
        rows = np.arange(0, M, max(1, M // 64))
        assert G.rel_err(got[torch.from_numpy(rows).cuda()].float().cpu().numpy(), G.gemm_ref(Aq[rows], Bq)) <= 1e-2


def test_noalloc_rejects_shapes_beyond_the_scratch(dev):
    lib = L.lib()
    M, K, N = 4352, 12288, 3072                      # a packed A of 4352 x 12288 stages 107 MB
    assert lib.rl_bfp16_gemm_workspace_size(L.RL_A_PACKED_A_LAYOUT, M, N, K) > L.RL_NOALLOC_SCRATCH_BYTES
    a = torch.zeros(M * K // 8 * 9, dtype=torch.uint8, device="cuda")
    b = torch.zeros(K * N // 8 * 9, dtype=torch.uint8, device="cuda")
    c = torch.zeros((M, N), dtype=torch.bfloat16, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.rl_bfp16_gemm_noalloc(ctypes.c_void_p(a.data_ptr()), L.RL_A_PACKED_A_LAYOUT, 0,
                                   ctypes.c_void_p(b.data_ptr()), ctypes.c_void_p(c.data_ptr()), N, M, N, K, None, st)
    assert rc == L.RL_ERR_WORKSPACE
    assert b"RL_NOALLOC_SCRATCH_BYTES" in lib.rl_last_error()
    torch.cuda.synchronize()
    assert (c == 0).all()                            # nothing was launched
