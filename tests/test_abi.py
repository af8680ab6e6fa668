"""The C ABI without a GPU: the library loads, exports every function include/rlbfp.h declares, and its host-side
validators reject bad shapes with the documented codes."""

import ctypes
import os
import re

import pytest

from rlbfp import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "rlbfp.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rl_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_symbol():
    lib = L.lib()
    names = header_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
        assert n in L.SIGNATURES, f"{n} has no ctypes signature"


def test_version_and_sizes():
    assert L.lib().rl_version().decode().startswith("rlbfp")
    assert L.lib().rl_packed_bytes(4096, 3072) == 4096 * 3072 // 8 * 9
    assert L.lib().rl_packed_bytes(1, 7) == -1


@pytest.mark.parametrize("args,code", [
    ((L.RL_DTYPE_BF16, 128, 64, 64, L.RL_ORDER_ROWBLOCK), L.RL_OK),
    ((L.RL_DTYPE_BF16, 128, 60, 64, L.RL_ORDER_ROWBLOCK), L.RL_ERR_SHAPE),
    ((L.RL_DTYPE_F32, 100, 64, 64, L.RL_ORDER_A_LAYOUT), L.RL_ERR_SHAPE),
    ((L.RL_DTYPE_F32, 512, 1024, 1024, L.RL_ORDER_C_ATB), L.RL_OK),
    ((L.RL_DTYPE_F32, 512, 512, 512, L.RL_ORDER_C_ATB), L.RL_ERR_SHAPE),
    ((7, 128, 64, 64, L.RL_ORDER_ROWBLOCK), L.RL_ERR_ARG),
    ((L.RL_DTYPE_F32, 128, 64, 32, L.RL_ORDER_ROWBLOCK), L.RL_ERR_SHAPE),
    ((L.RL_DTYPE_F32, 128, 64, 64, 9), L.RL_ERR_ARG),
])
def test_validate_quantize(args, code):
    assert L.lib().rl_validate_quantize(*args) == code
    if code:
        assert L.lib().rl_last_error().decode()


def ep(act=0, flags=0, residual=None, ld=0, split=0, packed=None, order=0, c_order=0):
    e = L.Epilogue()
    e.act, e.flags, e.residual, e.ld_residual, e.gate_split_row = act, flags, residual, ld, split
    e.packed_out, e.packed_order, e.c_order = packed, order, c_order
    return ctypes.byref(e)


@pytest.mark.parametrize("a_fmt,lda,ldc,M,N,K,e,code", [
    (L.RL_A_BF16, 3072, 9216, 4352, 9216, 3072, None, L.RL_OK),
    (L.RL_A_BF16, 3072, 12288, 4352, 24576, 3072, ep(L.RL_ACT_SWIGLU), L.RL_OK),
    (L.RL_A_BF16, 3072, 12288, 4352, 24576, 3072, ep(L.RL_ACT_NONE), L.RL_ERR_ALIGN),  # ldc < N
    (L.RL_A_BF16, 3072, 3072, 1, 3072, 3072, None, L.RL_OK),
    (L.RL_A_BF16, 3072, 3072, 0, 3072, 3072, None, L.RL_ERR_SHAPE),
    (L.RL_A_BF16, 3072, 3072, 64, 3000, 3072, None, L.RL_ERR_SHAPE),
    (L.RL_A_BF16, 3072, 3072, 64, 3072, 3000, None, L.RL_ERR_SHAPE),
    (L.RL_A_BF16, 3071, 3072, 64, 3072, 3072, None, L.RL_ERR_ALIGN),
    (L.RL_A_PACKED_A_LAYOUT, 0, 3072, 100, 3072, 3072, None, L.RL_ERR_SHAPE),
    (L.RL_A_PACKED_ROWBLOCK, 0, 3072, 100, 3072, 3072, None, L.RL_OK),
    (9, 3072, 3072, 64, 3072, 3072, None, L.RL_ERR_ARG),
    (L.RL_A_BF16, 3072, 3072, 64, 3072, 3072, ep(act=5), L.RL_ERR_ARG),
    (L.RL_A_BF16, 3072, 3072, 64, 3072, 3072, ep(flags=4), L.RL_ERR_ARG),
    (L.RL_A_BF16, 3072, 3072, 64, 3072, 3072, ep(residual=1, ld=100), L.RL_ERR_SHAPE),
    (L.RL_A_BF16, 3072, 3072, 64, 3072, 3072, ep(split=-1), L.RL_ERR_ARG),
    # packed output in the reference's stream orders: ATB C (M % 512, Nout % 1024), A layout (M % 128, Nout % 64)
    (L.RL_A_BF16, 3072, 9216, 4608, 9216, 3072, ep(packed=16, order=L.RL_ORDER_C_ATB), L.RL_OK),
    (L.RL_A_BF16, 3072, 9216, 4352, 9216, 3072, ep(packed=16, order=L.RL_ORDER_C_ATB), L.RL_ERR_SHAPE),
    (L.RL_A_BF16, 3072, 12288, 4352, 24576, 3072, ep(L.RL_ACT_SWIGLU, packed=16, order=L.RL_ORDER_A_LAYOUT),
     L.RL_OK),
    (L.RL_A_BF16, 3072, 12288, 4300, 24576, 3072, ep(L.RL_ACT_SWIGLU, packed=16, order=L.RL_ORDER_A_LAYOUT),
     L.RL_ERR_SHAPE),
    (L.RL_A_BF16, 3072, 3072, 512, 3072, 3072, ep(packed=16, order=L.RL_ORDER_ROWBLOCK), L.RL_ERR_ARG),
    (L.RL_A_BF16, 3072, 0, 512, 3072, 3072, ep(c_order=L.RL_C_ATB), L.RL_OK),  # ldc ignored
    (L.RL_A_BF16, 3072, 3072, 256, 3072, 3072, ep(c_order=L.RL_C_ATB), L.RL_ERR_SHAPE),
    (L.RL_A_BF16, 3072, 3072, 512, 3072, 3072, ep(c_order=2), L.RL_ERR_ARG),
])
def test_validate_gemm(a_fmt, lda, ldc, M, N, K, e, code):
    assert L.lib().rl_validate_gemm(a_fmt, lda, ldc, M, N, K, e) == code


@pytest.mark.parametrize("args,code", [
    ((3072, 18432, 1, 18432, 3072, L.RL_GEMV_SILU), L.RL_OK),
    ((3072, 18432, 9, 18432, 3072, L.RL_GEMV_SILU), L.RL_ERR_SHAPE),
    ((3072, 18432, 1, 18400, 3072, L.RL_GEMV_SILU), L.RL_ERR_SHAPE),
    ((3072, 18432, 1, 18432, 3072, L.RL_ACT_SWIGLU), L.RL_ERR_ARG),
    ((3000, 18432, 1, 18432, 3072, L.RL_ACT_NONE), L.RL_ERR_SHAPE),
])
def test_validate_gemv(args, code):
    assert L.lib().rl_validate_gemv(*args) == code


def test_null_pointers_rejected_before_any_gpu_call():
    """Argument errors are reported before the device is touched, so they work on a machine without a GPU."""
    lib = L.lib()
    s = lib.rl_bfp16_quantize(None, L.RL_DTYPE_BF16, 128, 64, 64, 0, None, None, None)
    assert s == L.RL_ERR_NULL
    s = lib.rl_bfp16_gemm(None, 0, 64, None, None, 128, 1, 128, 64, None, None)
    assert s == L.RL_ERR_NULL
    s = lib.rl_bfp16_gemv(None, 64, None, None, 128, 1, 128, 64, L.RL_GEMV_SILU, None)
    assert s == L.RL_ERR_NULL
    s = lib.rl_bfp16_gemm_grouped(None, 1, 0, None)
    assert s == L.RL_ERR_NULL


@pytest.mark.parametrize("args,code", [
    ((3072, L.RL_BRANCH_BF16, 3072, L.RL_NORM_LAYER, 3072, L.RL_ORDER_ROWBLOCK, 3072, 0, 4352, 3072), L.RL_OK),
    ((4096, L.RL_BRANCH_PACKED, 0, L.RL_NORM_RMS, 4096, L.RL_ORDER_A_LAYOUT, 4096, 0, 512, 4096), L.RL_OK),
    ((3072, L.RL_BRANCH_BF16, 3072, L.RL_NORM_LAYER, 3072, L.RL_ORDER_A_LAYOUT, 3072, 0, 100, 3072), L.RL_ERR_SHAPE),
    ((96, L.RL_BRANCH_BF16, 96, L.RL_NORM_LAYER, 96, L.RL_ORDER_ROWBLOCK, 96, 0, 4, 96), L.RL_ERR_SHAPE),
    ((16384, L.RL_BRANCH_BF16, 16384, L.RL_NORM_LAYER, 16384, L.RL_ORDER_ROWBLOCK, 16384, 0, 4, 16384),
     L.RL_ERR_SHAPE),
    ((3072, 7, 3072, L.RL_NORM_LAYER, 3072, L.RL_ORDER_ROWBLOCK, 3072, 0, 8, 3072), L.RL_ERR_ARG),
    ((3072, L.RL_BRANCH_BF16, 3072, 5, 3072, L.RL_ORDER_ROWBLOCK, 3072, 0, 8, 3072), L.RL_ERR_ARG),
    ((3072, L.RL_BRANCH_BF16, 3072, L.RL_NORM_LAYER, 3072, L.RL_ORDER_C_ATB, 3072, 0, 512, 3072), L.RL_ERR_ARG),
    ((3072, L.RL_BRANCH_BF16, 3072, L.RL_NORM_LAYER, 3072, L.RL_ORDER_ROWBLOCK, 3072, -1, 8, 3072), L.RL_ERR_ARG),
    ((3070, L.RL_BRANCH_BF16, 3072, L.RL_NORM_LAYER, 3072, L.RL_ORDER_ROWBLOCK, 3072, 0, 8, 3072), L.RL_ERR_ALIGN),
    ((3072, L.RL_BRANCH_BF16, 3076, L.RL_NORM_LAYER, 3072, L.RL_ORDER_ROWBLOCK, 3072, 0, 8, 3072), L.RL_ERR_ALIGN),
])
def test_validate_ln(args, code):
    assert L.lib().rl_validate_ln(*args) == code


def test_ln_null_pointers_rejected_before_any_gpu_call():
    lib = L.lib()
    s = lib.rl_ln_modulate(None, 64, None, 0, 64, None, 0, 0, None, 64, None, 0, None, 64, 4, 64, None)
    assert s == L.RL_ERR_NULL
    s = lib.rl_ln_modulate(16, 64, None, 0, 64, 16, 0, 0, None, 0, None, 0, None, 0, 4, 64, None)
    assert s == L.RL_ERR_NULL  # every output NULL


@pytest.mark.parametrize("args,code", [
    ((9216, 4352, 24), L.RL_OK),
    ((12288, 4096, 32), L.RL_OK),
    ((9216, 4350, 24), L.RL_ERR_SHAPE),
    ((9216, 0, 24), L.RL_ERR_SHAPE),
    ((9216, 4352, 0), L.RL_ERR_SHAPE),
    ((9000, 4352, 24), L.RL_ERR_ALIGN),
    ((9220, 4352, 24), L.RL_ERR_ALIGN),
])
def test_validate_qkv_post(args, code):
    assert L.lib().rl_validate_qkv_post(*args) == code


def test_qkv_post_null_pointers_rejected_before_any_gpu_call():
    lib = L.lib()
    assert lib.rl_qkv_post(None, 384, 64, 1, None, None, None, None, None, None, None, None, None, None) == \
        L.RL_ERR_NULL
    assert lib.rl_qkv_post(16, 384, 64, 1, 16, 16, 16, 16, None, None, None, None, None, None) == L.RL_ERR_NULL


@pytest.mark.parametrize("args,code", [
    ((24, 4352, 4352, 4352, 3072, 0), L.RL_OK),
    ((32, 4096, 8256, 8224, 4096, 0), L.RL_OK),
    ((2, 256, 512, 512, 768, 4), L.RL_OK),
    ((24, 4350, 4352, 4352, 3072, 0), L.RL_ERR_SHAPE),
    ((24, 4352, 4350, 4350, 3072, 0), L.RL_ERR_SHAPE),
    ((24, 4352, 4352, 0, 3072, 0), L.RL_ERR_SHAPE),
    ((24, 4352, 4352, 4353, 3072, 0), L.RL_ERR_SHAPE),
    ((24, 4352, 4352, 4352, 3000, 0), L.RL_ERR_ALIGN),
    ((2, 256, 512, 512, 768, 5), L.RL_ERR_ALIGN),
    ((2, 256, 512, 512, 768, -1), L.RL_ERR_ARG),
    ((0, 256, 512, 512, 768, 0), L.RL_ERR_SHAPE),
])
def test_validate_attention(args, code):
    assert L.lib().rl_validate_attention(*args) == code


def test_attention_null_pointers_rejected_before_any_gpu_call():
    assert L.lib().rl_attention(None, None, None, 1, 128, 64, 64, None, None, 128, 0, 0, None) == L.RL_ERR_NULL


def test_gemm_split_plan_without_a_gpu():
    """The K-split planner behind rl_bfp16_gemm_workspace_bytes (256 compute units when no device is visible, as on
    MI355X): the text encoder's down projection at M = 512 splits 4 ways with 128-row tiles (4 x 512 x 4096 fp32
    planes); shapes whose tiles fill the chip, and shallow K, run whole; invalid shapes give -1."""
    ws = L.lib().rl_bfp16_gemm_workspace_bytes
    if _has_gpu():
        pytest.skip("the plan depends on the visible device's compute units")
    assert ws(512, 4096, 12288) == 4 * 512 * 4096 * 4
    for M, N, K in ((4352, 24576, 3072), (4352, 3072, 12288), (4096, 3072, 3072), (512, 24576, 4096), (1, 128, 64)):
        assert ws(M, N, K) == 0, (M, N, K)
    assert ws(512, 100, 64) == -1  # N % 128 != 0
    assert ws(0, 128, 64) == -1


def test_gemm_ws_null_pointers_rejected_before_any_gpu_call():
    assert L.lib().rl_bfp16_gemm_ws(None, 0, 64, None, None, 128, 1, 128, 64, None, None, 0, None) == L.RL_ERR_NULL


@pytest.mark.parametrize("a_fmt,M,N,K", [
    (L.RL_A_BF16, 1, 32768, 65536),                 # packed B of 2.4 GB
    (L.RL_A_BF16, 40000, 128, 32768),               # bf16 A of 2.6 GB
    (L.RL_A_PACKED_ROWBLOCK, 40000, 128, 32768),    # packed A of 1.5 GB whose staged bf16 copy is 2.6 GB
])
def test_gemm_operands_above_2gb_rejected_before_any_gpu_call(a_fmt, M, N, K):
    """Buffer offsets are 32-bit: an operand (or the staged bf16 copy of a packed A) above 2^31 bytes is refused with
    RL_ERR_SHAPE while the arguments are checked, before the device is touched (the pointers are never read)."""
    A, B, C = ctypes.c_void_p(0x10000), ctypes.c_void_p(0x20000), ctypes.c_void_p(0x30000)
    lda = K if a_fmt == L.RL_A_BF16 else 0
    assert L.lib().rl_bfp16_gemm(A, a_fmt, lda, B, C, N, M, N, K, None, None) == L.RL_ERR_SHAPE
    assert b"2^31" in L.lib().rl_last_error()


def _has_gpu():
    try:
        import torch
        return torch.cuda.device_count() > 0
    except Exception:
        return False


def test_gemm_workspace_size_per_a_format():
    """rl_bfp16_gemm_workspace_size: the K-split partials for RL_A_BF16; for the other A formats also the staged bf16
    copy of A, M * K * 2 rounded up to 256 bytes; -1 for an invalid shape or format."""
    size, split = L.lib().rl_bfp16_gemm_workspace_size, L.lib().rl_bfp16_gemm_workspace_bytes
    for M, N, K in ((4352, 24576, 3072), (512, 4096, 12288), (100, 384, 4096), (1, 128, 64)):
        assert size(L.RL_A_BF16, M, N, K) == split(M, N, K)
        for fmt in (L.RL_A_BF16_QUANTIZE, L.RL_A_PACKED_ROWBLOCK):
            assert size(fmt, M, N, K) == (M * K * 2 + 255) // 256 * 256 + split(M, N, K)
    assert size(L.RL_A_PACKED_A_LAYOUT, 4096, 3072, 3072) == 4096 * 3072 * 2
    assert size(L.RL_A_PACKED_A_LAYOUT, 100, 384, 4096) == -1   # the A layout needs M % 128 == 0
    assert size(7, 128, 128, 64) == -1
    assert size(L.RL_A_BF16, 128, 100, 64) == -1


@pytest.mark.parametrize("args,code", [
    ((6144, 1536, 32, 8), L.RL_OK),
    ((9216, 4352, 24, 24), L.RL_OK),
    ((6144 - 8, 1536, 32, 8), L.RL_ERR_ALIGN),
    ((6144, 1536, 32, 0), L.RL_ERR_SHAPE),
    ((6144, 1500, 32, 8), L.RL_ERR_SHAPE),
])
def test_validate_qkv_post_gqa(args, code):
    assert L.lib().rl_validate_qkv_post_gqa(*args) == code


def test_qkv_post_gqa_null_pointers_rejected_before_any_gpu_call():
    assert L.lib().rl_qkv_post_gqa(None, 6144, 64, 32, 8, None, None, None, None, None, None, None, None, None,
                                   None) == L.RL_ERR_NULL
