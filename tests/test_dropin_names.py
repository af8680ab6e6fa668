"""Host-side parts of the drop-in boundary: the attention artifacts' parameters read from their names, and the
GEMM's K found from its three buffers (no GPU needed)."""

import torch

from rlbfp import forward as FW
from rlbfp import run_attn


def test_attention_artifact_names():
    """The parameters read from the reference's artifact names (redline/forward.py:273-275, :472-487, :529-530,
    :592; tools/programs.json)."""
    m = run_attn.attn_meta("attn32o-v6-s-h32-t8-pf-nk8256-nkv8224")
    assert (m["KVSPLIT"], m["PT"], m["P0"], m["NK"], m["NKV"], m.get("Q0", 0)) == (64, 136, 0, 8256, 8224, 0)
    m = run_attn.attn_meta("attn32o-v6-s-h32-t8-tr-nk8256-nkv8224")
    assert (m["QT"], m["Q0"], m["KT"], m["K0"], m["PT"], m["P0"]) == (136, 66, 136, 66, 136, 0)
    m = run_attn.attn_meta("attn32o-v6-a-h32-t8-tr-nk4160-nvrt3", {3: 8})
    assert ("KVSPLIT" not in m, m["Q0"], m["K0"], m["NKV"]) == (True, 0, 0, 4104)
    m = run_attn.attn_meta("attn32o-v6-s-h32-t8-tr72-nk4288-nvrt2--nv5")
    assert (m["QT"], m["Q0"], m["NKV"]) == (72, 8, 4229)
    m = run_attn.attn_meta("attn32q-v6-t8-nk512-pt72")
    assert (m["family"], m["NK"], m["PT"]) == ("attn32q", 512, 72)
    assert run_attn.attn_meta("vlm-attn-m1536-t17-x")["NQT"] == 17


def test_gemm_k_from_buffer_sizes():
    """K from the value counts of A (M K), B (K N) and C (M N, or M N / 2 after SwiGLU); V9 streams hold 8 values per
    9 bytes, bf16 tensors one per element."""
    a = torch.empty(4096 * 3072 // 8 * 9, dtype=torch.uint8)
    b = torch.empty(3072 * 24576 // 8 * 9, dtype=torch.uint8)
    h = torch.empty(4096 * 12288 // 8 * 9, dtype=torch.uint8)
    assert FW.gemm_k(a, b, h, swiglu=True) == 3072
    c16 = torch.empty(1536 * 4096, dtype=torch.bfloat16)
    a2 = torch.empty(1536 * 4096 // 8 * 9, dtype=torch.uint8)
    b2 = torch.empty(4096 * 4096 // 8 * 9, dtype=torch.uint8)
    assert FW.gemm_k(a2, b2, c16, swiglu=False) == 4096
    try:
        FW.gemm_k(a2, b, c16, swiglu=False)
    except ValueError:
        pass
    else:
        raise AssertionError("inconsistent sizes must raise")
