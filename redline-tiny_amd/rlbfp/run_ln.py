"""The host helpers of redline/run_ln.py over the HIP pass rl_ln_modulate (device tensors in and out).

``ln_pack_x`` / ``ln_pack_br`` / ``ln_params`` / ``ln_run`` / ``ln_unpack`` / ``rows_param`` keep the reference's
names and argument meanings (redline/run_ln.py:28-86). The residual stream x travels as bf16 in config3's C-stream
order (c_layout_atb(., 128, 128)) and the branch as bfp16 in the same order; x' comes back in that order and A as
bfp16 in the A layout (a_layout(., 128, 64)). ``ln_fused(art, X, BR, P, XO, AO)`` is the op itself with the argument
list of kernels/glue/ln_design.py:38 (the one ``NPU.run("ln_mod", art, args)`` dispatches to). It also takes the
build's native row-major forms: 2-D bf16 X / XO / branch, and a 2-D bf16 AO that receives A as bf16 for the next
rl_bfp16_gemm.

The artifact name carries the compile-time parameters, as ``glue-ln-m{M}-s{S}`` does (redline/forward.py:205, :466):
S is the number of 128-row M-tiles that take parameter row 1. A name containing "rms" selects RMSNorm (the kernels/vlm
copies); anything else selects LayerNorm.
"""

import re

import torch

from . import layouts, ops

D = 4096  # hidden width of the reference DiT (redline/run_ln.py:23); the functions below take D from their inputs


def art_params(art):
    """(S, norm) from an artifact name like 'glue-ln-m8704-s33' or 'vlm-rms-m1536'."""
    m = re.search(r"-s(\d+)(?:\D|$)", art)
    return (int(m.group(1)) if m else 0), ("rms" if "rms" in art else "layer")


def ln_pack_x(x):
    """Residual stream (M, D) -> bf16 in config3's C-stream order (redline/run_ln.py:28-30)."""
    return layouts.c_layout_atb_values(x.to(torch.bfloat16))


def ln_pack_br(br):
    """Branch (M, D) -> bfp16 in config3's C-stream order (redline/run_ln.py:33-35)."""
    return ops.quantize(br.contiguous(), order="c_atb")[0]


def ln_params(g, sc):
    """g, sc: (2, D) rows [real t, t = 0] -> the 2 x 2D bf16 parameter buffer (redline/run_ln.py:38-40)."""
    return torch.cat([g.float(), sc.float()], 1).to(torch.bfloat16).reshape(-1)


def rows_param(v, M, S):
    """Per-row parameter (M, D) from 2 rows: M-tiles < S use row 1 (redline/run_ln.py:82-86)."""
    out = v[0:1].repeat(M, 1)
    out[: S * 128] = v[1]
    return out


def ln_fused(art, X, BR, P, XO, AO):
    """x' = bf16(x + g * BR), A = LayerNorm(x') * sc (or RMSNorm) as bfp16; see the module docstring for the forms."""
    S, norm = art_params(art)
    d = P.numel() // 4
    stream = X.dim() == 1
    M = X.numel() // d
    x = layouts.c_unlayout_atb_values(X, M, d) if stream else X
    if BR is None:
        br = None
    elif BR.dtype == torch.uint8:
        br = ops.dequantize(BR, M, d, order="c_atb", dtype=torch.bfloat16) if stream else BR
    elif BR.dim() == 1:
        br = layouts.c_unlayout_atb_values(BR, M, d)  # bf16 branch in C order (kernels/vlm/rms16_mod.cc)
    else:
        br = BR
    packed = AO.dtype == torch.uint8
    x_out = XO if XO.dim() == 2 else None
    xp, a_p, a_d = ops.ln_modulate(x, P.reshape(2, 2 * d), branch=br, split_row=S * 128, norm=norm, x_out=x_out,
                                   packed=packed, a_order="a_layout", deq=not packed)
    if x_out is None:
        XO.copy_(layouts.c_layout_atb_values(xp))
    if packed:
        AO.copy_(a_p)
    else:
        AO.copy_(a_d)


def ln_run(art, xc, brc, p, iters=0, warmup=0):
    """Run once (or warmup + iters for timing). Returns (x' bf16 C stream, A bfp16 bytes in the A layout, list of
    device times in us) (redline/run_ln.py:43-57)."""
    xo = torch.zeros_like(xc)
    ao = torch.zeros(xc.numel() // 8 * 9, dtype=torch.uint8, device=xc.device)
    us = []
    for i in range(max(1, warmup + iters)):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        ln_fused(art, xc, brc, p, xo, ao)
        e1.record()
        if i >= warmup:
            e1.synchronize()
            us.append(e0.elapsed_time(e1) * 1e3)
    torch.cuda.current_stream().synchronize()
    return xo, ao, us


def ln_unpack(xo, ao, M):
    """-> x' (M, D) and y (M, D) float32 (redline/run_ln.py:60-63)."""
    d = xo.numel() // M
    return (layouts.c_unlayout_atb_values(xo, M, d).float(),
            ops.dequantize(ao, M, d, order="a_layout"))
