"""Tensor-level entry points over librlbfp: quantize / dequantize, the packed-weight GEMM with its fused epilogues,
grouped GEMMs, the GEMV, the residual + LayerNorm/RMSNorm + modulate pass that produces a GEMM's A, the QKV post pass
(per-head RMSNorm + RoPE -> attention tiles) and attention. Inputs are torch tensors on a ROCm device (gfx950);
outputs are allocated here with torch's caching allocator (or passed in) and the work is enqueued on torch's current
stream.

Packed streams are uint8 tensors of 9 bytes per 8 values. Packed weights are the bytes redline/pack_weights.py writes:
to_bfp16(b_layout(W.T, 64, 128)) of a Linear weight W (N, K).
"""

import ctypes

import torch

from . import _lib as L

ORDERS = {"rowblock": L.RL_ORDER_ROWBLOCK, "a_layout": L.RL_ORDER_A_LAYOUT, "b_layout": L.RL_ORDER_B_LAYOUT,
          "c_atb": L.RL_ORDER_C_ATB}
A_FORMATS = {"bf16": L.RL_A_BF16, "bf16_quantize": L.RL_A_BF16_QUANTIZE, "packed_rowblock": L.RL_A_PACKED_ROWBLOCK,
             "packed_a_layout": L.RL_A_PACKED_A_LAYOUT}
ACTS = {None: L.RL_ACT_NONE, "none": L.RL_ACT_NONE, "gelu_tanh": L.RL_ACT_GELU_TANH, "swiglu": L.RL_ACT_SWIGLU}


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _dev(t, name):
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise TypeError(f"{name} must be a torch tensor on a ROCm device")
    return t


def packed_bytes(rows, cols):
    """Bytes of a packed stream of rows x cols values."""
    if cols % 8:
        raise ValueError("cols must be a multiple of 8")
    return rows * cols // 8 * 9


# ---------------------------------------------------------------------------------------------------------------
# quantize / dequantize
# ---------------------------------------------------------------------------------------------------------------

def quantize(x, order="rowblock", packed=True, deq=False):
    """Encode an (R, C) float32 or bf16 tensor to bfp16 blocks of 8 consecutive columns, bit-exact to
    npu_layouts.to_bfp16 (redline/npu_layouts.py:62-73) applied to the layout `order`.

    Returns (packed uint8 [R*C/8*9] or None, deq bf16 (R, C) or None); ``deq`` holds the decoded values, which
    rl_bfp16_gemm consumes directly (a_fmt="bf16")."""
    _dev(x, "x")
    if x.dim() != 2 or x.dtype not in (torch.float32, torch.bfloat16) or x.stride(1) != 1:
        raise ValueError("x must be a 2-D float32/bfloat16 tensor with unit column stride")
    R, C = x.shape
    p = torch.empty(packed_bytes(R, C), dtype=torch.uint8, device=x.device) if packed else None
    q = torch.empty((R, C), dtype=torch.bfloat16, device=x.device) if deq else None
    dt = L.RL_DTYPE_BF16 if x.dtype == torch.bfloat16 else L.RL_DTYPE_F32
    L.check(L.lib().rl_bfp16_quantize(_ptr(x), dt, R, C, x.stride(0), ORDERS[order], _ptr(p), _ptr(q), _stream(x)))
    return p, q


def dequantize(packed, rows, cols, order="rowblock", dtype=torch.float32):
    """Decode a packed stream back to an (rows, cols) tensor (exact); for order "b_layout" the result is W (N, K)."""
    _dev(packed, "packed")
    out = torch.empty((rows, cols), dtype=dtype, device=packed.device)
    dt = L.RL_DTYPE_BF16 if dtype == torch.bfloat16 else L.RL_DTYPE_F32
    L.check(L.lib().rl_bfp16_dequantize(_ptr(packed), ORDERS[order], rows, cols, _ptr(out), dt, _stream(packed)))
    return out


def pack_weight(W):
    """Linear weight W (N, K) on the device -> the packed B stream of B = W.T, byte-identical to
    pack_weights.pack_b(W.T) (redline/pack_weights.py:72-79)."""
    p, _ = quantize(W, order="b_layout")
    return p


def interleave_up(wg, wp):
    """gate / proj weights (F, K) -> the Linear weight (2F, K) whose transpose is pack_weights.interleave_up's B:
    rows [gate 64 | proj 64] per group of 128 (redline/pack_weights.py:82-89)."""
    F, K = wg.shape
    if wp.shape != (F, K) or F % 64:
        raise ValueError("gate and proj must both be (F, K) with F % 64 == 0")
    return torch.stack([wg.reshape(F // 64, 64, K), wp.reshape(F // 64, 64, K)], 1).reshape(2 * F, K)


# ---------------------------------------------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------------------------------------------

def _epilogue(act, bias, gate, gate_split_row, residual, quantize_out):
    ep = L.Epilogue()
    ep.act = ACTS[act]
    ep.flags = L.RL_EP_QUANTIZE_OUT if quantize_out else 0
    for name, t, dt in (("bias", bias, torch.float32), ("gate", gate, torch.float32),
                        ("residual", residual, torch.bfloat16)):
        if t is not None:
            _dev(t, name)
            if t.dtype != dt or not t.is_contiguous() and name != "residual":
                raise ValueError(f"{name} must be a contiguous {dt} tensor")
    ep.bias = bias.data_ptr() if bias is not None else None
    ep.gate = gate.data_ptr() if gate is not None else None
    ep.gate_split_row = int(gate_split_row)
    if residual is not None:
        if residual.dim() != 2 or residual.stride(1) != 1:
            raise ValueError("residual must be 2-D with unit column stride")
        ep.residual = residual.data_ptr()
        ep.ld_residual = residual.stride(0)
    return ep


def _check_ep_sizes(M, N, nout, bias, gate, gate_split_row, residual):
    """Sizes the kernel reads from the epilogue vectors (the C ABI takes bare pointers)."""
    if bias is not None and bias.numel() != N:
        raise ValueError(f"bias must hold N = {N} values")
    if gate is not None and gate.numel() != (2 * nout if gate_split_row > 0 else nout) \
            and not (gate_split_row == 0 and gate.numel() == 2 * nout):
        raise ValueError(f"gate must hold {nout} values ({2 * nout} with gate_split_row > 0)")
    if residual is not None and (residual.shape[0] < M or residual.shape[1] < nout):
        raise ValueError(f"residual must be at least ({M}, {nout})")


def _a_args(a, a_fmt, M, K):
    if a_fmt in ("bf16", "bf16_quantize"):
        if a.dtype != torch.bfloat16 or a.dim() != 2 or a.stride(1) != 1 or a.shape[1] != K:
            raise ValueError(f"A must be a (M, {K}) bfloat16 tensor with unit column stride")
        return a.stride(0)
    if a.dtype != torch.uint8 or a.numel() != packed_bytes(M, K):
        raise ValueError(f"packed A must hold {packed_bytes(M, K)} bytes")
    return K


_GEMM_WS = {}


def gemm_workspace_bytes(M, N, K, device=None, a_fmt="bf16"):
    """Bytes of rl_bfp16_gemm_ws's workspace for this shape and A format: the K-split partials (0: the shape runs
    whole), plus the staged bf16 copy of A for a non-bf16 format; cached per shape."""
    key = (M, N, K, a_fmt, torch.cuda.current_device() if device is None else torch.device(device).index)
    if key not in _GEMM_WS:
        n = L.lib().rl_bfp16_gemm_workspace_size(A_FORMATS[a_fmt], M, N, K)
        if n < 0:
            raise ValueError(f"invalid GEMM shape M={M} N={N} K={K} for A format {a_fmt}")
        _GEMM_WS[key] = n
    return _GEMM_WS[key]


def staged_a_bytes(M, K):
    """Bytes of the bf16 A copy rl_bfp16_gemm_ws stages for a non-bf16 A format (rounded up to 256)."""
    return (M * K * 2 + 255) // 256 * 256


PACKED_ORDERS = {"c_atb": L.RL_ORDER_C_ATB, "a_layout": L.RL_ORDER_A_LAYOUT}
C_ORDERS = {"rowmajor": L.RL_C_ROWMAJOR, "c_atb": L.RL_C_ATB}


def gemm(a, b_packed, N, K, M=None, a_fmt="bf16", act=None, bias=None, gate=None, gate_split_row=0,
         residual=None, quantize_out=False, out=None, split=True, workspace=True, packed_out=None,
         packed_order="c_atb", c_order="rowmajor"):
    """C = epilogue(A @ B) with B the packed weight stream of a (K, N) matrix, bf16 output (M, N) (or (M, N/2) for
    act="swiglu"). See rl_bfp16_gemm in include/rlbfp.h for the epilogue order. split: let a small-M, deep-K GEMM
    split K into pieces (rl_bfp16_gemm_ws, workspace from torch's allocator); False: always whole K. An A format
    other than "bf16" is decoded (or quantized) into a bf16 copy first, then the bf16 kernel runs; workspace: that
    copy (and any K split) lives in a workspace from torch's allocator; False: rl_bfp16_gemm takes a stream-ordered
    allocation of its own (not allowed under graph capture).
    packed_out: a uint8 tensor of 9 M Nout / 8 bytes that the epilogue fills with to_bfp16 of the bf16 output in
    packed_order ("c_atb": the reference GEMM's C stream; "a_layout": the next GEMM's A, as the SwiGLU GEMM writes H);
    with packed_out and no out, no bf16 C is written and packed_out is returned. c_order="c_atb": the bf16 C is flat
    (M * Nout values) in the c_layout_atb element order (the C16 artifacts' output)."""
    _dev(a, "A")
    _dev(b_packed, "B")
    if M is None:
        if a_fmt not in ("bf16", "bf16_quantize"):
            raise ValueError("M is required for packed A")
        M = a.shape[0]
    lda = _a_args(a, a_fmt, M, K)
    if b_packed.dtype != torch.uint8 or b_packed.numel() != packed_bytes(K, N):
        raise ValueError(f"B must be a uint8 stream of {packed_bytes(K, N)} bytes")
    nout = N // 2 if act == "swiglu" else N
    if packed_out is not None:
        _dev(packed_out, "packed_out")
        if packed_out.dtype != torch.uint8 or not packed_out.is_contiguous() or \
                packed_out.numel() != packed_bytes(M, nout):
            raise ValueError(f"packed_out must be a contiguous uint8 tensor of {packed_bytes(M, nout)} bytes")
        if packed_order not in PACKED_ORDERS:
            raise ValueError(f"packed_order must be one of {sorted(PACKED_ORDERS)}")
    if c_order not in C_ORDERS:
        raise ValueError(f"c_order must be one of {sorted(C_ORDERS)}")
    no_c = out is None and packed_out is not None
    if c_order == "c_atb":
        if out is None and not no_c:
            out = torch.empty(M * nout, dtype=torch.bfloat16, device=a.device)
        if out is not None and (out.dtype != torch.bfloat16 or not out.is_contiguous() or out.numel() != M * nout):
            raise ValueError(f"out in the ATB order must be a contiguous bfloat16 tensor of {M * nout} values")
        ldc = nout
    else:
        if out is None and not no_c:
            out = torch.empty((M, nout), dtype=torch.bfloat16, device=a.device)
        if out is not None and (out.dtype != torch.bfloat16 or out.shape != (M, nout) or out.stride(1) != 1):
            raise ValueError(f"out must be ({M}, {nout}) bfloat16 with unit column stride")
        ldc = out.stride(0) if out is not None else nout
    _check_ep_sizes(M, N, nout, bias, gate, gate_split_row, residual)
    ep = _epilogue(act, bias, gate, gate_split_row, residual, quantize_out)
    if packed_out is not None:
        ep.packed_out = packed_out.data_ptr()
        ep.packed_order = PACKED_ORDERS[packed_order]
    ep.c_order = C_ORDERS[c_order]
    c_ptr = ctypes.c_void_p(out.data_ptr()) if out is not None else None
    if not workspace:
        nws = 0
    elif a_fmt == "bf16":
        nws = gemm_workspace_bytes(M, N, K, a.device) if split else 0
    else:
        nws = gemm_workspace_bytes(M, N, K, a.device, a_fmt) if split else staged_a_bytes(M, K)
    if nws and not split:
        ep.flags |= L.RL_EP_WHOLE_K  # a non-bf16 A staged in the workspace, the product whole K
    if nws:
        ws = torch.empty(nws, dtype=torch.uint8, device=a.device)
        L.check(L.lib().rl_bfp16_gemm_ws(_ptr(a), A_FORMATS[a_fmt], lda, _ptr(b_packed), c_ptr, ldc, M, N, K,
                                         ctypes.byref(ep), _ptr(ws), nws, _stream(a)))
    else:
        L.check(L.lib().rl_bfp16_gemm(_ptr(a), A_FORMATS[a_fmt], lda, _ptr(b_packed), c_ptr, ldc, M, N, K,
                                      ctypes.byref(ep), _stream(a)))
    return out if out is not None else packed_out


class GemmSpec:
    """One GEMM of a grouped launch (same arguments as gemm()); A is in the group's format (gemm_grouped's a_fmt),
    and M is required when that format is packed."""

    def __init__(self, a, b_packed, N, K, act=None, bias=None, gate=None, gate_split_row=0, residual=None,
                 quantize_out=False, out=None, M=None):
        self.a, self.b, self.N, self.K = a, b_packed, N, K
        self.M = a.shape[0] if M is None else M
        self.ep_args = (act, bias, gate, gate_split_row, residual, quantize_out)
        nout = N // 2 if act == "swiglu" else N
        self.out = out if out is not None else torch.empty((self.M, nout), dtype=torch.bfloat16, device=a.device)


def gemm_grouped(specs, a_fmt="bf16"):
    """Several independent GEMMs in one launch; returns their outputs."""
    if not 1 <= len(specs) <= L.RL_MAX_GROUP:
        raise ValueError(f"1..{L.RL_MAX_GROUP} GEMMs per group")
    arr = (L.GemmDesc * len(specs))()
    keep = []
    for i, s in enumerate(specs):
        _dev(s.a, "A")
        M = s.M
        arr[i].A = s.a.data_ptr()
        arr[i].lda = _a_args(s.a, a_fmt, M, s.K)
        arr[i].B_packed = s.b.data_ptr()
        arr[i].C = s.out.data_ptr()
        arr[i].ldc = s.out.stride(0)
        arr[i].M, arr[i].N, arr[i].K = M, s.N, s.K
        act, bias, gate, split, res, _q = s.ep_args
        _check_ep_sizes(M, s.N, s.out.shape[1], bias, gate, split, res)
        arr[i].ep = _epilogue(*s.ep_args)
        keep.append(s)
    L.check(L.lib().rl_bfp16_gemm_grouped(arr, len(specs), A_FORMATS[a_fmt], _stream(specs[0].a)))
    return [s.out for s in specs]


# ---------------------------------------------------------------------------------------------------------------
# GEMV
# ---------------------------------------------------------------------------------------------------------------

def gemv(x, b_packed, N, act="silu", out=None):
    """y (M, N) bf16 = Q(act(x)) @ B for 1 <= M <= 8, x (M, K) bf16, act "silu" or None evaluated in fp32, Q the
    bfp16 activation encoding (blocks of 8 along K); fp32 accumulation."""
    _dev(x, "x")
    _dev(b_packed, "B")
    if x.dim() != 2 or x.dtype != torch.bfloat16 or x.stride(1) != 1:
        raise ValueError("x must be a 2-D bfloat16 tensor with unit column stride")
    M, K = x.shape
    if b_packed.dtype != torch.uint8 or b_packed.numel() != packed_bytes(K, N):
        raise ValueError(f"B must be a uint8 stream of {packed_bytes(K, N)} bytes")
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    code = L.RL_GEMV_SILU if act == "silu" else L.RL_ACT_NONE
    L.check(L.lib().rl_bfp16_gemv(_ptr(x), x.stride(0), _ptr(b_packed), _ptr(out), out.stride(0), M, N, K, code,
                                  _stream(x)))
    return out


# ---------------------------------------------------------------------------------------------------------------
# residual add + LayerNorm / RMSNorm + modulate -> A
# ---------------------------------------------------------------------------------------------------------------

_NORMS = {"layer": L.RL_NORM_LAYER, "rms": L.RL_NORM_RMS}
_A_ORDERS = {"rowblock": L.RL_ORDER_ROWBLOCK, "a_layout": L.RL_ORDER_A_LAYOUT}


def ln_modulate(x, params, branch=None, split_row=0, norm="layer", x_out=None, packed=True, a_order="rowblock",
                deq=True):
    """x' = bf16(x + g * branch) and y = norm(x') * sc quantized to bfp16, per row of x (M, D) bf16.

    params: (2, 2D) bf16, row p = [g (D) | sc (D)]; rows < split_row use row 1, the rest row 0. branch: (M, D) bf16,
    or a uint8 stream of bfp16 blocks in row-block order (9 * M * D / 8 bytes), or None. norm: "layer" (mean and
    variance, eps 1e-6) or "rms". x_out: where x' goes (may be x itself; None allocates). Returns (x', A packed bytes
    in a_order or None, A as bf16 or None); see rl_ln_modulate in include/rlbfp.h."""
    _dev(x, "x")
    _dev(params, "params")
    if x.dim() != 2 or x.dtype != torch.bfloat16 or x.stride(1) != 1:
        raise ValueError("x must be a 2-D bfloat16 tensor with unit column stride")
    M, D = x.shape
    if params.dtype != torch.bfloat16 or params.numel() != 4 * D or not params.is_contiguous():
        raise ValueError(f"params must be a contiguous bfloat16 (2, {2 * D}) tensor")
    br_fmt, ld_br = L.RL_BRANCH_BF16, D
    if branch is not None:
        _dev(branch, "branch")
        if branch.dtype == torch.uint8:
            if branch.numel() != packed_bytes(M, D):
                raise ValueError(f"a packed branch must hold {packed_bytes(M, D)} bytes")
            br_fmt = L.RL_BRANCH_PACKED
        elif branch.dtype == torch.bfloat16 and branch.shape == (M, D) and branch.stride(1) == 1:
            ld_br = branch.stride(0)
        else:
            raise ValueError("branch must be (M, D) bfloat16 or a uint8 bfp16 stream")
    if x_out is None:
        x_out = torch.empty_like(x)
    elif x_out.dtype != torch.bfloat16 or x_out.shape != (M, D) or x_out.stride(1) != 1:
        raise ValueError("x_out must be (M, D) bfloat16 with unit column stride")
    a_p = torch.empty(packed_bytes(M, D), dtype=torch.uint8, device=x.device) if packed else None
    a_d = torch.empty((M, D), dtype=torch.bfloat16, device=x.device) if deq else None
    L.check(L.lib().rl_ln_modulate(_ptr(x), x.stride(0), _ptr(branch), br_fmt, ld_br, _ptr(params), split_row,
                                   _NORMS[norm], _ptr(x_out), x_out.stride(0), _ptr(a_p), _A_ORDERS[a_order],
                                   _ptr(a_d), D, M, D, _stream(x)))
    return x_out, a_p, a_d


# ---------------------------------------------------------------------------------------------------------------
# QKV post -> attention Q / K / V
# ---------------------------------------------------------------------------------------------------------------

def qkv_post(C, cos, sin, wq, wk, heads, tiles=True, native=False, kv_heads=None, out_tiles=None):
    """Per head of 128 dims: Q = rope(rms(q) * wq), K = rope(rms(k) * wk), V = v, quantized to bfp16 (Q, K in blocks
    of 8 dims, V in blocks of 8 tokens). C (M, (heads + 2 * kv_heads) * 128) bf16 (kv_heads None: = heads; fewer for
    grouped-query attention); cos, sin (M, 64) bf16; wq, wk (128,) bf16.
    Returns (q_tiles (heads, M/64, 9216) uint8, kv_tiles (kv_heads, M/64, 2, 9216) uint8) if tiles, else None, None;
    then, if native, q (heads, M, 128), k (kv_heads, M, 128) and v transposed, (kv_heads, 128, M), bf16, else
    None x 3. out_tiles: a (q_tiles, kv_tiles) pair of caller-owned uint8 tensors of those sizes to write instead.
    See rl_qkv_post_gqa in include/rlbfp.h."""
    for t, n in ((C, "C"), (cos, "cos"), (sin, "sin"), (wq, "wq"), (wk, "wk")):
        _dev(t, n)
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{n} must be bfloat16")
    hkv = heads if kv_heads is None else kv_heads
    M = C.shape[0]
    if C.dim() != 2 or C.stride(1) != 1 or C.shape[1] != 128 * (heads + 2 * hkv):
        raise ValueError(f"C must be (M, {128 * (heads + 2 * hkv)}) with unit column stride")
    if cos.shape != (M, 64) or sin.shape != (M, 64) or not cos.is_contiguous() or not sin.is_contiguous():
        raise ValueError("cos and sin must be contiguous (M, 64)")
    if wq.numel() != 128 or wk.numel() != 128 or not wq.is_contiguous() or not wk.is_contiguous():
        raise ValueError("wq and wk must be contiguous 128-vectors")
    T = M // 64
    if out_tiles is not None:
        qt, kvt = out_tiles
        for t, n, want in ((qt, "q tiles", heads * T * 9216), (kvt, "kv tiles", hkv * T * 2 * 9216)):
            _dev(t, n)
            if t.dtype != torch.uint8 or t.numel() != want or not t.is_contiguous():
                raise ValueError(f"{n} must be a contiguous uint8 tensor of {want} bytes")
    elif tiles:
        qt = torch.empty((heads, T, 9216), dtype=torch.uint8, device=C.device)
        kvt = torch.empty((hkv, T, 2, 9216), dtype=torch.uint8, device=C.device)
    else:
        qt = kvt = None
    q, k, v = ((torch.empty((heads, M, 128), dtype=torch.bfloat16, device=C.device),
                torch.empty((hkv, M, 128), dtype=torch.bfloat16, device=C.device),
                torch.empty((hkv, 128, M), dtype=torch.bfloat16, device=C.device)) if native else (None, None, None))
    L.check(L.lib().rl_qkv_post_gqa(_ptr(C), C.stride(0), M, heads, hkv, _ptr(cos), _ptr(sin), _ptr(wq), _ptr(wk),
                                    _ptr(qt), _ptr(kvt), _ptr(q), _ptr(k), _ptr(v), _stream(C)))
    return qt, kvt, q, k, v


# ---------------------------------------------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------------------------------------------

def attention(q, k, vt, nkv=None, lim=None, out=None, h0=0, quantize_out=False, split=True):
    """O = softmax2(Q K^T) V per head: q (heads, nq, 128) with the score scale log2(e)/sqrt(128) folded in, k (heads,
    nk, 128), vt (heads, 128, nk) = V transposed, all bf16 (rl_qkv_post's native outputs). Keys j >= nkv, and j >
    lim[i] for query i when lim (nq int32) is given, are not visible. Returns out, (nq, ldo) bf16 with head h at
    columns (h0 + h) * 128 (allocated as (nq, heads * 128) if None); quantize_out rounds each 8-dim block to bfp16.
    With split (the default) the tasks left over after whole rounds of the GPU are split along the keys, with a
    workspace from torch's allocator (rl_attention_ws); split=False runs every task whole (rl_attention).
    See rl_attention and rl_attention_ws in include/rlbfp.h."""
    for t, n in ((q, "q"), (k, "k"), (vt, "vt")):
        _dev(t, n)
        if t.dtype != torch.bfloat16 or not t.is_contiguous():
            raise ValueError(f"{n} must be a contiguous bfloat16 tensor")
    heads, nq, d = q.shape
    nk = k.shape[1]
    if d != 128 or k.shape != (heads, nk, 128) or vt.shape != (heads, 128, nk):
        raise ValueError("q (heads, nq, 128), k (heads, nk, 128) and vt (heads, 128, nk) expected")
    if out is None:
        out = torch.empty((nq, (h0 + heads) * 128), dtype=torch.bfloat16, device=q.device)
    elif out.dtype != torch.bfloat16 or out.shape[0] != nq or out.stride(1) != 1:
        raise ValueError("out must be (nq, ldo) bfloat16 with unit column stride")
    if lim is not None:
        _dev(lim, "lim")
        if lim.dtype != torch.int32 or lim.numel() != nq or not lim.is_contiguous():
            raise ValueError("lim must be a contiguous int32 tensor of nq entries")
    nbytes = L.lib().rl_attention_workspace_bytes(heads, nq, nk) if split else 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device) if nbytes > 0 else None
    L.check(L.lib().rl_attention_ws(_ptr(q), _ptr(k), _ptr(vt), heads, nq, nk, nk if nkv is None else nkv, _ptr(lim),
                                    _ptr(out), out.stride(0), h0, 1 if quantize_out else 0, _ptr(ws), max(nbytes, 0),
                                    _stream(q)))
    return out
