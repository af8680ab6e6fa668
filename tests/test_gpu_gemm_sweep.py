"""A seeded sweep of GEMM shapes, epilogues and A formats against the CPU emulation, so that launch plans and
epilogue paths the fixed-shape tests do not name are covered too: M from 1 to a few thousand rows (partial last tiles,
one-round and multi-round launches, a second launch of shorter tiles, K splits), K a multiple of 64, N a multiple of
128, each with one epilogue (none, bias, tanh GELU, SwiGLU with or without the re-quantize, gate and residual with a
gate-row split) and one A format. Sampled rows (the first and last rows, both sides of 64-row boundaries and random
rows) are checked with the reference's metric, max |got - ref| / max |ref| <= 1e-2 (redline/run_glue.py:158-159; 2e-2
for a re-quantized output), and element-wise within 2 bf16 ulps for 99.9% of the values."""

import numpy as np
import pytest
import torch

from oracle import bfp16 as F
from oracle import gemm as G
from rlbfp import ops

pytestmark = pytest.mark.gpu

EPILOGUES = ["none", "bias", "gelu_tanh", "swiglu", "swiglu_q", "gate_residual"]
A_FORMATS = ["bf16", "bf16_quantize", "packed_rowblock", "packed_a_layout"]


def _cases(n=24, seed=2026):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        kind = i % 4
        if kind == 0:
            M = int(rng.integers(1, 200))
        elif kind == 1:
            M = int(rng.integers(200, 1500))
        elif kind == 2:
            M = 128 * int(rng.integers(1, 24))  # a multiple of 128, so the NPU a_layout A format applies
        else:
            M = int(rng.integers(1500, 4400))
        K = 64 * int(rng.integers(1, 33))
        N = 128 * int(rng.integers(1, 25))
        ep = EPILOGUES[i % len(EPILOGUES)]
        fmts = A_FORMATS if M % 128 == 0 else A_FORMATS[:3]
        out.append((M, K, N, ep, fmts[int(rng.integers(0, len(fmts)))], 100 + i))
    # deep K with few rows: the K-split planner's shapes
    out += [(96, 8192, 256, "bias", "bf16", 200), (384, 6144, 512, "swiglu_q", "bf16_quantize", 201),
            (512, 12288, 1024, "gate_residual", "bf16", 202)]
    return out


def _rows(M, rng):
    r = np.concatenate([np.arange(0, min(M, 8)), np.arange(max(0, M - 8), M),
                        np.array([b + d for b in range(64, M, 64) for d in (-1, 0)], dtype=np.int64),
                        rng.integers(0, M, 48)])
    r = np.unique(r[(r >= 0) & (r < M)])
    if r.size > 192:
        r = np.unique(np.concatenate([r[:16], r[-16:], rng.choice(r, 160, replace=False)]))
    return r


@pytest.mark.parametrize("M,K,N,ep,a_fmt,seed", _cases())
def test_sweep(dev, M, K, N, ep, a_fmt, seed):
    rng = np.random.default_rng(seed)
    A = G.activations(rng, M, K)
    Aq = F.quantize_rows(A)
    W = torch.from_numpy(G.linear_weight(rng, N, K)).cuda()
    packed = ops.pack_weight(W)                       # bit-exact to pack_b (tests/test_gpu_quantize.py)
    Bq = F.decode_b(packed.cpu().numpy(), K, N)
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).cuda().to(dt)

    kw, ref_kw = {}, {}
    nout = N // 2 if ep.startswith("swiglu") else N
    if ep == "bias":
        bias = (rng.standard_normal(N) * 0.5).astype(np.float32)
        kw, ref_kw = {"bias": t(bias, torch.float32)}, {"bias": bias}
    elif ep == "gelu_tanh":
        bias = (rng.standard_normal(N) * 0.5).astype(np.float32)
        kw = {"bias": t(bias, torch.float32), "act": "gelu_tanh"}
        ref_kw = {"bias": bias, "act": G.ACT_GELU_TANH}
    elif ep.startswith("swiglu"):
        kw = {"act": "swiglu", "quantize_out": ep == "swiglu_q"}
        ref_kw = {"act": G.ACT_SWIGLU, "quantize_out": ep == "swiglu_q"}
    gate = res = None
    split = 0
    if ep == "gate_residual":
        gate = rng.standard_normal((2, N)).astype(np.float32)
        res = F.bf16_round(rng.standard_normal((M, N)).astype(np.float32))
        split = int(rng.integers(0, M + 1))
        kw = {"gate": t(gate, torch.float32), "gate_split_row": split, "residual": t(res, torch.bfloat16)}

    if a_fmt == "bf16":
        a = t(Aq, torch.bfloat16)
    elif a_fmt == "bf16_quantize":
        a = t(A, torch.bfloat16)
    elif a_fmt == "packed_rowblock":
        a = t(F.to_bfp16(A.reshape(-1)), torch.uint8)
    else:
        a = t(F.to_bfp16(F.a_layout(A)), torch.uint8)
    out = ops.gemm(a, packed, N, K, M=M, a_fmt=a_fmt, **kw)
    assert out.shape == (M, nout)

    rows = _rows(M, rng)
    got = out[torch.from_numpy(rows).cuda()].float().cpu().numpy()
    if ep == "gate_residual":
        # the gate row depends on the global row index: rows below the split take gate row 1
        ref = np.where((rows < split)[:, None], G.gemm_ref(Aq[rows], Bq, gate=gate[[1, 1]], residual=res[rows]),
                       G.gemm_ref(Aq[rows], Bq, gate=gate[[0, 0]], residual=res[rows]))
    else:
        ref = G.gemm_ref(Aq[rows], Bq, **ref_kw)
    err = G.rel_err(got, ref)
    # a re-quantized output may land one bfp16 step of its block away where the fp32 sums straddle a rounding point
    # (half a step of a block whose largest element is ~1/64 of the output's largest: the tolerance of
    # tests/test_gpu_gemm.py::test_quantize_out)
    assert err <= (2e-2 if ep == "swiglu_q" else 1e-2), f"rel err {err}"
    d = np.abs(got.astype(np.float64) - ref)
    bound = 2 * np.abs(ref) * 2.0 ** -8 + 1e-4 * np.abs(ref).max()
    assert (d <= bound).mean() > 0.999, f"{(d > bound).sum()} of {d.size} elements off"
    if ep == "swiglu_q":
        # every 8-column block of the output is an exact bfp16 block: re-encoding changes nothing, except a block whose
        # largest magnitude is a -128 element (-2^k), which re-encodes one exponent up with q = -64
        blocks = got.reshape(-1, 8).astype(np.float64)
        same = (F.quantize_rows(got).reshape(-1, 8) == blocks).all(1)
        vmax = blocks[np.arange(len(blocks)), np.abs(blocks).argmax(1)]
        corner = (vmax < 0) & (np.frexp(-vmax)[0] == 0.5)
        assert same[~corner].all()


def _gemv_cases(n=16, seed=2027):
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 9)), 64 * int(rng.integers(1, 97)), 128 * int(rng.integers(1, 65)),
             "silu" if i % 2 == 0 else None, 300 + i) for i in range(n)]


@pytest.mark.parametrize("M,K,N,act,seed", _gemv_cases())
def test_gemv_sweep(dev, M, K, N, act, seed):
    """The adaLN GEMV over M = 1..8, K to 6144 and N to 8192 (partial last iteration groups of K tiles, lanes past the
    last K tile), against the emulation."""
    rng = np.random.default_rng(seed)
    x = F.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    W = torch.from_numpy(G.linear_weight(rng, N, K)).cuda()
    packed = ops.pack_weight(W)
    got = ops.gemv(torch.from_numpy(x).cuda().bfloat16(), packed, N, act=act).float().cpu().numpy()
    ref = G.gemv_ref(x, F.decode_b(packed.cpu().numpy(), K, N), act=act or "none")
    assert G.rel_err(got, ref) <= 1e-2
    d = np.abs(got.astype(np.float64) - ref)
    assert (d <= 2 * np.abs(ref) * 2.0 ** -8 + 1e-5 * np.abs(ref).max()).mean() > 0.999


def _group_cases(n=8, seed=2028):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        members = []
        for j in range(int(rng.integers(2, 5))):
            M = int(rng.choice([int(rng.integers(1, 300)), int(rng.integers(300, 2500))]))
            members.append((M, 64 * int(rng.integers(1, 25)), 128 * int(rng.integers(1, 17)),
                            [None, "swiglu", "gelu_tanh", "bias"][int(rng.integers(0, 4))]))
        out.append((members, 400 + i))
    # the DiT block's shape of grouping: a 4096-row image stream and a 256-row text stream with separate weights
    out.append(([(4096, 256, 2048, "swiglu"), (256, 256, 2048, "swiglu")], 450))
    return out


@pytest.mark.parametrize("members,seed", _group_cases())
def test_grouped_sweep(dev, members, seed):
    """Grouped launches of 2-4 members with different shapes and epilogues give the bits of the members' single
    launches, whichever way the planner runs the group (one 8-wave launch, or each member as its own plan)."""
    rng = np.random.default_rng(seed)
    specs, refs = [], []
    for M, K, N, ep in members:
        a = torch.from_numpy(F.quantize_rows(G.activations(rng, M, K))).cuda().bfloat16()
        b = ops.pack_weight(torch.from_numpy(G.linear_weight(rng, N, K)).cuda())
        kw = {"act": ep} if ep in ("swiglu", "gelu_tanh") else {}
        if ep in ("bias", "gelu_tanh"):
            kw["bias"] = torch.from_numpy((rng.standard_normal(N) * 0.5).astype(np.float32)).cuda()
        specs.append(ops.GemmSpec(a, b, N, K, **kw))
        refs.append(ops.gemm(a, b, N, K, split=False, **kw))
    for o, r in zip(ops.gemm_grouped(specs), refs):
        assert torch.equal(o, r)
