"""The reference's own call sequences replayed through the mirror, op by op against the oracle:
  * CachedStep.embed / blocks / project (redline/forward.py:240-269): img_in, qkv, qkv_post, attn (two KV buffers,
    prefix from a larger buffer, key padding), o, ln_mod, up_swiglu, down, proj_out, all on the reference's V9 and
    flat bf16 buffers;
  * LM._layer (redline/vlm_run.py:427-449) with the text encoder's artifacts: rms / rms16, qkv / qkv16, the GQA
    qkv_post, causal GQA attention, o / o16, up+swiglu and the unfused up + swiglu glue, down / down16, x_out;
  * check_c16 (redline/vlm_run.py:95-120) at its own size;
  * the step-1 attention artifacts (tile ranges of the full Q / KV buffers, attn_ref, the small-query mode with
    per-row limits) and the V9-A GEMM staged in a workspace and in the library's own allocation.
Each op's outputs are compared with the oracle applied to the inputs it was given (tests/dropin_check.py)."""

import numpy as np
import pytest
import torch

from dropin_check import (TILE9, RecordingNPU, check_attn, check_gemm, check_ln, check_qkv_post, close_values, host,
                          stream_values)
from oracle import bfp16 as F
from oracle import gemm as G
from oracle import ln as LN
from oracle import qkv as QK
from rlbfp import forward as FW
from rlbfp import ops, pack, run_attn, vlm_run as V

pytestmark = pytest.mark.gpu


def cuda(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t.to(dtype) if dtype is not None else t


def rope_tables(rng, M):
    ang = rng.uniform(-np.pi, np.pi, (M, 64))
    return F.bf16_round(np.cos(ang).astype(np.float32)), F.bf16_round(np.sin(ang).astype(np.float32))


def kv_pack(rng, heads, tiles, scale=1.0):
    """A [head][tiles][K | V][tile] buffer of random keys and values (the prefix cache of a cached step)."""
    K = rng.standard_normal((heads, tiles * 64, 128)) * scale
    V = rng.standard_normal((heads, tiles * 64, 128))
    _, kv = QK.tiles(K[:1], K, V)
    return kv


def check_log(log, cos, sin, metas, norm):
    seen = set()
    for op, art, before, after in log:
        seen.add(op)
        if op in ("ln_mod", "rms"):
            check_ln(art, before, after, norm)
        elif op == "qkv_post":
            wqc, wk = id_of(before[1])
            check_qkv_post(before, after, cos, sin, wqc, wk)
        elif op.startswith("attn"):
            check_attn(metas(art), before, after)
        elif op == "swiglu":
            check_swiglu_glue(art, before, after)
        else:
            check_gemm(before, after, swiglu=op in ("up_swiglu", "up+swiglu"))
    return seen


_TABS = {}


def id_of(tabs):
    """The (wqc, wk) pair a TABS buffer was built with, found by its last 256 bf16 values."""
    key = tuple(host(tabs).reshape(-1)[-256:].tolist())
    return _TABS[key]


def remember_tables(tabs, wqc, wk):
    _TABS[tuple(host(tabs).reshape(-1)[-256:].tolist())] = (wqc, wk)


def check_swiglu_glue(art, before, after):
    import re
    M = int(re.search(r"-m(\d+)", art).group(1))
    n2 = before[0].numel() // 9 * 8
    Fh = n2 // (2 * M)
    v = stream_values(before[0], M, 2 * Fh, "c").astype(np.float64).reshape(M, Fh // 64, 2, 64)
    ref = (G.silu(v[:, :, 0]) * v[:, :, 1]).reshape(M, Fh)
    got = stream_values(after[1], M, Fh, "a")
    close_values(got, F.quantize_rows(F.bf16_round_f64(ref)), frac=0.995)


def test_cached_step_blocks(dev):
    """CachedStep.embed, two blocks and project at 512 rows x 1024 hidden (8 heads), FFN 2048, prefix cache of 7 tiles
    with 20 padded keys."""
    rng = np.random.default_rng(0)
    M, HID, FF, H = 512, 1024, 2048, 8
    mats = {}
    for i in range(2):
        mats[i, "qkv"] = F.pack_b(G.linear_weight(rng, 3 * HID, HID).T)
        mats[i, "o"] = F.pack_b(G.linear_weight(rng, HID, HID).T)
        mats[i, "up"] = F.pack_b(F.interleave_up(G.linear_weight(rng, FF, HID), G.linear_weight(rng, FF, HID)))
        mats[i, "down"] = F.pack_b(G.linear_weight(rng, HID, FF).T)
    mats["img_in"] = F.pack_b(G.linear_weight(rng, HID, 64, std=0.2).T)
    mats["proj_out"] = F.pack_b(G.linear_weight(rng, 1024, HID).T)
    w = FW.Weights.from_tensors({k: cuda(v) for k, v in mats.items()})
    for i in range(2):
        w.b[i, "norm_q"] = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
        w.b[i, "norm_k"] = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    cos, sin = rope_tables(rng, M)
    npu = RecordingNPU()
    art = "attn-test-pf"
    meta = {"family": "attn32o", "H": H, "QN": M // 64, "MQ": 64, "NT": 64, "NK": M + 7 * 64, "NKV": M + 7 * 64 - 20,
            "OA": 1, "OHEADS": H, "H0": 0, "KVSPLIT": M // 64, "PT": 12, "P0": 0}
    npu.meta[art] = meta
    cs = FW.CachedStep(w, cos, sin, lambda n, q, kvt, kvp, o: n.run("attn", art, [q, kvt, kvp, o]), M=M, n_blocks=2)
    for i in range(2):
        wqc = F.bf16_round(w.b[i, "norm_q"].astype(np.float32) * np.float32(QK.C_LOG2))
        remember_tables(cs.tabs[i], wqc, F.bf16_round(w.b[i, "norm_k"]))
    cs.set_t(0.3 * rng.standard_normal((2, 4 * HID)), 0.2 * rng.standard_normal((2, HID)))
    lat = rng.standard_normal((M, 64)).astype(np.float32)
    kv_prefix = {i: cuda(kv_pack(rng, H, 12, scale=0.3)).reshape(-1) for i in range(2)}
    cs.embed(npu, cuda(F.to_bfp16(F.a_layout(lat))))
    cs.blocks(npu, kv_prefix, 0, 1)
    v = cs.project(npu)
    assert v.shape == (M, 64)
    seen = check_log(npu.log, cos, sin, lambda a: meta, "layer")
    assert seen == {"img_in", "ln_mod", "qkv", "qkv_post", "attn", "o", "up_swiglu", "down", "proj_out"}
    assert npu.calls["qkv"] == 2 and npu.calls["ln_mod"] == 5


def test_extract_step_blocks(dev):
    """ExtractStep.blocks' op list for one block (redline/forward.py:362-388) through NPU.run at 1024 rows x 1024
    hidden (8 heads), FFN 2048, on the reference's V9 and flat bf16 buffers: qkv, qkv_post, the step-1 attention
    ("attn" for the target Q tiles 8..15 over their own keys and the prefix tiles 0..7 with 40 padded keys, "attn_ref"
    for Q tiles 0..7 over the prefix, "attn_small" for one 64-query group with per-row key limits), o, ln_mod with the
    step-1 parameter split (glue-ln-m1024-s3: rows below 384 take parameter row 1, as glue-ln-m8704-s33 does at
    M = 8704), up_swiglu, down and the closing ln_mod. Every op is checked against the oracle on the inputs it was
    given. The host-side merge of the small-query rows (ExtractStep._small_q / _merge_small) is orchestration, not a
    device op, and is not replayed."""
    rng = np.random.default_rng(4)
    M, HID, FF, H = 1024, 1024, 2048, 8
    T = M // 64
    mats = {(0, "qkv"): F.pack_b(G.linear_weight(rng, 3 * HID, HID).T),
            (0, "o"): F.pack_b(G.linear_weight(rng, HID, HID).T),
            (0, "up"): F.pack_b(F.interleave_up(G.linear_weight(rng, FF, HID), G.linear_weight(rng, FF, HID))),
            (0, "down"): F.pack_b(G.linear_weight(rng, HID, FF).T)}
    w = FW.Weights.from_tensors({k: cuda(v) for k, v in mats.items()})
    w.b[0, "norm_q"] = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    w.b[0, "norm_k"] = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    cos, sin = rope_tables(rng, M)
    # the buffers and per-step parameters of a step at M rows (CachedStep allocates the same V9 / flat bf16 set)
    ex = FW.CachedStep(w, cos, sin, None, M=M, n_blocks=1)
    wqc = F.bf16_round(w.b[0, "norm_q"].astype(np.float32) * np.float32(QK.C_LOG2))
    remember_tables(ex.tabs[0], wqc, F.bf16_round(w.b[0, "norm_k"]))
    ex.set_t(0.3 * rng.standard_normal((2, 4 * HID)), 0.2 * rng.standard_normal((2, HID)))
    x0 = F.bf16_round(rng.standard_normal((M, HID)).astype(np.float32) * 2)
    ex.x[0].copy_(cuda(F.c_layout_atb(x0), torch.bfloat16))
    ex.a.copy_(cuda(F.to_bfp16(F.a_layout(rng.standard_normal((M, HID)).astype(np.float32)))))
    npu = RecordingNPU()
    pad = 40
    metas = {
        "s1": {"family": "attn32o", "H": H, "QN": 8, "NK": 16 * 64, "NKV": 16 * 64 - pad, "OA": 1, "OHEADS": H,
               "H0": 0, "KVSPLIT": 8, "QT": T, "Q0": 8, "KT": T, "K0": 8, "PT": T, "P0": 0},
        "ref": {"family": "attn32o", "H": H, "QN": 8, "NK": 8 * 64, "NKV": 8 * 64 - pad, "OA": 1, "OHEADS": H,
                "H0": 0, "QT": T, "Q0": 0, "KT": T, "K0": 0},
        "small": {"family": "attn32q", "H": H, "NK": 8 * 64, "PT": T, "P0": 0, "OA": 1, "OHEADS": H, "H0": 0}}
    npu.meta.update(metas)
    strip = 128 * HID // 8 * 9                      # one 128-row strip of O (A layout)
    o_tgt, o_ref = ex.o[4 * strip:8 * strip], ex.o[:4 * strip]
    ln_art = "glue-ln-m1024-s3"
    # the block's op list, in ExtractStep.blocks' order
    FW.gemm(npu, w, "qkv", M, ex.a, ex.c_qkv, block=0)
    npu.run("qkv_post", "glue-qkv32-m1024", [ex.c_qkv, ex.tabs[0], ex.q, ex.kv])
    npu.run("attn", "s1", [ex.q, ex.kv, ex.kv, o_tgt])
    npu.run("attn_ref", "ref", [ex.q, ex.kv, o_ref])
    q_small = ex.q.reshape(H, T, TILE9)[:, 9:10].contiguous().reshape(-1)   # one query tile per head (rows 576..639)
    lim = np.concatenate([np.arange(16), rng.integers(0, 8 * 64 - pad - 1, 48)]).astype(np.int32)
    lim_buf = np.zeros(64 * 64 // 8 * 9, np.uint8)
    lim_buf[:256] = lim.view(np.uint8)
    o_small = FW.v9(128 * HID)
    npu.run("attn_small", "small", [q_small, cuda(lim_buf), ex.kv, o_small])
    FW.gemm(npu, w, "o", M, ex.o, ex.c, block=0)
    npu.run("ln_mod", ln_art, [ex.x[0], ex.c, ex.p_mlp, ex.x[1], ex.a])
    npu.run("up_swiglu", "atb3sw2-m1024", [ex.a, w.b[0, "up"], ex.h])
    FW.gemm(npu, w, "down", M, ex.h, ex.c, block=0)
    npu.run("ln_mod", ln_art, [ex.x[1], ex.c, ex.p_out, ex.x[0], ex.a])
    seen = check_log(npu.log, cos, sin, lambda art: metas[art], "layer")
    assert seen == {"qkv", "qkv_post", "attn", "attn_ref", "attn_small", "o", "ln_mod", "up_swiglu", "down"}
    # the parameter split really splits: rows below 384 and above it were normalised with different parameters
    lp = np.asarray(host(ex.p_mlp)).reshape(2, -1)
    assert not np.array_equal(lp[0], lp[1])


class _VlmW:
    pass


def vlm_weights(rng, layers, D, HQ, HKV, FF):
    w = _VlmW()
    w.w, w.qk, w.p_in, w.p_post = {}, {}, {}, {}
    for i in layers:
        w.w[i, "qkv"] = cuda(F.pack_b(G.linear_weight(rng, (HQ + 2 * HKV) * 128, D).T))
        w.w[i, "o"] = cuda(F.pack_b(G.linear_weight(rng, D, D).T))
        w.w[i, "up"] = cuda(F.pack_b(F.interleave_up(G.linear_weight(rng, FF, D), G.linear_weight(rng, FF, D))))
        w.w[i, "down"] = cuda(F.pack_b(G.linear_weight(rng, D, FF).T))
        qn, kn = 1 + 0.2 * rng.standard_normal(128), 3 * (1 + 0.2 * rng.standard_normal(128))
        w.qk[i] = tuple(t.cuda() for t in pack.balance_qk(qn, kn))
        w.p_in[i] = pack.rms_params(1 + 0.2 * rng.standard_normal(D))
        w.p_post[i] = pack.rms_params(1 + 0.2 * rng.standard_normal(D))
    w.hp = np.arange(D)
    return w


def test_lm_layers(dev, monkeypatch):
    """LM._layer twice at 512 rows x 2048 hidden, 16 q heads and 4 kv heads, FFN 2048, a 300-token prompt: layer 0
    with the bf16-C (C16) o / down GEMMs and the bf16-branch RMS glue; layer 1 with the bf16-C QKV GEMM, its QKV post
    and the unfused up GEMM + SwiGLU glue; then x_out."""
    rng = np.random.default_rng(1)
    M, D, HQ, HKV, FF, Lp = 512, 2048, 16, 4, 2048, 300
    wts = vlm_weights(rng, (0, 1), D, HQ, HKV, FF)
    cos, sin = rope_tables(rng, M)
    log = []
    orig = V.run

    def rec(art, args):
        before = [t.clone() for t in args]
        ms = orig(art, args)
        log.append((V._op(art), str(art), before, [t.clone() for t in args]))
        return ms

    monkeypatch.setattr(V, "run", rec)
    lm = V.LM(wts, cos, sin, m=M, hq=HQ, hkv=HKV, length=Lp)
    for i in (0, 1):
        wq, wk = (t.float().cpu().numpy() for t in wts.qk[i])
        remember_tables(lm.tabs[i], F.bf16_round(wq * np.float32(QK.C_LOG2)), F.bf16_round(wk))
    x = (rng.standard_normal((Lp, D)) * 2).astype(np.float32)
    x[:, 5] += 30
    lm.load_x(cuda(x))
    lm.c16_layers = {0}
    lm.layer(0)
    lm.qkv16, lm.fused_up = True, False
    lm.layer(1)
    out = lm.x_out(1)
    assert out.shape == (M, D)
    seen = check_log(log, cos, sin, lambda a: run_attn.attn_meta(a), "rms")
    assert seen == {"rms", "qkv", "qkv_post", "attn", "o", "up+swiglu", "up", "swiglu", "down"}
    assert set(lm.t) == seen


def test_check_c16(dev):
    """vlm_run.check_c16 at the reference's size (1536 x 4096): its own figures pass the reference's bars, and its
    buffers match the oracle (C16 GEMM within 1e-2, x' bit-exact, y within one quantization step)."""
    r = V.check_c16()
    assert r["c_err"] <= 1e-2 and r["c_corr"] > 0.9999 and r["x_exact"] and r["y_corr"] > 0.9999
    m, d = 1536, 4096
    rng = np.random.default_rng(3)
    a = rng.standard_normal((m, d)).astype(np.float32)
    b = (rng.standard_normal((d, d)) / 64).astype(np.float32)
    aq = F.quantize_rows(a)
    bq = F.decode_b(F.pack_b(b), d, d)
    c = F.c_unlayout_atb(host(r["c_t"]), m, d)
    assert G.rel_err(c, G.gemm_ref(aq, bq)) <= 1e-2
    x = (rng.standard_normal((m, d)) * 3).astype(np.float32)
    w = (1 + 0.2 * rng.standard_normal(d)).astype(np.float32)
    xr, yr = LN.ln_mod_ref(F.bf16_round(x), c, LN.rms_params(w), norm="rms")
    np.testing.assert_array_equal(F.c_unlayout_atb(host(r["xo_t"]), m, d), xr)
    close_values(F.a_unlayout(F.from_bfp16(host(r["ao_t"])), m, d), F.quantize_rows(yr.astype(np.float32)))


def test_step1_attention_artifacts(dev):
    """ExtractStep's attention calls on the full step-1 buffers, at 8 heads and T = 20 tiles per head (target Q / KV
    tiles 10..17, prefix tiles 0..8 with 40 padded keys): "attn" (two KV buffers, tile ranges), "attn_ref" (Q tiles
    0..7 over the prefix) and "attn_small" (one 64-query tile per head with per-row key limits), each against the
    oracle; O blocks outside a call's rows and heads stay as they were."""
    rng = np.random.default_rng(2)
    H, T = 8, 20
    Qv = rng.standard_normal((H, T * 64, 128)) * QK.C_LOG2 * 2
    q_buf = cuda(QK.tiles(Qv, Qv[:1], Qv[:1])[0]).reshape(-1)
    kv_buf = cuda(kv_pack(rng, H, T, scale=0.5)).reshape(-1)
    npu = RecordingNPU()
    npu.meta["s1"] = {"family": "attn32o", "H": H, "QN": 8, "NK": 8 * 64 + 9 * 64, "NKV": 8 * 64 + 9 * 64 - 40,
                      "OA": 1, "OHEADS": H, "H0": 0, "KVSPLIT": 8, "QT": T, "Q0": 10, "KT": T, "K0": 10, "PT": T,
                      "P0": 0}
    npu.meta["ref"] = {"family": "attn32o", "H": H, "QN": 8, "NK": 9 * 64, "NKV": 9 * 64 - 40, "OA": 1, "OHEADS": H,
                       "H0": 0, "QT": T, "Q0": 0, "KT": T, "K0": 0}
    npu.meta["small"] = {"family": "attn32q", "H": H, "NK": 9 * 64, "PT": T, "P0": 0, "OA": 1, "OHEADS": 2 * H,
                         "H0": H}
    o = cuda(rng.integers(0, 256, 18 * 64 * H * 128 // 8 * 9, dtype=np.uint8))
    tile_bytes = 128 * H * 128 // 8 * 9                      # one 128-row strip of O
    o_tgt = o[4 * tile_bytes:8 * tile_bytes]                   # 512 target rows from row 512
    o_ref = o[:4 * tile_bytes]
    npu.run("attn", "s1", [q_buf, kv_buf, kv_buf, o_tgt])
    npu.run("attn_ref", "ref", [q_buf, kv_buf, o_ref])
    qs = cuda(QK.tiles(Qv[:, :64], Qv[:1, :64], Qv[:1, :64])[0]).reshape(-1)
    lim = np.concatenate([np.arange(8), rng.integers(0, 9 * 64 - 41, 56)]).astype(np.int32)
    lim_buf = np.zeros(64 * 64 // 8 * 9, np.uint8)
    lim_buf[:256] = lim.view(np.uint8)
    o_small = cuda(rng.integers(0, 256, 128 * 2 * H * 128 // 8 * 9, dtype=np.uint8))
    npu.run("attn_small", "small", [qs, cuda(lim_buf), kv_buf, o_small])
    for op, art, before, after in npu.log:
        check_attn(npu.meta[art], before, after)


@pytest.mark.parametrize("M,K,N", [(4096, 3072, 3072), (512, 12288, 4096)])
def test_v9_a_staged_fast_path(dev, M, K, N):
    """A in the NPU's A layout (decoded to bf16, then the bf16 kernel). With a workspace from torch the call gets the
    bf16-A GEMM's bits on the decoded values, K split where the planner splits (the 512 x 12288 shape); in the
    library's own stream-ordered allocation (rl_bfp16_gemm, no workspace) and with split=False (RL_EP_WHOLE_K) it runs
    whole K, the bits of the whole-K bf16-A GEMM. All meet the oracle on sampled rows. The first shape is config 1's,
    the second the text encoder's down projection."""
    rng = np.random.default_rng(M + K)
    A = G.activations(rng, M, K)
    W = G.linear_weight(rng, N, K)
    a = cuda(F.to_bfp16(F.a_layout(A)))
    b = ops.pack_weight(cuda(W))
    fast = ops.gemm(a, b, N, K, M=M, a_fmt="packed_a_layout")
    own = ops.gemm(a, b, N, K, M=M, a_fmt="packed_a_layout", workspace=False)
    whole = ops.gemm(a, b, N, K, M=M, a_fmt="packed_a_layout", split=False)
    a16 = ops.dequantize(a, M, K, order="a_layout", dtype=torch.bfloat16)
    assert torch.equal(fast, ops.gemm(a16, b, N, K))
    assert torch.equal(own, whole)
    assert torch.equal(whole, ops.gemm(a16, b, N, K, split=False))
    rows = np.sort(rng.choice(M, 128, replace=False))
    Aq = F.quantize_rows(A[rows])
    Bq = F.decode_b(b.cpu().numpy(), K, N)
    ref = G.gemm_ref(Aq, Bq)
    for out in (fast, whole):
        got = out[torch.from_numpy(rows).cuda()].float().cpu().numpy()
        assert G.rel_err(got, ref) <= 1e-2
