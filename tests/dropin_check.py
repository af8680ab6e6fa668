"""Op-by-op checker for the reference's NPU call sequences replayed through the mirror (rlbfp.forward.NPU.run and
rlbfp.vlm_run.run): a recording NPU keeps every op's buffers before and after it ran, and ``check_op`` compares each
op's outputs with the oracle applied to the inputs it was given. Used by the GPU tests only."""

import numpy as np
import torch

from oracle import attn as AT
from oracle import bfp16 as F
from oracle import gemm as G
from oracle import ln as LN
from oracle import qkv as QK
from rlbfp import forward as FW

TILE9 = 9216


class RecordingNPU(FW.NPU):
    """forward.NPU that synchronises after every op and keeps copies of its buffers before and after."""

    def __init__(self, *a, **k):
        super().__init__(*a, **k)
        self.log = []

    def run(self, op, art, args):
        before = [t.clone() for t in args]
        super().run(op, art, args)
        torch.cuda.synchronize()
        self.log.append((op, str(art), before, [t.clone() for t in args]))


def host(t):
    return t.float().cpu().numpy() if t.dtype != torch.uint8 else t.cpu().numpy()


def stream_values(t, M, N, order):
    """A C / A buffer -> (M, N) float values: V9 bytes in `order`, flat bf16 in the C-stream order, or 2-D bf16."""
    if t.dtype == torch.uint8:
        v = F.from_bfp16(host(t).reshape(-1))
        return F.a_unlayout(v, M, N) if order == "a" else F.c_unlayout_atb(v, M, N)
    if t.dim() == 1:
        return F.c_unlayout_atb(host(t), M, N)
    return host(t)


def close_values(got, ref_q, frac=0.999):
    """Quantized values of the same 8-value blocks: >= frac equal, every other block within one quantization step."""
    got, ref_q = np.asarray(got, np.float64).reshape(-1), np.asarray(ref_q, np.float64).reshape(-1)
    eq = got == ref_q
    assert eq.mean() >= frac, f"{(~eq).sum()} of {eq.size} differ"
    m = np.abs(np.stack([got, ref_q])).reshape(2, -1, 8).max(2).max(0)
    step = 2.0 ** (np.floor(np.log2(np.maximum(m, 1e-30))) - 6)
    assert (np.abs(got - ref_q).reshape(-1, 8).max(1) <= step * 1.0000001).all()


def check_gemm(before, after, swiglu, tol=1e-2):
    a, b, c = before[0], before[1], after[2]
    va, vb = a.numel() // 9 * 8, b.numel() // 9 * 8
    vc = (c.numel() // 9 * 8 if c.dtype == torch.uint8 else c.numel()) * (2 if swiglu else 1)
    K = int(round((va * vb / vc) ** 0.5))
    M, N = va // K, vb // K
    Aq = F.a_unlayout(F.from_bfp16(host(a)), M, K)
    Bq = F.decode_b(host(b), K, N)
    nout = N // 2 if swiglu else N
    got = stream_values(c, M, nout, "a" if swiglu else "c")
    ref = G.gemm_ref(Aq, Bq, act=G.ACT_SWIGLU if swiglu else G.ACT_NONE)
    if c.dtype == torch.uint8:   # the V9 C holds the bf16 result re-encoded in 8-column blocks
        ref = F.quantize_rows(ref)
    err = G.rel_err(got, ref)
    assert err <= tol, f"GEMM rel err {err}"
    assert G.corr(got, ref) > 0.9999
    return err


def check_ln(art, before, after, norm):
    x_in, br, p = before[0], before[1], before[2]
    xo, ao = after[3], after[4]
    d = p.numel() // 4
    M = x_in.numel() // d
    x = F.c_unlayout_atb(host(x_in), M, d)
    if br.dtype == torch.uint8:
        brv = F.c_unlayout_atb(F.from_bfp16(host(br)), M, d)
    else:
        brv = F.c_unlayout_atb(host(br), M, d)
    import re
    s = re.search(r"-s(\d+)(?:\D|$)", art)
    split = int(s.group(1)) * 128 if s else 0
    xr, yr = LN.ln_mod_ref(x, brv, host(p).reshape(2, 2 * d), split_row=split, norm=norm)
    np.testing.assert_array_equal(F.c_unlayout_atb(host(xo), M, d), xr)            # x' bit-exact
    y = F.a_unlayout(F.from_bfp16(host(ao)), M, d)
    close_values(y, F.quantize_rows(yr.astype(np.float32)))
    assert G.rel_err(y, yr) <= 1e-2


def check_qkv_post(before, after, cos, sin, wqc, wk):
    cin, tabs = before[0], before[1]
    q, kv = after[2], after[3]
    T = tabs.numel() // 8448
    M = 64 * T
    hq, hkv = q.numel() // (T * TILE9), kv.numel() // (T * 2 * TILE9)
    ncols = 128 * (hq + 2 * hkv)
    C = stream_values(cin, M, ncols, "c")
    Q, K, V = QK.qkv_post_ref(C, cos, sin, wqc, wk, hq, hkv)
    Qq, Kq, Vq = QK.quantize_qkv(Q, K, V)
    qn = host(q).reshape(hq, T, TILE9)
    kvn = host(kv).reshape(hkv, T, 2, TILE9)
    _, kv_ref = QK.tiles(Q[:1], K, V)
    np.testing.assert_array_equal(kvn[:, :, 1], kv_ref[:, :, 1])                  # V tiles bit-exact
    for h in range(hq):
        close_values(F.a_unlayout(F.from_bfp16(qn[h].ravel()), M, 128, 64, 128), Qq[h])
    for h in range(hkv):
        kd = F.b_unlayout(F.from_bfp16(kvn[h, :, 0].ravel()), 128, M, 128, 64).T
        close_values(kd, Kq[h])


def decode_q(buf, heads, t_all, t0, n):
    raw = host(buf).reshape(heads, t_all, TILE9)[:, t0:t0 + n]
    return np.stack([F.a_unlayout(F.from_bfp16(raw[h].ravel()), n * 64, 128, 64, 128) for h in range(heads)])


def decode_kv(buf, heads, t_all, t0, n):
    raw = host(buf).reshape(heads, t_all, 2, TILE9)[:, t0:t0 + n]
    k = np.stack([F.b_unlayout(F.from_bfp16(raw[h, :, 0].ravel()), 128, n * 64, 128, 64).T for h in range(heads)])
    v = np.stack([F.b_unlayout(F.from_bfp16(raw[h, :, 1].ravel()), n * 64, 128, 64, 128) for h in range(heads)])
    return k, v


def _kv_rows(buf, heads):
    """Every token row of a [head][tiles][K | V][tile] buffer: (K, V), each (heads, 64 tiles, 128)."""
    t_all = buf.numel() // (heads * 2 * TILE9)
    return decode_kv(buf, heads, t_all, 0, t_all)


def check_attn(meta, before, after):
    """O of an attention artifact against the oracle on its decoded tiles; blocks of O it does not own unchanged."""
    o_before, o_after = host(before[-1]).reshape(-1, 9), host(after[-1]).reshape(-1, 9)
    fam = meta["family"]
    if fam == "causal":
        Mr, nqt = meta["M"], meta["NQT"]
        T = Mr // 64
        hq, hkv = before[0].numel() // (T * TILE9), before[1].numel() // (T * 2 * TILE9)
        q = decode_q(before[0], hq, T, 0, nqt)
        k, v = decode_kv(before[1], hkv, T, 0, nqt)
        g = hq // hkv
        n = nqt * 64
        ref = AT.attention_ref(q, np.repeat(k, g, 0), np.repeat(v, g, 0), lim=np.arange(n))
        rows_all, cols_all, h0, nrows = Mr, hq * 128, 0, n
    elif fam == "attn32q":
        # one 64-query tile per head; keys = token rows [64 P0, 64 P0 + NK) of the KV buffer, whose tiles per head
        # come from its size
        H, nk = meta.get("H", 32), meta["NK"]
        q = decode_q(before[0], H, 1, 0, 1)
        lim = host(before[1]).reshape(-1)[:256].view(np.int32)
        k_all, v_all = _kv_rows(before[2], H)
        r0 = 64 * meta.get("P0", 0)
        assert r0 + nk <= k_all.shape[1]
        ref = AT.attention_ref(q, k_all[:, r0:r0 + nk], v_all[:, r0:r0 + nk], lim=lim)
        rows_all, cols_all, h0, nrows = 128, meta.get("OHEADS", 32) * 128, meta.get("H0", 0), 64
    else:
        # token rows, from the artifact's offsets and each buffer's own size (kernels/attn/attn_design.py:235-240):
        # queries [64 Q0, 64 (Q0 + QN)) of the Q buffer; keys [64 K0, 64 K0 + n1) of the first KV buffer, then
        # [64 P0, 64 P0 + NK - n1) of the second, n1 = 64 KVSPLIT (all NK keys from the first without a split)
        H, nk = meta["H"], meta["NK"]
        nq = 64 * (meta.get("QN") or meta.get("W", 2) * 32)
        q_all = decode_q(before[0], H, before[0].numel() // (H * TILE9), 0, before[0].numel() // (H * TILE9))
        q0 = 64 * meta.get("Q0", 0)
        assert q0 + nq <= q_all.shape[1]
        q = q_all[:, q0:q0 + nq]
        n1 = 64 * meta["KVSPLIT"] if meta.get("KVSPLIT") else nk
        ranges = [(64 * meta.get("K0", 0), n1)] + ([(64 * meta.get("P0", 0), nk - n1)] if n1 < nk else [])
        ks, vs = [], []
        for buf, (r0, n) in zip(before[1:-1], ranges):
            k_all, v_all = _kv_rows(buf, H)
            assert r0 + n <= k_all.shape[1]
            ks.append(k_all[:, r0:r0 + n])
            vs.append(v_all[:, r0:r0 + n])
        ref = AT.attention_ref(q, np.concatenate(ks, 1), np.concatenate(vs, 1), nkv=meta.get("NKV") or nk)
        rows_all, cols_all, h0, nrows = nq, meta.get("OHEADS", 32) * 128, meta.get("H0", 0), nq
    heads = ref.shape[0]
    pos = F.a_pos(*np.meshgrid(np.arange(rows_all), np.arange(0, cols_all, 8), indexing="ij"), rows_all, cols_all)
    blk = (pos // 8).reshape(rows_all, cols_all // 8)
    own = np.zeros(o_after.shape[0], bool)
    own[blk[:nrows, h0 * 16:(h0 + heads) * 16].reshape(-1)] = True
    np.testing.assert_array_equal(o_after[~own], o_before[~own])                  # other rows / heads untouched
    got_blocks = F.from_bfp16(o_after[blk[:nrows, h0 * 16:(h0 + heads) * 16].reshape(-1)].reshape(-1))
    got = got_blocks.reshape(nrows, heads, 128).transpose(1, 0, 2)
    err = G.rel_err(got, ref[:, :nrows])
    assert err <= 1e-2, f"attention rel err {err}"
    assert G.corr(got, ref[:, :nrows]) > 0.9999
    return err
