"""The host helpers of redline/run_attn.py over the HIP attention pass rl_attention (device tensors in and out).

The reference feeds its attention artifacts packed bfp16 tiles (redline/run_attn.py:27-34, :67-82):
  Q: per head, consecutive MQ-query tiles a_layout(Q_t * log2(e)/sqrt(128), MQ, 128);
  KV: per head K0 V0 K1 V1 ... with K tile = b_layout(K_t^T, 128, NT) and V tile = b_layout(V_t, NT, 128), NT keys each.
``pack_q`` / ``pack_kv`` write those bytes on the GPU; ``unpack_q`` / ``unpack_kv`` decode them into the native operands
of ops.attention (Q and K head major, V transposed); ``attn_npu`` runs the pass on packed buffers and returns O per
head, like the reference's. The artifact's compile-time parameters come as its meta dict (or a directory holding
meta.json): MQ, NK, NT and optionally NKV, OA, OHEADS, H0.
"""

import json
import re
from pathlib import Path

import numpy as np
import torch

from . import layouts, ops

D = 128
C_LOG2 = float(np.log2(np.e) / np.sqrt(D))


def _meta(art):
    if isinstance(art, dict):
        return art
    return json.loads((Path(art) / "meta.json").read_text())


def _blocks(x):
    """(R, 128) or (128, R) values -> bfp16 bytes of its rows' 8-column blocks, as (R * C / 8, 9)."""
    return ops.quantize(x.contiguous())[0].reshape(-1, 9)


def pack_q(q, mq):
    """q (H, NQ, 128) with the score scale already folded in -> per head, consecutive a_layout(., mq, 128) tiles."""
    H, NQ, _ = q.shape
    idx = layouts.a_block_index(mq, D, mq, D, q.device)
    out = torch.empty((H, NQ // mq, mq * D // 8, 9), dtype=torch.uint8, device=q.device)
    for h in range(H):
        for t in range(NQ // mq):
            out[h, t, idx] = _blocks(q[h, t * mq:(t + 1) * mq])
    return out.reshape(-1)


def pack_kv(k, v, nt):
    """k, v (NK, 128) of one head -> K0 V0 K1 V1 ...: K tile = b_layout(K_t^T, 128, nt), V tile = b_layout(V_t, nt,
    128), each bfp16 (redline/run_attn.py:27-34)."""
    nk = k.shape[0]
    ik = layouts.b_block_index(D, nt, D, nt, k.device)    # block (dim block kb, key c) at kb * nt + c
    iv = layouts.b_block_index(nt, D, nt, D, k.device)    # block (key block kb, dim c) at kb * 128 + c
    out = torch.empty((nk // nt, 2, nt * D // 8, 9), dtype=torch.uint8, device=k.device)
    for i in range(nk // nt):
        kt, vt = k[i * nt:(i + 1) * nt], v[i * nt:(i + 1) * nt]
        # K^T blocks (8 dims of one key) are K's row blocks; V blocks (8 keys of one dim) are V^T's row blocks
        out[i, 0, ik] = _blocks(kt).reshape(nt, D // 8, 9).transpose(0, 1).reshape(-1, 9)
        out[i, 1, iv] = _blocks(vt.t()).reshape(D, nt // 8, 9).transpose(0, 1).reshape(-1, 9)
    return out.reshape(-1)


def unpack_q(q_pack, H, NQ, mq):
    """Packed Q tiles -> q (H, NQ, 128) bf16."""
    t = q_pack.reshape(H, NQ // mq, -1)
    return torch.stack([torch.cat([layouts.a_unlayout(t[h, i], mq, D, mq, D) for i in range(NQ // mq)])
                        for h in range(H)]).to(torch.bfloat16)


def unpack_kv(kv_pack, H, NK, nt):
    """Packed per-head K/V tiles -> k (H, NK, 128) and vt (H, 128, NK), bf16."""
    t = kv_pack.reshape(H, NK // nt, 2, -1)
    k = torch.stack([torch.cat([layouts.b_unlayout(t[h, i, 0], D, nt, D, nt).t() for i in range(NK // nt)])
                     for h in range(H)])
    vt = torch.stack([torch.cat([layouts.b_unlayout(t[h, i, 1], nt, D, nt, D) for i in range(NK // nt)]).t()
                      for h in range(H)])
    return k.to(torch.bfloat16).contiguous(), vt.to(torch.bfloat16).contiguous()


def attn_npu(art, q_pack, kv_pack, H, NQ, MQ):
    """Run attention on packed bfp16 bytes: q_pack = per head, MQ-query a_layout tiles of Q * log2(e)/sqrt(D) in
    order; kv_pack = per head K0 V0 K1 V1 ... (pack_kv format), or a [target, prefix] pair of such packs (each per
    head, the reference's KVSPLIT buffers). Returns O (H, NQ, D) float32 (redline/run_attn.py:67-82); with OA in the
    meta, O passes through the bfp16 out-projection operand (each 8-dim block quantized), as the reference's OA
    artifacts write it."""
    meta = _meta(art)
    NK, NT = meta["NK"], meta["NT"]
    NKV = meta.get("NKV") or NK
    q = unpack_q(q_pack, H, NQ, MQ)
    if isinstance(kv_pack, (list, tuple)):
        parts = [p.reshape(H, -1) for p in kv_pack]
        kv_pack = torch.cat(parts, 1).reshape(-1)
    k, vt = unpack_kv(kv_pack, H, NK, NT)
    o = ops.attention(q, k, vt, nkv=NKV, quantize_out=bool(meta.get("OA")))
    return o.float().reshape(NQ, H, D).permute(1, 0, 2).contiguous()


# ---------------------------------------------------------------------------------------------------------------
# NPU.run("attn" | "attn_ref" | "attn_small", art, args): the artifacts' buffer contracts on rl_attention
# ---------------------------------------------------------------------------------------------------------------

TILE9 = 64 * D // 8 * 9          # bytes of one 64-token Q, K or V tile
# first target Q / KV tile of the step-1 layouts, by tiles per head T = M / 64: the edit layout (M 8704, target from
# row 4224) and the text-to-image layout (M 4608, target from row 512) (redline/forward.py:29, :452)
Q0_BY_T = {8704 // 64: 4224 // 64, 4608 // 64: 512 // 64}
_NUM = re.compile(r"^([a-z]+?)(\d*)$")


def attn_meta(art, nv=None):
    """The compile-time parameters of an attention artifact, keyed as its meta.json (family, H, W, MQ, NT, NK, NKV,
    OA, OHEADS, H0, KVSPLIT, QT, Q0, KT, K0, PT, P0; "causal" family: M, NQT), from the artifact names that
    redline/forward.py and redline/vlm_run.py use (forward.py:273-275, :472-487, :496-530, :592; vlm_run.py:177,
    vlm_encode.py:26):
      attn32o-v6-{s|a}-h{H}-t{tau}-{pf|tr}[T]-nk{NK}[-nkv{NKV}][-nvrt{id}][--nv{nv}]   (s: two KV buffers,
          KVSPLIT = 64 target tiles then the prefix; a: one buffer; pf: prefix tiles 0.. of a T-tile buffer; tr: Q and
          KV as tile ranges of the step-1 buffers, from the target's first tile (s) or from tile 0 (a))
      attn32q-v6-t{tau}-nk{NK}-pt{PT}     small-query mode, per-query key limits
      vlm-attn-m{M}-t{NQT}-x              the text encoder's causal GQA attention
    nv: {NVRT marker id: valid keys of the last tile} (forward.NPU.set_nv). A dict is returned unchanged."""
    if isinstance(art, dict):
        return dict(art)
    name = Path(str(art)).name
    nv_rt = None
    if "--nv" in name:
        name, tail = name.split("--nv", 1)
        nv_rt = int(tail)
    m = re.match(r"vlm-attn-m(\d+)-t(\d+)", name)
    if m:
        return {"family": "causal", "M": int(m.group(1)), "NQT": int(m.group(2)), "MQ": 64, "NT": 64}
    toks = name.split("-")
    fam = toks[0]
    if fam not in ("attn32o", "attn32", "attn32q"):
        raise KeyError(f"{art}: not an attention artifact name")
    meta = {"family": fam, "MQ": 64, "NT": 64, "H": 32, "W": 2, "OA": int(fam != "attn32"), "OHEADS": 32, "H0": 0}
    vals, flags = {}, set()
    for t in toks[1:]:
        mm = _NUM.match(t)
        if not mm:
            continue
        if mm.group(2):
            vals[mm.group(1)] = int(mm.group(2))
        else:
            flags.add(mm.group(1))
    meta["NK"] = vals["nk"]
    if fam == "attn32q":
        meta.update(OA=1, PT=vals.get("pt", meta["NK"] // 64), P0=0)
        return meta
    meta["H"] = vals.get("h", 32)
    split = "s" in flags
    if split:
        meta["KVSPLIT"] = 64
    T = vals.get("tr", vals.get("pf", 8704 // 64 if ("tr" in flags or "pf" in flags) else 0))
    if "tr" in flags or "tr" in vals:
        first = Q0_BY_T[T] if split else 0
        meta.update(QT=T, Q0=first, KT=T, K0=first)
        if split:
            meta.update(PT=T, P0=0)
    elif "pf" in flags or "pf" in vals:
        meta.update(PT=T, P0=0)
    nkv = vals.get("nkv")
    marker = vals.get("nvrt")
    if nv_rt is not None:
        nkv = meta["NK"] - 64 + nv_rt
    elif marker is not None and nv and marker in nv:
        nkv = meta["NK"] - 64 + int(nv[marker])
    meta["NKV"] = nkv or meta["NK"]
    return meta


def _q_tiles(buf, heads, t_all, t0, n):
    """Q tiles t0..t0+n-1 of a [head][t_all][tile] buffer -> (heads, 64 n, 128) bf16."""
    raw = buf.reshape(heads, t_all, TILE9)[:, t0:t0 + n].reshape(-1)
    return layouts.a_unlayout(raw, heads * n * 64, D, 64, D).reshape(heads, n * 64, D).to(torch.bfloat16)


def _kv_tiles(buf, heads, t_all, t0, n):
    """K / V tiles t0..t0+n-1 of a [head][t_all][K | V][tile] buffer -> k (heads, 64 n, 128), v (heads, 64 n, 128)."""
    t = buf.reshape(heads, t_all, 2, TILE9)[:, t0:t0 + n]
    kt = layouts.b_unlayout(t[:, :, 0].reshape(-1), D, heads * n * 64, D, 64)   # K^T of all heads side by side
    v = layouts.b_unlayout(t[:, :, 1].reshape(-1), heads * n * 64, D, 64, D)
    return kt.t().reshape(heads, n * 64, D), v.reshape(heads, n * 64, D)


def _write_a_rows(out, o, rows_all, cols_all, col0):
    """Rows 0..len(o)-1 of O_all (rows_all x cols_all), columns col0.., as bfp16 blocks of the out-projection's A
    operand to_bfp16(a_layout(O_all, 128, 64)) in the flat uint8 buffer `out`; other blocks are left as they are.
    o holds exact bfp16 values (attention's quantize_out), so re-encoding them is exact."""
    n, c = o.shape
    blocks = ops.quantize(o.contiguous())[0].reshape(-1, 9)
    idx = layouts.a_block_index(rows_all, cols_all, 128, 64, out.device).reshape(rows_all, cols_all // 8)
    out.reshape(-1, 9)[idx[:n, col0 // 8:(col0 + c) // 8].reshape(-1)] = blocks


def _write_c_tiles(out, o, heads, nq):
    """O (heads, nq, 128) -> bf16 C tiles [head][tile][64 x 128], each c_layout(tile, 64, 128): 16-row bands, 16-column
    bands, 8-row halves, 8-column halves, row, column (redline/run_attn.py:38-41)."""
    t = o.reshape(heads, nq // 64, 4, 2, 8, 8, 2, 8)          # h, tile, sbr, br, rib, sbc, bc, cib
    out.reshape(-1).copy_(t.permute(0, 1, 2, 5, 3, 6, 4, 7).reshape(-1).to(torch.bfloat16))


def run_artifact(meta, args):
    """Run one attention artifact's contract on its NPU buffers (uint8 bfp16 streams, written in place):
      attn32 / attn32o: [Q, KV, O] or, with KVSPLIT, [Q, KV target, KV prefix, O] (attn_design.py:131-281);
      attn32q: [Q, LIM, KV, O] (attn_design.py:284-366);
      causal: [Q, KV, O] (kernels/vlm/attn_causal_design.py:1-10).
    Q / K / V are decoded from their tiles and the product runs on rl_attention."""
    fam = meta["family"]
    if meta.get("MQ", 64) != 64 or meta.get("NT", 64) != 64:
        raise ValueError("64-token Q and KV tiles expected")
    if fam == "causal":
        return _run_causal(meta, *args)
    if fam == "attn32q":
        return _run_small(meta, *args)
    H, nk = meta["H"], meta["NK"]
    nqt = meta.get("QN") or meta.get("W", 2) * 32          # Q tiles per head of this call
    split = meta.get("KVSPLIT", 0)
    nkt = nk // 64
    parts = [split or nkt] + ([nkt - split] if split else [])
    geo = [(meta.get("KT") or parts[0], meta.get("K0", 0))]
    if split:
        geo.append((meta.get("PT") or parts[1], meta.get("P0", 0)))
    q_buf, kv_bufs, o_buf = args[0], list(args[1:-1]), args[-1]
    if len(kv_bufs) != len(geo):
        raise ValueError(f"{len(geo) + 2} buffers expected")
    q = _q_tiles(q_buf, H, meta.get("QT") or nqt, meta.get("Q0", 0), nqt)
    ks, vs = zip(*(_kv_tiles(b, H, t_all, t0, n) for b, (t_all, t0), n in zip(kv_bufs, geo, parts)))
    k = torch.cat(ks, 1).to(torch.bfloat16).contiguous()
    vt = torch.cat(vs, 1).transpose(1, 2).to(torch.bfloat16).contiguous()
    oa = bool(meta.get("OA"))
    o = ops.attention(q.contiguous(), k, vt, nkv=meta.get("NKV") or nk, quantize_out=oa)
    if oa:
        oh, h0 = meta.get("OHEADS", 32), meta.get("H0", 0)
        _write_a_rows(o_buf, o, nqt * 64, oh * D, h0 * D)
    else:
        _write_c_tiles(o_buf, o.reshape(nqt * 64, H, D).permute(1, 0, 2), H, nqt * 64)


def _run_small(meta, Q, LIM, KV, O):
    """attn32q: one 64-query tile per head; query row i sees keys j <= LIM[i]; K / V tiles P0.. of a [head][PT][K|V]
    buffer; O rows 0..63 of a_layout((128, OHEADS * 128), 128, 64)."""
    H = meta.get("H", 32)
    nkt = meta["NK"] // 64
    q = _q_tiles(Q, H, 1, 0, 1)
    lim = LIM.reshape(-1)[:4 * 64].view(torch.int32)
    k, v = _kv_tiles(KV, H, meta.get("PT") or nkt, meta.get("P0", 0), nkt)
    qp = torch.zeros((H, 128, D), dtype=torch.bfloat16, device=Q.device)
    qp[:, :64] = q
    lp = torch.zeros(128, dtype=torch.int32, device=Q.device)
    lp[:64] = lim.clamp(0, meta["NK"] - 1)
    o = ops.attention(qp, k.to(torch.bfloat16).contiguous(), v.transpose(1, 2).to(torch.bfloat16).contiguous(),
                      lim=lp, quantize_out=True)
    _write_a_rows(O, o[:64], 128, meta.get("OHEADS", 32) * D, meta.get("H0", 0) * D)


def _run_causal(meta, Q, KV, O):
    """The text encoder's causal GQA attention: Q (HQ, T, tile), KV (HKV, T, K|V, tile), q head h on kv head
    h // (HQ / HKV); the first NQT tiles are computed with key j visible to query i when j <= i, and written to their
    rows of O = a_layout((M, HQ * 128), 128, 64); the other rows stay as they are."""
    M, nqt = meta["M"], meta["NQT"]
    T = M // 64
    hq, hkv = Q.numel() // (T * TILE9), KV.numel() // (T * 2 * TILE9)
    n = nqt * 64
    nq = -(-n // 128) * 128
    q = torch.zeros((hq, nq, D), dtype=torch.bfloat16, device=Q.device)
    q[:, :n] = _q_tiles(Q, hq, T, 0, nqt)
    k, v = _kv_tiles(KV, hkv, T, 0, nqt)
    kp = torch.zeros((hkv, nq, D), dtype=torch.bfloat16, device=Q.device)
    vp = torch.zeros_like(kp)
    kp[:, :n], vp[:, :n] = k, v
    g = hq // hkv
    kp, vtp = kp.repeat_interleave(g, 0).contiguous(), vp.transpose(1, 2).repeat_interleave(g, 0).contiguous()
    lim = torch.arange(nq, dtype=torch.int32, device=Q.device)
    o = ops.attention(q, kp, vtp, lim=lim, quantize_out=True)
    _write_a_rows(O, o[:n], M, hq * D, 0)
