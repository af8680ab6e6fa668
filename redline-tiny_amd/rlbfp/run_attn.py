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
