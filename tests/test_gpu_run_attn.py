"""The run_attn call surface on the GPU (redline-tiny_amd/rlbfp/run_attn.py), the way redline/run_attn.py:186-226
checks its artifacts: Q and K/V packed as bfp16 tiles, O per head against float64 attention of the packed values."""

import numpy as np
import pytest
import torch

from oracle import attn as A
from oracle import bfp16 as F
from oracle import gemm as G
from rlbfp import run_attn

pytestmark = pytest.mark.gpu


def oracle_pack_kv(k, v, nt):
    """redline/run_attn.py:27-34 restated with the oracle's encoder and layouts."""
    out = []
    for i in range(0, k.shape[0], nt):
        out.append(F.to_bfp16(F.b_layout(np.ascontiguousarray(k[i:i + nt].T), 128, nt)))
        out.append(F.to_bfp16(F.b_layout(v[i:i + nt], nt, 128)))
    return np.concatenate(out)


@pytest.mark.parametrize("H,NQ,MQ,NK,NT,NKV", [(2, 256, 64, 512, 32, 512), (1, 128, 128, 384, 64, 360)])
def test_attn_npu(dev, H, NQ, MQ, NK, NT, NKV):
    rng = np.random.default_rng(H + NK)
    q = F.bf16_round(rng.standard_normal((H, NQ, 128)).astype(np.float32))
    k = F.bf16_round(rng.standard_normal((H, NK, 128)).astype(np.float32))
    v = F.bf16_round(rng.standard_normal((H, NK, 128)).astype(np.float32))
    k[:, NKV:] = 0
    v[:, NKV:] = 0
    tt = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    q_pack = run_attn.pack_q(tt(q * A.C_LOG2), MQ)
    kv_pack = torch.cat([run_attn.pack_kv(tt(k[h]), tt(v[h]), NT) for h in range(H)])
    # the GPU packers write the reference's bytes
    q_ref = np.concatenate([F.to_bfp16(F.a_layout(q[h, i:i + MQ] * A.C_LOG2, MQ, 128))
                            for h in range(H) for i in range(0, NQ, MQ)])
    np.testing.assert_array_equal(q_pack.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(kv_pack.cpu().numpy(), np.concatenate([oracle_pack_kv(k[h], v[h], NT)
                                                                         for h in range(H)]))
    meta = {"MQ": MQ, "NK": NK, "NT": NT, "NKV": NKV}
    o = run_attn.attn_npu(meta, q_pack, kv_pack, H, NQ, MQ).cpu().numpy()
    qd = run_attn.unpack_q(q_pack, H, NQ, MQ).float().cpu().numpy()
    kd, vtd = (x.float().cpu().numpy() for x in run_attn.unpack_kv(kv_pack, H, NK, NT))
    ref = A.attention_ref(qd, kd, vtd.transpose(0, 2, 1), nkv=NKV)
    assert G.rel_err(o, ref) <= 1e-2 and G.corr(o, ref) > 0.9999
    # the reference's own bar against attention of the unpacked float inputs (redline/run_attn.py:201-208)
    ref0 = A.attention_ref(q * A.C_LOG2, k, v, nkv=NKV)
    assert G.corr(o, ref0) > 0.995
