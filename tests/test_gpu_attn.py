"""GPU attention (rl_attention, rl_attention_ws) against the oracle (oracle/attn.py): fp32 scores and sums, P rounded
to bf16, bf16 out. Bar: max |O - O_ref| / max |O_ref| <= 1e-2 (the reference's metric, redline/run_glue.py:158-159)
and correlation > 0.9999 (the reference's own attention check accepts 0.995, redline/run_attn.py:208). With
quantize_out the stored O is an exact bfp16 block stream within one quantization step of the unquantized O.

Small shapes have fewer tasks than the GPU has resident workgroups, so with split=True (the default) their keys are
cut into pieces of 4 key blocks and merged by the combine launch; split=False runs every task whole."""

import numpy as np
import pytest
import torch

from oracle import attn as A
from oracle import bfp16 as F
from oracle import gemm as G
from oracle import qkv as QK
from rlbfp import ops

pytestmark = pytest.mark.gpu


def tt(a, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to("cuda").to(dtype)


def make(H, NQ, NK, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    q = F.bf16_round((rng.standard_normal((H, NQ, 128)) * A.C_LOG2 * scale).astype(np.float32))
    k = F.bf16_round(rng.standard_normal((H, NK, 128)).astype(np.float32))
    v = F.bf16_round(rng.standard_normal((H, NK, 128)).astype(np.float32))
    return rng, q, k, v


def run(q, k, v, **kw):
    vt = np.ascontiguousarray(v.transpose(0, 2, 1))
    return ops.attention(tt(q), tt(k), tt(vt), **kw)


def check(o_got, o_ref):
    assert G.rel_err(o_got, o_ref) <= 1e-2, G.rel_err(o_got, o_ref)
    assert G.corr(o_got, o_ref) > 0.9999


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("H,NQ,NK,NKV", [(1, 128, 64, 64), (2, 256, 320, 300), (3, 128, 1024, 1000),
                                         (1, 384, 2048, 2048), (1, 128, 4352, 4000)])
def test_attention(dev, H, NQ, NK, NKV, split):
    """(1, 128, 4352, 4000) splits one task into 17 pieces; its last ones see no key at all (merged with weight 0)."""
    rng, q, k, v = make(H, NQ, NK, H + NQ + NK, scale=2.0)
    o = run(q, k, v, nkv=NKV, split=split).float().cpu().numpy().reshape(NQ, H, 128).transpose(1, 0, 2)
    check(o, A.attention_ref(q, k, v, nkv=NKV))


@pytest.mark.parametrize("split", [True, False])
def test_limits_offset_and_quantize(dev, split):
    """Per-query key limits (row 0 sees one key: every piece but the first has none), an output wider than the heads
    (h0 = 2), and bfp16 output."""
    H, NQ, NK = 2, 256, 512
    rng, q, k, v = make(H, NQ, NK, 7)
    lim = rng.integers(0, NK, NQ).astype(np.int32)
    lim[:4] = [0, 1, 63, 64]
    out = torch.full((NQ, 6 * 128), 3.0, dtype=torch.bfloat16, device="cuda")
    run(q, k, v, lim=torch.from_numpy(lim).cuda(), out=out, h0=2, split=split)
    ref = A.attention_ref(q, k, v, lim=lim)
    got = out[:, 256:512].float().cpu().numpy().reshape(NQ, H, 128).transpose(1, 0, 2)
    check(got, ref)
    np.testing.assert_allclose(got[:, 0], v[:, 0], rtol=2 ** -8)  # query 0 sees key 0 only
    assert (out[:, :256] == 3.0).all() and (out[:, 512:] == 3.0).all()
    oq = run(q, k, v, lim=torch.from_numpy(lim).cuda(), quantize_out=True, split=split).float().cpu().numpy()
    of = run(q, k, v, lim=torch.from_numpy(lim).cuda(), split=split).float().cpu().numpy()
    # each 8-dim block is a bfp16 block (re-encoding it changes nothing outside the -128 corner), within one
    # quantization step of the unquantized output
    blocks = oq.reshape(-1, 8)
    same = (F.quantize_rows(oq) == oq).reshape(-1, 8).all(1)
    assert same.mean() > 0.995
    m = np.maximum(np.abs(blocks).max(1), np.abs(of.reshape(-1, 8)).max(1)).astype(np.float64)
    step = 2.0 ** (np.floor(np.log2(np.maximum(m, 1e-30))) - 6)
    assert (np.abs(blocks - of.reshape(-1, 8)).max(1) <= step * 1.0000001).all()


def test_full_size_dit_heads(dev):
    """4352 tokens x 24 heads (hidden 3072): 408 tasks of 256 queries, of which 152 (from head 15 on) are split along
    the keys on a 256-CU device. Heads 0 and 23 checked against the float64 oracle; every head of the split launch
    against the unsplit one (same arithmetic up to fp32 summation order); the split launch is deterministic."""
    H, N = 24, 4352
    rng, q, k, v = make(H, N, N, 0, scale=3.0)
    vt = tt(np.ascontiguousarray(v.transpose(0, 2, 1)))
    qt, kt = tt(q), tt(k)
    o_split = ops.attention(qt, kt, vt)
    o_whole = ops.attention(qt, kt, vt, split=False)
    assert torch.equal(o_split, ops.attention(qt, kt, vt))
    o = o_split.float().cpu().numpy().reshape(N, H, 128)
    for h in (0, 23):
        check(o[:, h], A.attention_ref(q[h:h + 1], k[h:h + 1], v[h:h + 1])[0])
    ow = o_whole.float().cpu().numpy()
    osp = o_split.float().cpu().numpy()
    assert np.abs(osp - ow).max() <= 2.0 ** -7 * np.abs(ow).max()
    # tasks that run whole in both launches (heads 0..14) are the same computation: bit-identical. Split tasks round
    # P to bf16 against each piece's own running max, so their last bits differ.
    np.testing.assert_array_equal(osp[:, :15 * 128], ow[:, :15 * 128])


def test_workspace_too_small(dev):
    from rlbfp import _lib as L
    H, N = 24, 4352
    need = L.lib().rl_attention_workspace_bytes(H, N, N)
    assert need > 0
    q = torch.zeros((H, N, 128), dtype=torch.bfloat16, device="cuda")
    vt = torch.zeros((H, 128, N), dtype=torch.bfloat16, device="cuda")
    out = torch.empty((N, H * 128), dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    p = lambda t: t.data_ptr()
    st = torch.cuda.current_stream().cuda_stream
    code = L.lib().rl_attention_ws(p(q), p(q), p(vt), H, N, N, N, None, p(out), H * 128, 0, 0, p(ws), need - 16, st)
    assert code == L.RL_ERR_WORKSPACE


def test_after_qkv_post(dev):
    """The QKV post pass's native outputs feed attention directly (Q with the score scale folded into wq)."""
    M, H = 256, 2
    rng = np.random.default_rng(3)
    C = F.bf16_round(rng.standard_normal((M, 3 * H * 128)).astype(np.float32))
    ang = rng.uniform(-np.pi, np.pi, (M, 64))
    cs, sn = F.bf16_round(np.cos(ang).astype(np.float32)), F.bf16_round(np.sin(ang).astype(np.float32))
    wq = F.bf16_round(((1 + 0.1 * rng.standard_normal(128)) * QK.C_LOG2).astype(np.float32))
    wk = F.bf16_round((1 + 0.1 * rng.standard_normal(128)).astype(np.float32))
    _, _, q, k, vt = ops.qkv_post(tt(C), tt(cs), tt(sn), tt(wq), tt(wk), H, tiles=False, native=True)
    o = ops.attention(q, k, vt).float().cpu().numpy().reshape(M, H, 128).transpose(1, 0, 2)
    ref = A.attention_ref(q.float().cpu().numpy(), k.float().cpu().numpy(),
                          vt.float().cpu().numpy().transpose(0, 2, 1))
    check(o, ref)
