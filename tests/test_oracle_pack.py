"""The weight-file tooling's host-side pieces (oracle/pack.py and rlbfp/pack.py without a GPU): the RoPE head
permutation against the closed form it exists for, the q/k balancing invariants, and the product's torch versions
against the oracle."""

import numpy as np
import torch

from oracle import pack as P
from oracle import qkv as QK
from rlbfp import pack as RP


def test_perm_turns_rotate_half_into_adjacent_pairs():
    """The model rotates dims (i, i + 64); after PERM (i -> 2i, i + 64 -> 2i + 1) the same rotation is the adjacent-
    pair RoPE of the QKV post pass (redline/vlm_pack.py:11-12)."""
    rng = np.random.default_rng(0)
    y = rng.standard_normal((6, 128))
    ang = rng.uniform(-np.pi, np.pi, (6, 64))
    c, s = np.cos(ang), np.sin(ang)
    np.testing.assert_allclose(P.rope_rotate_half(y, c, s)[:, P.PERM], QK.rope(y[:, P.PERM], c, s), atol=1e-12)
    assert sorted(P.PERM) == list(range(128))


def test_permute_heads_keeps_q_dot_k():
    rng = np.random.default_rng(1)
    K, heads = 64, 2
    wq, wk = rng.standard_normal((heads * 128, K)), rng.standard_normal((heads * 128, K))
    x = rng.standard_normal((5, K))
    q, k = x @ wq.T, x @ wk.T
    qp, kp = x @ P.permute_heads(wq, heads).T, x @ P.permute_heads(wk, heads).T
    for h in range(heads):
        sl = slice(h * 128, (h + 1) * 128)
        np.testing.assert_allclose(qp[:, sl] @ kp[:, sl].T, q[:, sl] @ k[:, sl].T, rtol=1e-12)
    np.testing.assert_array_equal(RP.permute_heads(torch.from_numpy(wq), heads).numpy(), P.permute_heads(wq, heads))


def test_balance_qk_invariants():
    rng = np.random.default_rng(2)
    wq = rng.uniform(0.5, 4, 128) * rng.choice([-1, 1], 128)
    wk = rng.uniform(0.5, 35, 128) * rng.choice([-1, 1], 128)
    bq, bk = P.balance_qk(wq, wk)
    np.testing.assert_allclose(bq * bk, wq * wk, rtol=1e-12)              # q.k unchanged, dim by dim
    a = bq / wq
    np.testing.assert_allclose(a[0::2], a[1::2], rtol=1e-12)              # one factor per RoPE pair
    np.testing.assert_allclose(np.abs(bq[0::2] * bq[1::2]), np.abs(bk[0::2] * bk[1::2]), rtol=1e-9)  # balanced pairs
    same = np.abs(wq)
    np.testing.assert_allclose(P.balance_qk(same, -same)[0], same, rtol=1e-12)  # |wq| = |wk| -> unchanged
    tq, tk = RP.balance_qk(wq, wk)
    np.testing.assert_allclose(tq.numpy(), bq, rtol=1e-6)
    np.testing.assert_allclose(tk.numpy(), bk, rtol=1e-6)


def test_rms_params_and_identity_perm(tmp_path):
    w = np.linspace(0.5, 1.5, 64).astype(np.float32)
    p = RP.rms_params(w, device="cpu")
    assert p.shape == (2, 128) and p.dtype == torch.bfloat16
    assert (p[:, :64] == 1).all()
    np.testing.assert_array_equal(p[0, 64:].float().numpy(), torch.from_numpy(w).to(torch.bfloat16).float().numpy())
    np.testing.assert_array_equal(RP.hidden_perm(tmp_path, 16), np.arange(16))
    np.save(tmp_path / "hidden_perm.npy", np.arange(16)[::-1].copy())
    np.testing.assert_array_equal(RP.hidden_perm(tmp_path, 16), np.arange(16)[::-1])
