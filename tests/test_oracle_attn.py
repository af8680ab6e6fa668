"""The oracle's attention (oracle/attn.py), pinned against torch's float64 scaled_dot_product_attention (a library
routine), the reference's own check formula (redline/run_attn.py:147-150, natural-log softmax of unscaled scores),
and closed forms: equal keys average V, a single visible key returns its V row."""

import numpy as np
import torch

from oracle import attn as A


def rand(rng, H, NQ, NK):
    q = rng.standard_normal((H, NQ, 128))
    k = rng.standard_normal((H, NK, 128))
    v = rng.standard_normal((H, NK, 128))
    return q, k, v


def test_matches_torch_sdpa():
    rng = np.random.default_rng(0)
    q, k, v = rand(rng, 2, 40, 70)
    o = A.attention_ref(q * A.C_LOG2, k, v)
    ref = torch.nn.functional.scaled_dot_product_attention(*(torch.from_numpy(x) for x in (q, k, v))).numpy()
    np.testing.assert_allclose(o, ref, rtol=1e-10, atol=1e-12)


def test_matches_reference_check_with_padding_and_limits():
    rng = np.random.default_rng(1)
    H, NQ, NK, NKV = 1, 24, 50, 41
    q, k, v = rand(rng, H, NQ, NK)
    lim = rng.integers(0, NKV, NQ)
    lim[:3] = [0, 1, 2]
    o = A.attention_ref(q * A.C_LOG2, k, v, nkv=NKV, lim=lim)
    s = q[0] @ k[0, :NKV].T / np.sqrt(128)
    s = np.where(np.arange(NKV)[None, :] <= lim[:, None], s, -np.inf)
    w = np.exp(s - s.max(1, keepdims=True))
    ref = (w / w.sum(1, keepdims=True)) @ v[0, :NKV]
    np.testing.assert_allclose(o[0], ref, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(o[0, 0], v[0, 0], rtol=1e-12)  # only key 0 visible


def test_equal_keys_average_values():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((1, 5, 128))
    k = np.repeat(rng.standard_normal((1, 1, 128)), 9, 1)
    v = rng.standard_normal((1, 9, 128))
    np.testing.assert_allclose(A.attention_ref(q, k, v)[0], np.repeat(v[0].mean(0, keepdims=True), 5, 0), rtol=1e-12)
