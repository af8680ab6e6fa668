"""CPU restatement of the weight-file tooling: the DiT block packer, the text encoder's layer packer with its channel
permutations, and the q/k norm balancing (oracle; test infrastructure only).

Follows:
  pack_block     redline/pack_weights.py:92-119   B = [Wq.T | Wk.T | Wv.T], Wo.T, interleave_up(gate, proj), Wdown.T
  PERM           redline/vlm_pack.py:34           head dim i -> 2i, i + 64 -> 2i + 1 (rotate-half RoPE -> adjacent pairs)
  permute_heads  redline/vlm_pack.py:37-39
  pack_layer     redline/vlm_pack.py:49-72        B rows (hidden in) or columns (hidden out) permuted by hidden_perm
  balance_qk     redline/vlm_run.py:281-288       wq * alpha, wk / alpha, alpha = sqrt(|wk| / |wq|) (floored at 1e-2),
                                                  geometric mean over each RoPE pair
"""

import numpy as np

from . import bfp16 as F

HEAD_DIM = 128
PERM = np.stack([np.arange(64), np.arange(64) + 64], 1).ravel()  # new dim 2i <- i, 2i+1 <- i+64


def permute_heads(w, heads):
    """(heads*128, K) projection weight -> rows permuted per head by PERM."""
    return np.asarray(w).reshape(heads, HEAD_DIM, -1)[:, PERM, :].reshape(heads * HEAD_DIM, -1)


def block_mats(get, i):
    """The four B matrices (K x N) of DiT block i, as pack_weights.pack_block builds them."""
    p = f"transformer_blocks.{i}."
    return {
        "qkv": np.concatenate([get(p + f"attn.to_{x}.weight").T for x in "qkv"], 1),
        "o": get(p + "attn.to_out.0.weight").T,
        "up": F.interleave_up(get(p + "img_mlp.gate_layer.weight"), get(p + "img_mlp.proj.weight")),
        "down": get(p + "img_mlp.out.weight").T,
    }


def layer_mats(get, i, hp, hq, hkv):
    """The four B matrices of text-encoder layer i, as vlm_pack.pack_layer builds them (hp: new channel n = old
    channel hp[n])."""
    p = f"model.language_model.layers.{i}."
    g = lambda n: get(p + n)
    return {
        "qkv": np.concatenate([permute_heads(g("self_attn.q_proj.weight"), hq).T,
                               permute_heads(g("self_attn.k_proj.weight"), hkv).T,
                               g("self_attn.v_proj.weight").T], 1)[hp],
        "o": g("self_attn.o_proj.weight").T[:, hp],
        "up": F.interleave_up(g("mlp.gate_proj.weight"), g("mlp.up_proj.weight"))[hp],
        "down": g("mlp.down_proj.weight").T[:, hp],
    }


def layer_norms(get, i, hp):
    p = f"model.language_model.layers.{i}."
    g = lambda n: get(p + n)
    return {"w_in": g("input_layernorm.weight")[hp], "w_post": g("post_attention_layernorm.weight")[hp],
            "q_norm": g("self_attn.q_norm.weight")[PERM], "k_norm": g("self_attn.k_norm.weight")[PERM]}


def balance_qk(wq, wk):
    """q_norm / k_norm weights (RoPE-permuted: pairs at 2j, 2j+1) -> (wq * alpha, wk / alpha)."""
    a = np.sqrt(np.maximum(np.abs(wk), 1e-2) / np.maximum(np.abs(wq), 1e-2))
    a = np.repeat(np.sqrt(a[0::2] * a[1::2]), 2)
    return wq * a, wk / a


def rope_rotate_half(y, cos, sin):
    """The model's RoPE: dims (i, i + 64) rotate together (rotate-half convention), cos/sin (n, 64)."""
    a, b = y[:, :64], y[:, 64:]
    return np.concatenate([a * cos - b * sin, a * sin + b * cos], 1)
