"""Weight-file tooling on the GPU: the packers of redline/pack_weights.py (DiT blocks, bNN_*.bin) and
redline/vlm_pack.py (text-encoder layers, vlm/LNN_*.bin), and a manifest-verified loader for the text encoder's files
(the DiT's is forward.Weights).

The files are byte-identical to the reference packers': every matrix is B = W.T (K x N) packed as
to_bfp16(b_layout(B, 64, 128)), written by ops.pack_weight from the Linear weight W, with the same per-file manifest
fields (file, K, N, bytes, sha256). Text-encoder layers carry two channel permutations (redline/vlm_pack.py:1-13):
  * PERM per head of 128 dims, i -> 2i and i + 64 -> 2i + 1, so the model's rotate-half RoPE becomes the adjacent-pair
    RoPE the QKV post pass applies (q.k is unchanged because q and k are permuted alike);
  * hidden_perm (new channel n = old channel hp[n]): hidden channels sorted by peak |x|, so the few massive channels
    share bfp16 blocks instead of each crushing 7 ordinary channels. RMSNorm and every matmul are permutation
    invariant.
The GEMMs read the packed bytes as they are, so no other repack exists or is cached.
"""

import hashlib
import json
from pathlib import Path

import numpy as np
import torch

from . import ops

HEAD_DIM = 128
PERM = np.stack([np.arange(64), np.arange(64) + 64], 1).ravel()  # new dim 2i <- i, 2i+1 <- i+64 (vlm_pack.py:34)


def permute_heads(w, heads):
    """(heads*128, K) projection weight -> rows permuted per head by PERM (redline/vlm_pack.py:37-39)."""
    idx = torch.as_tensor(PERM, device=w.device)
    return w.reshape(heads, HEAD_DIM, -1)[:, idx, :].reshape(heads * HEAD_DIM, -1)


def hidden_perm(wdir, hidden=4096):
    """The packed weights' hidden-channel order: hidden_perm.npy in the weight directory, identity if absent
    (redline/vlm_pack.py:42-47)."""
    f = Path(wdir) / "hidden_perm.npy"
    return np.load(f, allow_pickle=False) if f.exists() else np.arange(hidden)


def balance_qk(wq, wk):
    """q_norm / k_norm weights (RoPE-permuted: pairs at 2j, 2j+1) -> (wq * alpha, wk / alpha), alpha =
    sqrt(|wk| / |wq|) per dim (magnitudes floored at 1e-2), as the geometric mean over each RoPE pair: q.k is unchanged
    and q, k get similar magnitudes per dim, so their 8-dim bfp16 blocks lose far less (redline/vlm_run.py:281-288)."""
    wq, wk = torch.as_tensor(wq, dtype=torch.float32), torch.as_tensor(wk, dtype=torch.float32)
    a = torch.sqrt(wk.abs().clamp_min(1e-2) / wq.abs().clamp_min(1e-2))
    a = torch.sqrt(a[0::2] * a[1::2]).repeat_interleave(2)
    return wq * a, wk / a


def _write(raw, path):
    host = raw.cpu().numpy()
    host.tofile(path)
    return int(host.size), hashlib.sha256(host.tobytes()).hexdigest()


def _pack_write(W, path):
    """Linear weight W (N, K) on the GPU -> the packed file of B = W.T; its manifest fields."""
    raw = ops.pack_weight(W.float().contiguous())
    nbytes, sha = _write(raw, path)
    return {"file": Path(path).name, "K": int(W.shape[1]), "N": int(W.shape[0]), "bytes": nbytes, "sha256": sha}


def pack_block(get, i, out_dir):
    """DiT block i -> b{i:02d}_{qkv,o,up,down}.bin and b{i:02d}_norm_{q,k}.npy in out_dir; returns the block's
    manifest entry (redline/pack_weights.py:92-119). get(name) returns a checkpoint tensor (any device, float)."""
    out, p = Path(out_dir), f"transformer_blocks.{i}."
    g = lambda n: torch.as_tensor(get(p + n)).to("cuda", torch.float32)
    mats = {
        "qkv": (lambda: torch.cat([g(f"attn.to_{x}.weight") for x in "qkv"], 0),
                [p + f"attn.to_{x}.weight" for x in "qkv"], "[Wq.T | Wk.T | Wv.T]"),
        "o": (lambda: g("attn.to_out.0.weight"), [p + "attn.to_out.0.weight"], "Wo.T"),
        "up": (lambda: ops.interleave_up(g("img_mlp.gate_layer.weight"), g("img_mlp.proj.weight")),
               [p + "img_mlp.gate_layer.weight", p + "img_mlp.proj.weight"],
               "[gate 64 | proj 64] per 128-col tile of [Wgate.T, Wproj.T]"),
        "down": (lambda: g("img_mlp.out.weight"), [p + "img_mlp.out.weight"], "Wdown.T"),
    }
    entry = {}
    for name, (build, src, how) in mats.items():
        entry[name] = _pack_write(build(), out / f"b{i:02d}_{name}.bin")
        entry[name].update({"source": src, "B": how})
    for name in ("norm_q", "norm_k"):
        path = out / f"b{i:02d}_{name}.npy"
        np.save(path, np.asarray(torch.as_tensor(get(p + f"attn.{name}.weight")).float().cpu().numpy()))
        entry[name] = {"file": path.name, "shape": [HEAD_DIM], "dtype": "float32", "source": [p + f"attn.{name}.weight"]}
    return entry


def pack_vlm_layer(get, i, out_dir, hp=None, hq=32, hkv=8):
    """Text-encoder layer i -> L{i:02d}_{qkv,o,up,down}.bin and L{i:02d}_norms.npz in out_dir; returns the layer's
    manifest entry (redline/vlm_pack.py:49-72). hp: hidden_perm (None = identity). B = W.T: hidden-in rows (qkv, up)
    or hidden-out columns (o, down) are permuted, i.e. the columns or the rows of W."""
    out, p = Path(out_dir), f"model.language_model.layers.{i}."
    g = lambda n: torch.as_tensor(get(p + n)).to("cuda", torch.float32)
    hidden = g("input_layernorm.weight").numel()
    h = torch.as_tensor(np.arange(hidden) if hp is None else np.asarray(hp), device="cuda", dtype=torch.int64)
    mats = {
        "qkv": lambda: torch.cat([permute_heads(g("self_attn.q_proj.weight"), hq),
                                  permute_heads(g("self_attn.k_proj.weight"), hkv),
                                  g("self_attn.v_proj.weight")], 0)[:, h],
        "o": lambda: g("self_attn.o_proj.weight")[h, :],
        "up": lambda: ops.interleave_up(g("mlp.gate_proj.weight"), g("mlp.up_proj.weight"))[:, h],
        "down": lambda: g("mlp.down_proj.weight")[h, :],
    }
    entry = {name: _pack_write(build(), out / f"L{i:02d}_{name}.bin") for name, build in mats.items()}
    perm = torch.as_tensor(PERM, device="cuda")
    norms = {"w_in": g("input_layernorm.weight")[h], "w_post": g("post_attention_layernorm.weight")[h],
             "q_norm": g("self_attn.q_norm.weight")[perm], "k_norm": g("self_attn.k_norm.weight")[perm]}
    np.savez(out / f"L{i:02d}_norms.npz", **{k: v.cpu().numpy() for k, v in norms.items()})
    entry["norms"] = {"file": f"L{i:02d}_norms.npz"}
    return entry


def write_manifest(out_dir, key, entries, **fields):
    """manifest.json with the per-block (key "blocks", 2-digit ids) or per-layer (key "layers") entries merged into
    an existing manifest, plus top-level fields (redline/pack_weights.py:140-181, redline/vlm_pack.py:83-97)."""
    path = Path(out_dir) / "manifest.json"
    man = json.loads(path.read_text()) if path.exists() else {}
    man.update(fields)
    man.setdefault(key, {}).update({(f"{i:02d}" if key == "blocks" else str(i)): e for i, e in entries.items()})
    path.write_text(json.dumps(man, indent=1))
    return man


def _verify(raw, entry, name):
    if entry is None:
        raise ValueError(f"{name}: not in manifest.json")
    if int(entry["bytes"]) != raw.size:
        raise ValueError(f"{name}: {raw.size} bytes, manifest says {entry['bytes']}")
    if hashlib.sha256(raw.tobytes()).hexdigest() != entry["sha256"]:
        raise ValueError(f"{name}: sha256 mismatch")


class VlmWeights:
    """The text encoder's packed layers resident on the GPU, as LM.__init__ loads them (redline/vlm_run.py:303-318):
    per layer the qkv / o / up / down streams (uint8 tensors), the balanced q/k norm weights (``qk[i]``), and the two
    RMSNorm parameter buffers (``p_in[i]``, ``p_post[i]``: rms_params of the permuted norm weights, bf16 (2, 2D), for
    rl_ln_modulate with RL_NORM_RMS). ``hp`` is the hidden-channel order. With ``verify=True`` every file's size and
    sha256 are checked against manifest.json; a mismatch raises ValueError."""

    MATS = ("qkv", "o", "up", "down")

    def __init__(self, wdir, layers, verify=False, device="cuda"):
        wdir = Path(wdir)
        self.manifest = json.loads((wdir / "manifest.json").read_text()) if (wdir / "manifest.json").exists() else {}
        self.w, self.qk, self.p_in, self.p_post, self.norms = {}, {}, {}, {}, {}
        self.layers = list(layers)
        hidden = None
        for i in self.layers:
            entry = self.manifest.get("layers", {}).get(str(i), {})
            for m in self.MATS:
                raw = np.fromfile(wdir / f"L{i:02d}_{m}.bin", np.uint8)
                if verify:
                    _verify(raw, entry.get(m), f"L{i:02d}_{m}.bin")
                self.w[i, m] = torch.from_numpy(raw).to(device)
            with np.load(wdir / f"L{i:02d}_norms.npz", allow_pickle=False) as nz:
                self.norms[i] = {k: nz[k] for k in nz.files}
            n = self.norms[i]
            hidden = len(n["w_in"])
            self.qk[i] = tuple(t.to(device) for t in balance_qk(n["q_norm"], n["k_norm"]))
            self.p_in[i] = rms_params(n["w_in"], device=device)
            self.p_post[i] = rms_params(n["w_post"], device=device)
        self.hp = hidden_perm(wdir, hidden or 4096)

    def unperm(self, x):
        """A (rows, hidden) tensor in the packed channel order -> the model's order (x_model[:, hp[n]] = x[:, n])."""
        out = torch.empty_like(x)
        out[:, torch.as_tensor(self.hp, device=x.device)] = x
        return out


def rms_params(w, g=1.0, device="cuda"):
    """RMSNorm parameter buffer for rl_ln_modulate: both rows [g | w], bf16 (2, 2D) (redline/vlm_run.py:62-65)."""
    w = torch.as_tensor(np.asarray(w, np.float32))
    row = torch.cat([torch.full_like(w, g), w])
    return torch.stack([row, row]).to(device=device, dtype=torch.bfloat16)
