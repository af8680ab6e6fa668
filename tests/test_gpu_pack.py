"""The GPU weight packers write the reference packers' files byte for byte (oracle/pack.py, which follows
redline/pack_weights.py and redline/vlm_pack.py), and the manifest-verified loaders read them back."""

import json

import numpy as np
import pytest
import torch

from oracle import bfp16 as F
from oracle import pack as P
from rlbfp import forward
from rlbfp import pack as RP

pytestmark = pytest.mark.gpu


def dit_checkpoint(rng, hidden=256, ff=512):
    p = "transformer_blocks.0."
    w = lambda n, k: (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    ck = {p + f"attn.to_{x}.weight": w(hidden, hidden) for x in "qkv"}
    ck.update({p + "attn.to_out.0.weight": w(hidden, hidden), p + "img_mlp.gate_layer.weight": w(ff, hidden),
               p + "img_mlp.proj.weight": w(ff, hidden), p + "img_mlp.out.weight": w(hidden, ff),
               p + "attn.norm_q.weight": rng.standard_normal(128).astype(np.float32),
               p + "attn.norm_k.weight": rng.standard_normal(128).astype(np.float32)})
    return ck


def vlm_checkpoint(rng, i, hidden=256, hq=2, hkv=1, ff=512):
    p = f"model.language_model.layers.{i}."
    w = lambda n, k: (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    return {p + "self_attn.q_proj.weight": w(hq * 128, hidden), p + "self_attn.k_proj.weight": w(hkv * 128, hidden),
            p + "self_attn.v_proj.weight": w(hkv * 128, hidden), p + "self_attn.o_proj.weight": w(hidden, hq * 128),
            p + "mlp.gate_proj.weight": w(ff, hidden), p + "mlp.up_proj.weight": w(ff, hidden),
            p + "mlp.down_proj.weight": w(hidden, ff),
            p + "input_layernorm.weight": (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32),
            p + "post_attention_layernorm.weight": (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32),
            p + "self_attn.q_norm.weight": rng.uniform(0.5, 4, 128).astype(np.float32),
            p + "self_attn.k_norm.weight": rng.uniform(0.5, 35, 128).astype(np.float32)}


def test_dit_block_files(dev, tmp_path):
    ck = dit_checkpoint(np.random.default_rng(0))
    entry = RP.pack_block(ck.get, 0, tmp_path)
    RP.write_manifest(tmp_path, "blocks", {0: entry}, model="synthetic")
    for name, B in P.block_mats(ck.get, 0).items():
        raw = np.fromfile(tmp_path / f"b00_{name}.bin", np.uint8)
        np.testing.assert_array_equal(raw, F.pack_b(B), err_msg=name)
        assert (entry[name]["K"], entry[name]["N"]) == B.shape
    w = forward.Weights(tmp_path, blocks=[0], verify=True)
    assert np.array_equal(w.b[0, "up"].cpu().numpy(), np.fromfile(tmp_path / "b00_up.bin", np.uint8))
    np.testing.assert_array_equal(w.b[0, "norm_q"], ck["transformer_blocks.0.attn.norm_q.weight"])
    # a changed byte is caught by the sha256 check
    raw = np.fromfile(tmp_path / "b00_o.bin", np.uint8)
    raw[100] ^= 1
    raw.tofile(tmp_path / "b00_o.bin")
    with pytest.raises(ValueError, match="sha256"):
        forward.Weights(tmp_path, blocks=[0], verify=True)


def test_vlm_layer_files(dev, tmp_path):
    rng = np.random.default_rng(1)
    hidden, hq, hkv = 256, 2, 1
    hp = rng.permutation(hidden)
    np.save(tmp_path / "hidden_perm.npy", hp)
    ck = {}
    for i in (0, 1):
        ck.update(vlm_checkpoint(rng, i, hidden, hq, hkv))
    entries = {i: RP.pack_vlm_layer(ck.get, i, tmp_path, hp=hp, hq=hq, hkv=hkv) for i in (0, 1)}
    RP.write_manifest(tmp_path, "layers", entries, rope_perm="head dim i -> 2i, i+64 -> 2i+1")
    man = json.loads((tmp_path / "manifest.json").read_text())
    assert set(man["layers"]) == {"0", "1"}
    for i in (0, 1):
        for name, B in P.layer_mats(ck.get, i, hp, hq, hkv).items():
            np.testing.assert_array_equal(np.fromfile(tmp_path / f"L{i:02d}_{name}.bin", np.uint8), F.pack_b(B),
                                          err_msg=f"layer {i} {name}")
        with np.load(tmp_path / f"L{i:02d}_norms.npz") as nz:
            for k, v in P.layer_norms(ck.get, i, hp).items():
                np.testing.assert_array_equal(nz[k], v)
    w = RP.VlmWeights(tmp_path, layers=[0, 1], verify=True)
    np.testing.assert_array_equal(w.hp, hp)
    bq, bk = P.balance_qk(*(P.layer_norms(ck.get, 1, hp)[k] for k in ("q_norm", "k_norm")))
    np.testing.assert_allclose(w.qk[1][0].cpu().numpy(), bq, rtol=1e-6)
    np.testing.assert_allclose(w.qk[1][1].cpu().numpy(), bk, rtol=1e-6)
    assert w.p_in[0].shape == (2, 2 * hidden)
    x = torch.arange(2 * hidden, dtype=torch.float32, device="cuda").reshape(2, hidden)
    xm = w.unperm(x)
    assert torch.equal(xm[:, torch.as_tensor(hp, device="cuda")], x)
    raw = np.fromfile(tmp_path / "L01_down.bin", np.uint8)
    raw[7] ^= 4
    raw.tofile(tmp_path / "L01_down.bin")
    with pytest.raises(ValueError, match="sha256"):
        RP.VlmWeights(tmp_path, layers=[1], verify=True)
