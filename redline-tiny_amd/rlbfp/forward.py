"""The DiT call surface of redline/forward.py, on the HIP path.

Names, arguments and meaning follow the reference: ``GEMMS`` (artifact name per (op, M)), ``GEMM_KN``, ``LN_ART``,
``QKV_ART``, ``v9``, ``NPU.run(op, art, args)`` / ``NPU.sync()`` / ``NPU.report()`` / ``NPU.set_nv()``, ``Weights``
(the packed ``bNN_*.bin`` files plus ``manifest.json`` that redline/pack_weights.py writes) and
``gemm(npu, w, op, M, a, c, block=None)`` (redline/forward.py:33-44, :82-84, :87-172, :175-197, :205-206).

``NPU.run`` takes every op of CachedStep.blocks / ExtractStep.blocks / step1_embed (:240-254, :362-388, :399-413) and
of the text encoder's LM._layer (redline/vlm_run.py:427-449):
  * GEMMs [A, B, C] ("qkv", "o", "down", "img_in", "proj_out", "up"; "up_swiglu" / "up+swiglu" with the SwiGLU
    epilogue);
  * "ln_mod" / "rms" [X, BR, P, XO, AO] (run_ln.ln_fused);
  * "qkv_post" [C, TABS, Q, KV] (run_qkv.qkv_post_run);
  * "attn", "attn_ref", "attn_small" [Q, KV(, KV prefix), O] / [Q, LIM, KV, O] (run_attn.run_artifact, the artifact's
    parameters from its name, or from ``NPU.meta[art]`` for artifacts built for other shapes);
  * "swiglu" [C_up, H] (the unfused SwiGLU glue).

Differences, all deliberate:
  * buffers are torch tensors on the GPU, and work is enqueued on torch's current HIP stream (``run`` never blocks;
    ``sync`` synchronises the stream);
  * A may be a bf16 (M, K) activation tensor (the build's native operand, already bfp16 values or quantized while it
    is loaded, see ``NPU.a_fmt``) or a V9 uint8 tensor in the reference's A layout (a_layout(., 128, 64)), which is
    decoded to bf16 in a workspace (one HBM-bound pass) before the fast bf16 kernel runs;
  * C may be a bf16 (M, N) tensor (the build's native output: fp32 accumulation, one bf16 rounding), a flat bf16
    tensor, which receives the C16 artifacts' element order c_layout_atb(., 128, 128) (kernels/vlm/mm_bfp_c16.cc:1-2),
    or a V9 uint8 tensor, which receives the reference's own stream order: the ATB C order for plain GEMMs and the
    down-GEMM A layout (a_layout(., 128, 64)) for the SwiGLU GEMM.
"""

import hashlib
import json
import re
import time
from collections import defaultdict
from pathlib import Path

import numpy as np
import torch

from . import layouts, ops, run_attn, run_ln, run_qkv

N_BLOCKS, HID, FF = 32, 4096, 12288
M_S1 = 8704

# artifact names per (op, M) as in redline/forward.py:33-42; here they select the epilogue of the HIP GEMM
LN_ART = {4096: "glue-ln-m4096-s0", M_S1: "glue-ln-m8704-s33"}  # redline/forward.py:205
QKV_ART = {4096: "glue-qkv32-m4096", M_S1: "glue-qkv32-m8704"}  # redline/forward.py:206
GEMMS = {
    ("qkv", 4096): "atb3d2-qkv", ("qkv", M_S1): "atb3d2-s1qkv",
    ("o", 4096): "atb3d2-4096", ("o", M_S1): "atb3d2-s1o",
    ("down", 4096): "atb3d2-down", ("down", M_S1): "atb3d2-s1down",
    ("up_swiglu", 4096): "atb3sw2-m4096", ("up_swiglu", M_S1): "atb3sw2-m8704",
    ("img_in", 4096): "q-atb3k-imgin", ("img_in", M_S1): "q-atb3k-s1imgin",
    ("proj_out", 4096): "q-atb3k-projout",
}
GEMM_KN = {"qkv": (HID, 3 * HID), "o": (HID, HID), "up": (HID, 2 * FF), "down": (FF, HID), "img_in": (64, HID),
           "proj_out": (HID, 1024)}


SWIGLU_OPS = ("up_swiglu", "up+swiglu")


def artifact_kind(art):
    """'swiglu' for the SwiGLU-flush GEMMs (atb3sw*, vlm-upsw*), else 'gemm'."""
    art = str(art)
    return "swiglu" if art.startswith("atb3sw") or "upsw" in art else "gemm"


def gemm_k(a, b, c, swiglu):
    """K of a GEMM from its three buffers' value counts (A: M K, B: K N, C: M N, or M N / 2 after SwiGLU)."""
    vals = lambda t: t.numel() // 9 * 8 if t.dtype == torch.uint8 else t.numel()
    ab, cc = vals(a) * vals(b), vals(c) * (2 if swiglu else 1)
    K = int(round((ab / cc) ** 0.5)) if cc else 0
    if K <= 0 or K * K * cc != ab:
        raise ValueError("A, B and C sizes do not describe one GEMM")
    return K


def v9(nvals, device="cuda"):
    """A device buffer holding nvals bfp16 values (nvals / 8 blocks of 9 bytes), zeroed (redline/forward.py:82-84)."""
    return torch.zeros(nvals // 8 * 9, dtype=torch.uint8, device=device)


def bf16_tensor(a, device="cuda"):
    """float array (numpy or torch) -> flat bf16 device tensor (redline/forward.py:200-202)."""
    t = a.float() if torch.is_tensor(a) else torch.as_tensor(np.asarray(a, np.float32))
    return t.to(device=device, dtype=torch.bfloat16).reshape(-1)


class NPU:
    """Kernel runner with per-op timing (device time from HIP events, wall time of the enqueue), like
    redline/forward.py:87-172. ``kn`` maps op -> (K, N) for A operands that do not carry K (packed A)."""

    def __init__(self, kn=None, a_fmt="bf16"):
        self.kn = dict(GEMM_KN if kn is None else kn)
        self.a_fmt = a_fmt
        self.t_npu, self.t_wall, self.calls = defaultdict(float), defaultdict(float), defaultdict(int)
        self.pending = []  # (op, start event, end event, args kept alive until sync)
        self.nv = {}       # runtime valid-key counts of NVRT attention artifacts, {marker id: keys in the last tile}
        self.meta = {}     # attention artifact name -> parameters, for artifacts built for other shapes

    def set_nv(self, nv):
        """Runtime valid-key counts {marker id: valid keys of the last tile} for the NVRT attention artifacts
        (redline/forward.py:97-108); later runs of those artifacts mask the keys past them."""
        self.nv = dict(nv)

    def sync(self):
        """Wait for every enqueued run and account its device time."""
        torch.cuda.current_stream().synchronize()
        for op, e0, e1, _args in self.pending:
            self.t_npu[op] += e0.elapsed_time(e1) / 1e3
        self.pending = []

    def run(self, op, art, args):
        """Enqueue one op of the reference's call sequences; see the module docstring for the ops and buffer forms."""
        t = time.perf_counter()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        self._dispatch(op, str(art), list(args))
        e1.record()
        self.pending.append((op, e0, e1, list(args)))
        self.t_wall[op] += time.perf_counter() - t
        self.calls[op] += 1

    def _dispatch(self, op, art, args):
        name = Path(art).name
        if op == "qkv_post" or name.startswith(("glue-qkv", "vlm-qkv")):
            run_qkv.qkv_post_run(art, *args)
        elif op.startswith("attn") or name.startswith(("attn", "vlm-attn")):
            meta = self.meta.get(art) or self.meta.get(name) or run_attn.attn_meta(art, self.nv)
            run_attn.run_artifact(meta, args)
        elif len(args) == 5:
            run_ln.ln_fused(art, *args)
        elif op == "swiglu" or name.startswith("vlm-swiglu"):
            swiglu_glue(art, *args)
        elif len(args) == 3:
            self._gemm(op, art, *args)
        else:
            raise ValueError(f"{op} / {art}: {len(args)} arguments match no artifact contract")

    def _gemm(self, op, art, a, b, c):
        swiglu = op in SWIGLU_OPS or artifact_kind(art) == "swiglu"
        base = "up" if swiglu else op
        if a.dtype == torch.bfloat16 and a.dim() == 2:
            M, K = a.shape
            fmt = self.a_fmt
        else:
            if a.dtype != torch.uint8:
                raise ValueError("A must be a 2-D bf16 tensor or a V9 (uint8) stream in the A layout")
            try:
                K = gemm_k(a, b, c, swiglu)
            except ValueError:
                K = self.kn[base][0]
            M = a.numel() // 9 * 8 // K
            fmt = "packed_a_layout"
        N = b.numel() // 9 * 8 // K
        act = "swiglu" if swiglu else None
        nout = N // 2 if act else N
        if c.dtype == torch.bfloat16 and c.dim() == 2:
            ops.gemm(a, b, N, K, M=M, a_fmt=fmt, act=act, out=c.view(M, nout))
            return
        if c.dtype == torch.bfloat16:
            # flat bf16 C: the C16 artifacts' element order (kernels/vlm/mm_bfp_c16.cc:1-2), written by the epilogue
            if act:
                raise ValueError("the SwiGLU GEMM writes H as a V9 stream or a 2-D bf16 tensor")
            ops.gemm(a, b, N, K, M=M, a_fmt=fmt, out=c, c_order="c_atb")
            return
        # V9 output: the reference's stream order (the ATB C stream, or H in the down GEMM's A layout), written as
        # bfp16 blocks by the GEMM's own epilogue (kernels/atb3/mm_bfp_mixed.cc:153-168, mm_bfp_swiglu.cc:73-86)
        ops.gemm(a, b, N, K, M=M, a_fmt=fmt, act=act, packed_out=c, packed_order="a_layout" if act else "c_atb")

    def report(self):
        tot_w, tot_n = sum(self.t_wall.values()), sum(self.t_npu.values())
        for op in sorted(self.t_wall, key=lambda o: -self.t_npu[o]):
            print(f"  {op:12s} {self.calls[op]:5d} calls  gpu {self.t_npu[op] * 1e3:9.3f} ms  "
                  f"wall {self.t_wall[op] * 1e3:9.3f} ms")
        print(f"  {'total':12s} {sum(self.calls.values()):5d} calls  gpu {tot_n * 1e3:9.3f} ms  "
              f"wall {tot_w * 1e3:9.3f} ms")


class Weights:
    """Packed weights resident on the GPU: per block the qkv / o / up / down B streams (uint8 tensors) and norm_q /
    norm_k, read from a pack_weights.py output directory (redline/forward.py:175-191).

    With ``verify=True`` every file's byte count and sha256 are checked against manifest.json
    (redline/pack_weights.py:111-112); a mismatch raises ValueError."""

    MATS = ("qkv", "o", "up", "down")

    def __init__(self, wdir=None, blocks=range(N_BLOCKS), verify=False, device="cuda"):
        self.b, self.host, self.manifest = {}, {}, {}
        if wdir is None:
            return
        wdir = Path(wdir)
        self.manifest = json.loads((wdir / "manifest.json").read_text())
        t = time.perf_counter()
        for i in blocks:
            entry = self.manifest.get("blocks", {}).get(f"{i:02d}", {})
            for m in self.MATS:
                raw = np.fromfile(wdir / f"b{i:02d}_{m}.bin", np.uint8)
                if verify:
                    self._verify(raw, entry.get(m), f"b{i:02d}_{m}.bin")
                self.b[i, m] = torch.from_numpy(raw).to(device)
            for m in ("norm_q", "norm_k"):
                p = wdir / f"b{i:02d}_{m}.npy"
                if p.exists():
                    self.b[i, m] = np.load(p, allow_pickle=False)
        for m in ("img_in", "proj_out"):
            p = wdir / f"{m}.bin"
            if p.exists():
                raw = np.fromfile(p, np.uint8)
                if verify:
                    self._verify(raw, self.manifest.get(m), p.name)
                self.b[m] = torch.from_numpy(raw).to(device)
        hd = wdir / "host"
        if hd.is_dir():
            self.host = {p.stem: np.load(p, allow_pickle=False) for p in hd.glob("*.npy")}
        print(f"weights: {len(list(blocks))} blocks resident in {time.perf_counter() - t:.1f} s")

    @staticmethod
    def _verify(raw, entry, name):
        if entry is None:
            raise ValueError(f"{name}: not in manifest.json")
        if int(entry["bytes"]) != raw.size:
            raise ValueError(f"{name}: {raw.size} bytes, manifest says {entry['bytes']}")
        if hashlib.sha256(raw.tobytes()).hexdigest() != entry["sha256"]:
            raise ValueError(f"{name}: sha256 mismatch")

    @classmethod
    def from_tensors(cls, mats):
        """Resident weights from already-packed device tensors: {(block, op) or op: uint8 tensor}."""
        w = cls()
        w.b.update(mats)
        return w


def gemm(npu, w, op, M, a, c, block=None):
    """C = A @ W for op at M rows (redline/forward.py:194-197)."""
    b = w.b[block, op] if block is not None else w.b[op]
    npu.run(op, GEMMS.get((op, M), op), [a, b, c])


def swiglu_glue(art, c_up, h):
    """The unfused SwiGLU glue (kernels/glue/swiglu_bfp.cc, run as "vlm-swiglu-m{M}" by redline/vlm_run.py:444-446):
    C_up, the up GEMM's output (V9 in the C-stream order c_layout_atb(., 128, 128), [gate 64 | proj 64] per 128
    columns) -> H = silu(gate) * proj as the down GEMM's A (V9, a_layout(., 128, 64)). M comes from the artifact
    name; silu(gate) * proj is evaluated in fp32 on the decoded bfp16 values and rounded to bf16 before the encode."""
    m = re.search(r"-m(\d+)", Path(art).name)
    if not m:
        raise ValueError(f"{art}: the SwiGLU glue needs its row count in the artifact name (-m<M>)")
    M = int(m.group(1))
    n2 = c_up.numel() // 9 * 8
    if n2 % (2 * M) or h.numel() // 9 * 8 * 2 != n2:
        raise ValueError("C_up must hold M x 2F values and H M x F")
    F = n2 // (2 * M)
    v = ops.dequantize(c_up.reshape(-1), M, 2 * F, order="c_atb").reshape(M, F // 64, 2, 64)
    g, p = v[:, :, 0], v[:, :, 1]
    y = (g / (1.0 + torch.exp(-g)) * p).reshape(M, F).to(torch.bfloat16)
    h.reshape(-1).copy_(ops.quantize(y, order="a_layout")[0])


class CachedStep:
    """Device buffers + call sequence for a cached step (redline/forward.py:209-269), M target rows (4096 in the
    reference). The attention call is pluggable: attn(npu, q, kv_target, kv_prefix, o) (O in the out-proj A layout).
    Hidden and FFN widths come from the weights; every buffer is a V9 (uint8) stream or flat bf16, as the reference's.
    """

    def __init__(self, w, cos, sin, attn, M=4096, n_blocks=N_BLOCKS, device="cuda"):
        self.M, self.w, self.attn, self.n_blocks = M, w, attn, n_blocks
        blocks = sorted({k[0] for k in w.b if isinstance(k, tuple)})
        b0 = blocks[0]
        hid = int(round((w.b[b0, "o"].numel() // 9 * 8) ** 0.5))
        ff = w.b[b0, "down"].numel() // 9 * 8 // hid
        self.hid, self.ff, self.heads = hid, ff, hid // 128
        T = M // 64
        z = lambda n: torch.zeros(n, dtype=torch.bfloat16, device=device)
        self.x = [z(M * hid), z(M * hid)]
        self.zero_x = z(M * hid)
        self.zero_br, self.a, self.o, self.c = (v9(M * hid, device) for _ in range(4))
        self.c_qkv, self.h = v9(M * 3 * hid, device), v9(M * ff, device)
        self.c_in, self.c_out = v9(M * hid, device), v9(M * 1024, device)
        self.q, self.kv = v9(self.heads * T * 64 * 128, device), v9(self.heads * T * 2 * 64 * 128, device)
        c = float(np.log2(np.e) / np.sqrt(128))
        cos, sin = torch.as_tensor(cos).to(device), torch.as_tensor(sin).to(device)
        wq = lambda i: torch.as_tensor(np.asarray(w.b[i, "norm_q"], np.float32) * np.float32(c)).to(device)
        self.tabs = {i: run_qkv.qkv_tables(cos, sin, wq(i), torch.as_tensor(np.asarray(w.b[i, "norm_k"])).to(device))
                     .reshape(-1) for i in blocks}

    def set_t(self, mod, out_scale):
        """Per-step parameters from the shared modulation (2, 4 hidden) and the norm_out scale (2, hidden)
        (redline/forward.py:231-238)."""
        hid = self.hid
        mod = torch.as_tensor(mod).float().cuda()
        out_scale = torch.as_tensor(out_scale).float().cuda()
        s1, g1, s2, g2 = (mod[:, i * hid:(i + 1) * hid] for i in range(4))
        lp = lambda g, sc: run_ln.ln_params(g, sc)
        self.p_first = lp(torch.ones_like(s1), 1 + s1)
        self.p_mlp = lp(torch.tanh(g1), 1 + s2)
        self.p_attn = lp(torch.tanh(g2), 1 + s1)
        self.p_out = lp(torch.tanh(g2), 1 + out_scale)

    def blocks(self, npu, kv_prefix, first, last):
        """Run blocks first..last (redline/forward.py:240-254); x[0] / a hold block `first`'s x and LN1 output on
        entry. Returns the index of the x buffer holding the result."""
        M, w = self.M, self.w
        ln_art = LN_ART.get(M, f"glue-ln-m{M}-s0")
        for i in range(first, last + 1):
            gemm(npu, w, "qkv", M, self.a, self.c_qkv, block=i)
            npu.run("qkv_post", QKV_ART.get(M, f"glue-qkv32-m{M}"), [self.c_qkv, self.tabs[i], self.q, self.kv])
            self.attn(npu, self.q, self.kv, kv_prefix[i], self.o)
            gemm(npu, w, "o", M, self.o, self.c, block=i)
            npu.run("ln_mod", ln_art, [self.x[0], self.c, self.p_mlp, self.x[1], self.a])
            npu.run("up_swiglu", GEMMS.get(("up_swiglu", M), f"atb3sw2-m{M}"), [self.a, w.b[i, "up"], self.h])
            gemm(npu, w, "down", M, self.h, self.c, block=i)
            p = self.p_out if i == self.n_blocks - 1 else self.p_attn
            npu.run("ln_mod", ln_art, [self.x[1], self.c, p, self.x[0], self.a])
        return 0

    def embed(self, npu, latents_pack):
        """img_in on the target latents (A layout, V9) and block 0's LN1: x[0] = img_in, a = LN1 (:256-259)."""
        gemm(npu, self.w, "img_in", self.M, latents_pack, self.c_in)
        npu.run("ln_mod", LN_ART.get(self.M, f"glue-ln-m{self.M}-s0"),
                [self.zero_x, self.c_in, self.p_first, self.x[0], self.a])

    def project(self, npu, a=None):
        """proj_out on a (the norm_out output after the last block) -> v (M, 64) float32 on the device (:261-269)."""
        if a is not None:
            self.a = a
        gemm(npu, self.w, "proj_out", self.M, self.a, self.c_out)
        npu.sync()
        return layouts.from_bfp16_c_atb(self.c_out, self.M, 1024)[:, :64]
