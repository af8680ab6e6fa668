"""The DiT GEMM call surface of redline/forward.py, on the HIP path.

Names, arguments and meaning follow the reference: ``GEMMS`` (artifact name per (op, M)), ``GEMM_KN``, ``v9``,
``NPU.run(op, art, args)`` / ``NPU.sync()`` / ``NPU.report()`` (GEMMs and the "ln_mod" pass), ``Weights`` (the packed ``bNN_*.bin`` files plus
``manifest.json`` that redline/pack_weights.py writes) and ``gemm(npu, w, op, M, a, c, block=None)``
(redline/forward.py:33-44, :82-84, :87-172, :175-197).

Differences, all deliberate:
  * buffers are torch tensors on the GPU, and work is enqueued on torch's current HIP stream (``run`` never blocks;
    ``sync`` synchronises the stream);
  * A may be a bf16 (M, K) activation tensor (the build's native operand, already bfp16 values or quantized while it
    is loaded, see ``NPU.a_fmt``) or a V9 uint8 tensor in the reference's A layout (a_layout(., 128, 64));
  * C may be a bf16 (M, N) tensor (the build's native output: fp32 accumulation, one bf16 rounding) or a V9 uint8
    tensor, which then receives the reference's own stream order: the ATB C order for plain GEMMs
    (c_layout_atb(., 128, 128)) and the down-GEMM A layout (a_layout(., 128, 64)) for ``up_swiglu``.
"""

import hashlib
import json
import time
from collections import defaultdict
from pathlib import Path

import numpy as np
import torch

from . import ops, run_ln

N_BLOCKS, HID, FF = 32, 4096, 12288
M_S1 = 8704

# artifact names per (op, M) as in redline/forward.py:33-42; here they select the epilogue of the HIP GEMM
LN_ART = {4096: "glue-ln-m4096-s0", M_S1: "glue-ln-m8704-s33"}  # redline/forward.py:205
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


def artifact_kind(art):
    """'swiglu' for the SwiGLU-flush GEMMs (atb3sw*, vlm-upsw*), else 'gemm'."""
    return "swiglu" if art.startswith("atb3sw") or "upsw" in art else "gemm"


def v9(nvals, device="cuda"):
    """A device buffer holding nvals bfp16 values (nvals / 8 blocks of 9 bytes), zeroed (redline/forward.py:82-84)."""
    return torch.zeros(nvals // 8 * 9, dtype=torch.uint8, device=device)


def bf16_tensor(a, device="cuda"):
    """float array -> flat bf16 device tensor (redline/forward.py:200-202)."""
    return torch.as_tensor(np.asarray(a, np.float32)).to(device=device, dtype=torch.bfloat16).reshape(-1)


class NPU:
    """Kernel runner with per-op timing (device time from HIP events, wall time of the enqueue), like
    redline/forward.py:87-172. ``kn`` maps op -> (K, N) for A operands that do not carry K (packed A)."""

    def __init__(self, kn=None, a_fmt="bf16"):
        self.kn = dict(GEMM_KN if kn is None else kn)
        self.a_fmt = a_fmt
        self.t_npu, self.t_wall, self.calls = defaultdict(float), defaultdict(float), defaultdict(int)
        self.pending = []  # (op, start event, end event, args kept alive until sync)

    def sync(self):
        """Wait for every enqueued run and account its device time."""
        torch.cuda.current_stream().synchronize()
        for op, e0, e1, _args in self.pending:
            self.t_npu[op] += e0.elapsed_time(e1) / 1e3
        self.pending = []

    def run(self, op, art, args):
        """args = [A, B, C] (or [A, W_up, H] for up_swiglu), see the module docstring for the accepted forms; or
        [X, BR, P, XO, AO] for the fused residual + LayerNorm + modulate artifacts ("ln_mod", glue-ln-m{M}-s{S}, and
        the RMSNorm copies), run by run_ln.ln_fused."""
        t = time.perf_counter()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        if len(args) == 5:
            run_ln.ln_fused(art, *args)
        else:
            a, b, c = args
            self._gemm(op, art, a, b, c)
        e1.record()
        self.pending.append((op, e0, e1, list(args)))
        self.t_wall[op] += time.perf_counter() - t
        self.calls[op] += 1

    def _gemm(self, op, art, a, b, c):
        kind = "swiglu" if op == "up_swiglu" else artifact_kind(art)
        base = "up" if op == "up_swiglu" else op
        if a.dtype == torch.bfloat16:
            M, K = a.shape
            fmt = self.a_fmt
        else:
            K = self.kn[base][0]
            M = a.numel() // 9 * 8 // K
            fmt = "packed_a_layout"
        N = b.numel() // 9 * 8 // K
        act = "swiglu" if kind == "swiglu" else None
        nout = N // 2 if act else N
        if c.dtype == torch.bfloat16:
            ops.gemm(a, b, N, K, M=M, a_fmt=fmt, act=act, out=c.view(M, nout))
            return
        # V9 output: the reference's stream order, from the bf16 result
        y = ops.gemm(a, b, N, K, M=M, a_fmt=fmt, act=act)
        p, _ = ops.quantize(y, order="a_layout" if act else "c_atb")
        c.copy_(p)

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
