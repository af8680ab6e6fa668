"""The text encoder's NPU call surface of redline/vlm_run.py, on the HIP path.

``run(art, args)`` takes the artifacts that LM._run and LM._rms issue (redline/vlm_run.py:56-57, :340-344, :427-449)
and returns the device time in ms once the run is done, as ``DefaultNPURuntime.run(...).npu_time / 1e6`` does:

  vlm-rms-m{M}, vlm-rms16-m{M}            [X, BR, P, XO, AO]  residual + RMSNorm glue (run_ln.ln_fused): X / XO bf16
                                                               in the C-stream order, BR bfp16 (or bf16 for rms16) in
                                                               that order, AO bfp16 in the A layout
  vlm-gemm-{qkv,o,up,down}[16]            [A, B, C]           GEMMs: A bfp16 in the A layout, C bfp16 in the C-stream
                                                               order, or flat bf16 in that order for the "16" copies
  vlm-upsw-m{M}, vlm-upswx-m{M}           [A, W_up, H]        up GEMM with the SwiGLU epilogue, H in the A layout
  vlm-qkv-m{M}, vlm-qkv16-m{M}            [C, TABS, Q, KV]    GQA QKV post (run_qkv.qkv_post_run)
  vlm-attn-m{M}-t{NQT}-x                  [Q, KV, O]          causal GQA attention (run_attn.run_artifact)
  vlm-swiglu-m{M}                         [C_up, H]           the unfused SwiGLU glue

``rms_params``, ``rms_ref``, ``check_c16`` and ``LM`` keep the reference's names and meaning; ``LM`` runs one decoder
layer as the chain of those artifacts over device buffers, with the shapes taken from its weights.
"""

import math
from pathlib import Path

import numpy as np
import torch

from . import forward, layouts, ops, run_qkv

M, D, L = 1536, 4096, 1070      # padded prompt rows, hidden width, prompt length (redline/vlm_run.py:22)
HQ, HKV, HD = 32, 8, 128         # q heads, kv heads, head dim (:23)
C_LOG2 = float(np.log2(np.e) / np.sqrt(HD))

_NPU = forward.NPU()

# artifact prefix -> NPU.run op key
_OPS = (("vlm-rms", "rms"), ("vlm-gemm-", None), ("vlm-upsw", "up+swiglu"), ("vlm-qkv", "qkv_post"),
        ("vlm-attn", "attn"), ("vlm-swiglu", "swiglu"))


def _op(art):
    name = Path(str(art)).name
    for prefix, op in _OPS:
        if name.startswith(prefix):
            return op or name[len(prefix):].rstrip("0123456789").split("-")[0]
    raise KeyError(f"{art}: not a text-encoder artifact")


def run(art, args):
    """Run one artifact on its buffers (redline/vlm_run.py:56-57); returns its device time in ms."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    _NPU._dispatch(_op(art), str(art), list(args))
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1)


def v9(nvals, device="cuda"):
    return forward.v9(nvals, device)


def bf(a):
    """Values rounded to bf16 (RNE), as float32 (redline/vlm_run.py:26-27)."""
    return torch.as_tensor(a).to(torch.bfloat16).to(torch.float32)


def rms_params(w, g=1.0, device="cuda"):
    """P buffer: rows [g | w] x 2 (row 1 unused at S = 0), flat bf16 (redline/vlm_run.py:62-65)."""
    w = torch.as_tensor(w, dtype=torch.float32).to(device)
    row = torch.cat([torch.full_like(w, g), w])
    return torch.cat([row, row]).to(torch.bfloat16)


def rms_ref(xq, brq, w):
    """x' = bf16(x + br), y = x' / rms(x') * w with float64 statistics (redline/vlm_run.py:68-70)."""
    xp = bf(torch.as_tensor(xq) + torch.as_tensor(brq))
    xd = xp.double()
    return xp, xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + 1e-6) * torch.as_tensor(w).double()


def stats(name, got, ref):
    """Correlation and max |got - ref| / max |ref| (redline/vlm_run.py:30-36); printed and returned."""
    got, ref = got.double().reshape(-1), ref.double().reshape(-1)
    c = float(torch.corrcoef(torch.stack([got, ref]))[0, 1])
    e = float((got - ref).abs().max() / ref.abs().max())
    print(f"  {name:34s} corr {c:.6f}  max err {e:.4f}")
    return c, e


def check_c16(m=M, d=D, seed=3, device="cuda"):
    """bf16-C GEMM (vlm-gemm-o16) and the bf16-branch RMS glue (vlm-rms16) on random data, as
    redline/vlm_run.py:95-120: the C16 output against float64 on the bfp16 inputs, x' bit-exact, y against the
    float64 RMSNorm. Returns the figures, and the C16 (c_t), x' (xo_t) and A (ao_t) buffers, as a dict."""
    rng = np.random.default_rng(seed)
    a = torch.as_tensor(rng.standard_normal((m, d)).astype(np.float32), device=device)
    b = torch.as_tensor((rng.standard_normal((d, d)) / 64).astype(np.float32), device=device)
    ap, aq = ops.quantize(a, order="a_layout", deq=True)
    bp = layouts.pack_b(b)
    bq = layouts.unpack_b(bp, d, d)
    c_t = torch.zeros(m * d, dtype=torch.bfloat16, device=device)
    ms_gemm = run("vlm-gemm-o16", [ap, bp, c_t])
    c = layouts.c_unlayout_atb_values(c_t, m, d).float()
    print(f"gemm-o16: {ms_gemm:.3f} ms")
    c_corr, c_err = stats("bf16 C vs float64 (bfp16 inputs)", c, aq.double() @ bq.double())
    x = torch.as_tensor((rng.standard_normal((m, d)) * 3).astype(np.float32), device=device)
    w = torch.as_tensor((1 + 0.2 * rng.standard_normal(d)).astype(np.float32), device=device)
    xo_t, ao_t = torch.zeros(m * d, dtype=torch.bfloat16, device=device), v9(m * d, device)
    x_t = layouts.c_layout_atb_values(bf(x).to(torch.bfloat16))
    ms_rms = run(f"vlm-rms16-m{m}", [x_t, c_t, rms_params(w, device=device), xo_t, ao_t])
    xo = layouts.c_unlayout_atb_values(xo_t, m, d).float()
    y = layouts.a_unlayout(ao_t, m, d, 128, 64)
    xr, yr = rms_ref(bf(x), c, w)
    exact = bool(torch.equal(xo, xr))
    print(f"rms16: {ms_rms:.3f} ms;  x' bit-exact: {exact}")
    y_corr, y_err = stats("y vs numpy RMSNorm", y, yr)
    return {"c_corr": c_corr, "c_err": c_err, "x_exact": exact, "y_corr": y_corr, "y_err": y_err,
            "ms_gemm": ms_gemm, "ms_rms": ms_rms, "c_t": c_t, "xo_t": xo_t, "ao_t": ao_t}


class LM:
    """Resident weights + device buffers; layer(i) runs one decoder layer as the chain of artifacts of
    redline/vlm_run.py:427-449 (buffers chained, no host round trips).

    weights: pack.VlmWeights, or any object with ``w[i, m]`` (the packed qkv / o / up / down streams), ``qk[i]``
    (balanced q/k norm weights), ``p_in[i]`` / ``p_post[i]`` (rms_params buffers) and ``hp`` (hidden channel order).
    m (rows), hq / hkv (heads) and the prompt length select the shapes; hidden width and FFN width come from the
    weights."""

    def __init__(self, weights, cos, sin, layers=None, attn=None, m=M, hq=HQ, hkv=HKV, length=L, device="cuda"):
        self.wts, self.m, self.hq, self.hkv, self.length = weights, m, hq, hkv, length
        self.layers = sorted({k[0] for k in weights.w}) if layers is None else list(layers)
        l0 = self.layers[0]
        self.d = weights.p_in[l0].numel() // 4
        self.f = weights.w[l0, "up"].numel() // 9 * 8 // self.d // 2
        self.hp = torch.as_tensor(np.asarray(weights.hp), device=device)
        self.w = {k: v for k, v in weights.w.items()}
        d, f, T = self.d, self.f, m // 64
        z = lambda n: torch.zeros(n, dtype=torch.bfloat16, device=device)
        self.x = [z(m * d), z(m * d), z(m * d)]          # residual stream ping-pong (bf16, C-stream order)
        self.br_zero = v9(m * d, device)
        self.a1, self.a2, self.oa = v9(m * d, device), v9(m * d, device), v9(m * d, device)
        nqkv = (hq + 2 * hkv) * HD
        self.cqkv, self.co, self.cup, self.h, self.cd = (v9(m * nqkv, device), v9(m * d, device),
                                                         v9(m * 2 * f, device), v9(m * f, device), v9(m * d, device))
        self.q, self.kv = v9(hq * T * 64 * HD, device), v9(hkv * T * 2 * 64 * HD, device)
        self.t = {}
        self.attn = attn or f"vlm-attn-m{m}-t{math.ceil(length / 64)}-x"
        self.fused_up = True
        self.upsw_art = f"vlm-upsw-m{m}"
        self.c16_layers = set()
        self.co16, self.cd16 = z(m * d), z(m * d)
        self.br16 = False
        self.qkv16 = False
        self.cqkv16 = z(m * nqkv)
        self.tabs = {}
        self.set_tables(cos, sin)
        self.cur, self.br = 0, self.br_zero

    def _run(self, op, art, args):
        self.t[op] = self.t.get(op, 0.0) + run(art, args)

    def _rms(self, x, br, br16, p, xo, a):
        self._run("rms", f"vlm-rms16-m{self.m}" if br16 else f"vlm-rms-m{self.m}", [x, br, p, xo, a])

    def set_tables(self, cos, sin):
        """qkv_post tables for the prompt's positions (cos / sin (m, 64) per row), per layer with its balanced q/k norm
        weights, q's carrying log2(e)/sqrt(128) (redline/vlm_run.py:352-361)."""
        cos, sin = torch.as_tensor(cos).cuda(), torch.as_tensor(sin).cuda()
        for i in self.layers:
            wq, wk = self.wts.qk[i]
            self.tabs[i] = run_qkv.qkv_tables(cos, sin, bf(torch.as_tensor(wq).cuda() * C_LOG2),
                                              torch.as_tensor(wk).cuda()).reshape(-1)

    def load_x(self, x):
        """x (rows, hidden) in the model's channel order; stored in the packed weights' order (:363-366)."""
        xp = torch.zeros((self.m, self.d), dtype=torch.float32, device=self.hp.device)
        x = torch.as_tensor(x, device=self.hp.device).float()
        xp[:x.shape[0]] = x
        self.x[0] = layouts.c_layout_atb_values(bf(xp[:, self.hp]).to(torch.bfloat16))
        self.cur, self.br, self.br16 = 0, self.br_zero, False

    def unperm(self, xp):
        out = torch.empty_like(xp)
        out[:, self.hp] = xp
        return out

    def layer(self, i):
        self._layer(i)

    def _layer(self, i):
        w = self.wts
        x0, x1 = self.x[self.cur], self.x[(self.cur + 1) % 3]
        self._rms(x0, self.br, self.br16, w.p_in[i], x1, self.a1)
        if self.qkv16:
            self._run("qkv", "vlm-gemm-qkv16", [self.a1, self.w[i, "qkv"], self.cqkv16])
            self._run("qkv_post", f"vlm-qkv16-m{self.m}", [self.cqkv16, self.tabs[i], self.q, self.kv])
        else:
            self._run("qkv", "vlm-gemm-qkv", [self.a1, self.w[i, "qkv"], self.cqkv])
            self._run("qkv_post", f"vlm-qkv-m{self.m}", [self.cqkv, self.tabs[i], self.q, self.kv])
        self._run("attn", self.attn, [self.q, self.kv, self.oa])
        c16 = i in self.c16_layers
        co = self.co16 if c16 else self.co
        self._run("o", "vlm-gemm-o16" if c16 else "vlm-gemm-o", [self.oa, self.w[i, "o"], co])
        x2 = self.x[(self.cur + 2) % 3]
        self._rms(x1, co, c16, w.p_post[i], x2, self.a2)
        if self.fused_up:
            self._run("up+swiglu", self.upsw_art, [self.a2, self.w[i, "up"], self.h])
        else:
            self._run("up", "vlm-gemm-up", [self.a2, self.w[i, "up"], self.cup])
            self._run("swiglu", f"vlm-swiglu-m{self.m}", [self.cup, self.h])
        cd = self.cd16 if c16 else self.cd
        self._run("down", "vlm-gemm-down16" if c16 else "vlm-gemm-down", [self.h, self.w[i, "down"], cd])
        self.cur, self.br, self.br16 = (self.cur + 2) % 3, cd, c16

    def x_out(self, last_i):
        """The residual stream after the last layer (x2 + down), via one more rms pass (its A output unused)."""
        x0, x1 = self.x[self.cur], self.x[(self.cur + 1) % 3]
        self._rms(x0, self.br, self.br16, self.wts.p_in[last_i], x1, self.a1)
        return self.unperm(layouts.c_unlayout_atb_values(x1, self.m, self.d).float())
