"""Projection-stack driver: the seven NF4 projections of n Qwen2 decoder layers, forward and
backward, on an unpadded (varlen) token batch.

Reference: the projection GEMMs of FusedDecoderLayer (/root/reference/solution/layer.py:871-929
forward; 982-1090 backward, LoRA on q and v at 1072-1090) applied to the packed token matrix
whose row count is the number of real tokens, cu_seqlens[-1] (unpad.py:249-250, 283-292).
Everything between the projections (norms, RoPE, attention, SwiGLU) is outside this path: each
layer reads fixed input buffers, so a step is exactly the projection work of the stack.

Every launch goes through the C ABI with argument arrays built once, on torch's current
stream, in the order the reference runs them:
  forward, per layer:  q|k|v (+bias, +LoRA, whose t_q = X A_q^T and t_v = X A_v^T the call
                       computes and keeps per layer for the backward: inside the GEMM launch
                       on the skinny small-M path, else one launch of its own before it); o;
                       gate|up; down
  backward, reversed:  dX down; dX gate|up; dX o; da_q, da_v (one launch); dB_q, dB_v, dA_q,
                       dA_v (one launch); dX q|k|v (+LoRA)
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .quant_state import quantize_4bit, weight_desc

GROUPS = (("qkv", ("q", "k", "v")), ("o", ("o",)), ("gu", ("gate", "up")), ("down", ("down",)))
GEMMS = ("fwd_qkv", "fwd_o", "fwd_gu", "fwd_down", "dx_down", "dx_gu", "dx_o", "dx_qkv")


@dataclass(frozen=True)
class Qwen2Shape:
    """Projection shapes of a Qwen2 decoder layer: q and o are hidden x hidden, k and v
    kv x hidden, gate and up inter x hidden, down hidden x inter ([out, in])."""
    hidden: int
    inter: int
    kv: int

    def weights(self):
        h, i, kv = self.hidden, self.inter, self.kv
        return {"q": (h, h), "k": (kv, h), "v": (kv, h), "o": (h, h),
                "gate": (i, h), "up": (i, h), "down": (h, i)}


QWEN2_15B = Qwen2Shape(hidden=1536, inter=8960, kv=256)
QWEN2_7B = Qwen2Shape(hidden=3584, inter=18944, kv=512)


def tokens_from_cu_seqlens(cu_seqlens) -> int:
    """Total real tokens of a varlen batch; cu_seqlens must start at 0 and not decrease."""
    c = torch.as_tensor(cu_seqlens).to("cpu", torch.int64)
    if c.dim() != 1 or c.numel() < 1 or int(c[0]) != 0 or bool((c[1:] < c[:-1]).any()):
        raise ValueError("cu_seqlens must be a 1-D non-decreasing sequence starting at 0")
    return int(c[-1])


class ProjectionStack:
    """n layers of NF4 projections with LoRA (rank r, scale alpha / r) on q and v and a q|k|v
    bias, fp16 or bf16, sized for up to `max_tokens` rows."""

    def __init__(self, layers, shape: Qwen2Shape, max_tokens: int, dtype=torch.float16,
                 device="cuda", rank: int = 16, alpha: float = 32.0, seed: int = 0):
        if dtype not in (torch.float16, torch.bfloat16):
            raise ValueError("the projection stack runs in float16 or bfloat16")
        self.lib = _lib.load()
        self.dt = _lib.DTYPE_CODE[dtype]
        self.dtype, self.dev, self.shape = dtype, torch.device(device), shape
        self.rank, self.scale = rank, alpha / rank
        self.max_tokens = max_tokens
        self.layers = layers
        h, i, kv = shape.hidden, shape.inter, shape.kv
        self.n_qkv = h + 2 * kv
        gen = torch.Generator(device=self.dev)

        def rnd(shp, s, std=1.0):
            gen.manual_seed(seed + s)
            return (torch.randn(shp, generator=gen, device=self.dev) * std).to(dtype)

        # activations (inputs of each projection) and upstream gradients: seeded N(0,1) and
        # N(0,1e-3), shared by every layer
        mt = max_tokens
        self.x, self.attn, self.x2 = rnd((mt, h), 1), rnd((mt, h), 11), rnd((mt, h), 12)
        self.act = rnd((mt, i), 13)
        self.dy_qkv, self.dy_o = rnd((mt, self.n_qkv), 2, 1e-3), rnd((mt, h), 21, 1e-3)
        self.dy_gu, self.dy_d = rnd((mt, 2 * i), 22, 1e-3), rnd((mt, h), 23, 1e-3)
        e = lambda *s: torch.empty(s, dtype=dtype, device=self.dev)  # noqa: E731
        self.da_q, self.da_v = e(mt, rank), e(mt, rank)
        self.y_qkv, self.y_o, self.y_gu, self.y_d = e(mt, self.n_qkv), e(mt, h), e(mt, 2 * i), e(mt, h)
        self.dx_d, self.dx_gu, self.dx_o, self.dx_qkv = e(mt, i), e(mt, h), e(mt, h), e(mt, h)

        # per layer: descriptor arrays, LoRA A (kaiming-uniform bound 1/sqrt(in)) / B
        # (N(0, 0.01)), the q|k|v bias and fp32 LoRA gradients
        self.per_layer = []
        for li, w in enumerate(layers):
            L = {}
            for g, names in GROUPS:
                L[g] = (_lib.NF4Weight * len(names))(*[weight_desc(*w[n]) for n in names])
                L[g + "_n"] = len(names)
            gen.manual_seed(seed + 3 + 1000 * li)
            bound = 1.0 / h ** 0.5
            L["a_q"] = ((torch.rand(rank, h, generator=gen, device=self.dev) * 2 - 1) * bound).to(dtype)
            L["a_v"] = ((torch.rand(rank, h, generator=gen, device=self.dev) * 2 - 1) * bound).to(dtype)
            gen.manual_seed(seed + 4 + 1000 * li)
            L["b_q"] = (torch.randn(h, rank, generator=gen, device=self.dev) * 0.01).to(dtype)
            L["b_v"] = (torch.randn(kv, rank, generator=gen, device=self.dev) * 0.01).to(dtype)
            L["bias"] = rnd((self.n_qkv,), 14 + 1000 * li, 0.1)
            f = lambda *s: torch.empty(s, dtype=torch.float32, device=self.dev)  # noqa: E731
            L["gb_q"], L["gb_v"], L["ga_q"], L["ga_v"] = f(h, rank), f(kv, rank), f(rank, h), f(rank, h)
            P, Lo = (lambda t: t.data_ptr()), _lib.NF4Lora
            # t = X A^T, computed by the q|k|v forward itself (A given) and read again by dB
            L["t_q"], L["t_v"] = e(mt, rank), e(mt, rank)
            L["fwd_loras"] = (Lo * 2)(Lo(0, rank, self.scale, P(L["t_q"]), P(L["b_q"]), P(L["a_q"]), None),
                                      Lo(2, rank, self.scale, P(L["t_v"]), P(L["b_v"]), P(L["a_v"]), None))
            L["dx_loras"] = (Lo * 2)(Lo(0, rank, self.scale, None, None, P(L["a_q"]), P(self.da_q)),
                                     Lo(2, rank, self.scale, None, None, P(L["a_v"]), P(self.da_v)))
            # the side products of both adapters, one launch each (nf4_lora_job arrays)
            J, es = _lib.NF4LoraJob, self.dy_qkv.element_size()
            dq, dv = P(self.dy_qkv), P(self.dy_qkv) + (h + kv) * es
            nq = self.n_qkv
            L["da_jobs"] = (J * 2)(J(dq, nq, h, P(L["b_q"]), P(self.da_q), self.scale, 0),
                                   J(dv, nq, kv, P(L["b_v"]), P(self.da_v), self.scale, 0))
            L["wg_jobs"] = (J * 4)(J(dq, nq, h, P(L["t_q"]), P(L["gb_q"]), self.scale, 0),
                                   J(dv, nq, kv, P(L["t_v"]), P(L["gb_v"]), self.scale, 0),
                                   J(P(self.x), h, h, P(self.da_q), P(L["ga_q"]), 1.0, 1),
                                   J(P(self.x), h, h, P(self.da_v), P(L["ga_v"]), 1.0, 1))
            self.per_layer.append(L)
        self.ws = {}
        self.set_tokens(torch.tensor([0, max_tokens], dtype=torch.int32))

    # ---------------------------------------------------------------------------- building

    @classmethod
    def synthetic(cls, shape: Qwen2Shape, n_layers: int, max_tokens: int, dtype=torch.float16,
                  device="cuda", seed_base: int = 100, seed_stride: int = 7, **kw):
        """Layers of seeded N(0, 0.02) weights quantized to NF4 with double quant on the GPU:
        layer l, weight i (q, k, v, o, gate, up, down) uses seed seed_base + seed_stride*l + i."""
        dev = torch.device(device)
        layers = []
        for li in range(n_layers):
            w = {}
            for i, (name, (n, k)) in enumerate(shape.weights().items()):
                g = torch.Generator(device=dev).manual_seed(seed_base + seed_stride * li + i)
                packed, qs = quantize_4bit(torch.randn(n, k, generator=g, device=dev) * 0.02)
                w[name] = (packed.view(-1), qs)
            layers.append(w)
        return cls(layers, shape, max_tokens, dtype, dev, **kw)

    def set_tokens(self, cu_seqlens) -> int:
        """Use the first cu_seqlens[-1] rows of every buffer (the batch's real tokens)."""
        m = tokens_from_cu_seqlens(cu_seqlens)
        if m > self.max_tokens:
            raise ValueError(f"{m} tokens exceed the stack's max_tokens {self.max_tokens}")
        self.m = m
        lib, L0 = self.lib, self.per_layer[0]
        need = {}
        for g, _ in GROUPS:
            need[g] = (lib.nf4_linear_fwd_workspace(m, L0[g], L0[g + "_n"], self.dt),
                       lib.nf4_linear_dx_workspace(m, L0[g], L0[g + "_n"], self.dt))
        need["wgrad"] = (lib.nf4_lora_wgrad_multi_workspace(L0["wg_jobs"], 4, m, self.rank), 0)
        for key, (fb, db) in need.items():
            have = self.ws.get(key)
            if have is None or have[1] < fb or have[3] < db:
                self.ws[key] = (torch.empty(max(fb, 1), dtype=torch.uint8, device=self.dev), fb,
                                torch.empty(max(db, 1), dtype=torch.uint8, device=self.dev), db)
        return m

    # ------------------------------------------------------------------------------ counts

    def flops(self) -> dict:
        """Algorithmic flops of one forward+backward at the current token count: 2 M N K per
        projection each way, LoRA 2 M r (K + N) forward and 2 M r (2 K + 2 N) backward on q, v."""
        m, r, h, kv = self.m, self.rank, self.shape.hidden, self.shape.kv
        f = {}
        for g, names in GROUPS:
            nk = sum(self.shape.weights()[n][0] * self.shape.weights()[n][1] for n in names)
            f["fwd_" + g] = 2 * m * nk
            f["dx_" + g] = 2 * m * nk
        f["lora_fwd"] = 2 * m * r * (h + h) + 2 * m * r * (h + kv)
        f["lora_bwd"] = 2 * 2 * m * r * (h + h) + 2 * 2 * m * r * (h + kv)
        per_layer = sum(f.values())
        return {"per_layer": f, "total": per_layer * len(self.per_layer)}

    def weight_bytes(self) -> int:
        """NF4 bytes the stack reads per pass over its weights (packed + uint8 absmax + fp32
        absmax2), the GEMV-regime traffic floor."""
        total = 0
        for w in self.layers:
            for _, (packed, qs) in w.items():
                n = int(qs.shape[0]) * int(qs.shape[1])
                total += n // 2 + n // 64 + 4 * -(-n // 16384)
        return total

    # ----------------------------------------------------------------------------- launches

    def _chk(self, st, what):
        if st != 0:
            raise RuntimeError(f"{what}: status {st} ({self.lib.nf4_status_string(st).decode()})")

    def forward(self, ev=None, layers=None):
        """Queue the forward projections of every layer (or of `layers`).  `ev`: dict GEMM name
        -> (start, end) events recorded around that GEMM's launch (one layer at a time); GEMMs
        not in it run unbracketed."""
        lib, dt, m = self.lib, self.dt, self.m
        s = torch.cuda.current_stream(self.dev).cuda_stream
        P = lambda t: t.data_ptr()  # noqa: E731
        h, i, nq, r = self.shape.hidden, self.shape.inter, self.n_qkv, self.rank
        ws = self.ws
        for li in (range(len(self.per_layer)) if layers is None else layers):
            L = self.per_layer[li]
            self._timed(ev, "fwd_qkv", lambda: lib.nf4_linear_fwd(
                P(self.x), m, h, L["qkv"], 3, P(L["bias"]), L["fwd_loras"], 2, P(self.y_qkv), nq,
                dt, P(ws["qkv"][0]), ws["qkv"][1], s))
            self._timed(ev, "fwd_o", lambda: lib.nf4_linear_fwd(
                P(self.attn), m, h, L["o"], 1, None, None, 0, P(self.y_o), h, dt,
                P(ws["o"][0]), ws["o"][1], s))
            self._timed(ev, "fwd_gu", lambda: lib.nf4_linear_fwd(
                P(self.x2), m, h, L["gu"], 2, None, None, 0, P(self.y_gu), 2 * i, dt,
                P(ws["gu"][0]), ws["gu"][1], s))
            self._timed(ev, "fwd_down", lambda: lib.nf4_linear_fwd(
                P(self.act), m, i, L["down"], 1, None, None, 0, P(self.y_d), h, dt,
                P(ws["down"][0]), ws["down"][1], s))

    def backward(self, ev=None, layers=None):
        """Queue the backward projections (input gradients and LoRA gradients), last layer
        first."""
        lib, dt, m = self.lib, self.dt, self.m
        s = torch.cuda.current_stream(self.dev).cuda_stream
        P = lambda t: t.data_ptr()  # noqa: E731
        h, i, nq, r = self.shape.hidden, self.shape.inter, self.n_qkv, self.rank
        ws = self.ws
        wg, wb = P(ws["wgrad"][0]), ws["wgrad"][1]
        order = reversed(range(len(self.per_layer))) if layers is None else layers
        for li in order:
            L = self.per_layer[li]
            self._timed(ev, "dx_down", lambda: lib.nf4_linear_dx(
                P(self.dy_d), m, h, L["down"], 1, None, 0, P(self.dx_d), i, 0, dt,
                P(ws["down"][2]), ws["down"][3], s))
            self._timed(ev, "dx_gu", lambda: lib.nf4_linear_dx(
                P(self.dy_gu), m, 2 * i, L["gu"], 2, None, 0, P(self.dx_gu), h, 0, dt,
                P(ws["gu"][2]), ws["gu"][3], s))
            self._timed(ev, "dx_o", lambda: lib.nf4_linear_dx(
                P(self.dy_o), m, h, L["o"], 1, None, 0, P(self.dx_o), h, 0, dt,
                P(ws["o"][2]), ws["o"][3], s))
            dq = P(self.dy_qkv)
            self._chk(lib.nf4_lora_da_multi(L["da_jobs"], 2, m, r, dt, s), "da")
            self._chk(lib.nf4_lora_wgrad_multi(L["wg_jobs"], 4, m, r, dt, wg, wb, s), "wgrad")
            self._timed(ev, "dx_qkv", lambda: lib.nf4_linear_dx(
                dq, m, nq, L["qkv"], 3, L["dx_loras"], 2, P(self.dx_qkv), h, 0, dt,
                P(ws["qkv"][2]), ws["qkv"][3], s))

    def step(self, ev=None):
        self.forward(ev)
        self.backward(ev)

    def _timed(self, ev, name, fn):
        timed = ev is not None and name in ev
        if timed:
            ev[name][0].record()
        self._chk(fn(), name)
        if timed:
            ev[name][1].record()
