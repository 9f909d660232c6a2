"""Benchmark of the NF4 quantized-linear path on one MI355X (gfx950).

One step = forward + backward of the seven NF4 projections of one Qwen2.5-1.5B decoder layer
at M = 2048 tokens: q|k|v stacked with bias and LoRA r=16 on q and v,
o, gate|up stacked, down; backward = the input gradients of all of them plus the LoRA dA/dB.
Every weight is dequantized inside the fused GEMMs (twice per step, as in the reference).
Inputs are synthetic (seeded N(0,1) activations, N(0,0.02) weights quantized to NF4 with double
quant, LoRA A kaiming-uniform, B N(0,0.01), dY N(0,1e-3)) and resident in HBM before timing.

Prints ONE JSON line: value = algorithmic TFLOP/s of the whole step (384.28 GFLOP), the
roofline of the dominant GEMM kernel (HIP events around its launches, on the launch stream),
the standalone dequant's HBM GB/s over the 28-layer stack (3.3 GB), and the CPU oracle timed on
the host cores as a baseline.  The other BASELINE configs ride along in the same line:
`varlen_stack` (config 3: the 28-layer Qwen2.5-1.5B projection stack on a varlen batch),
`qwen7b_m8192` (config 4: a Qwen2.5-7B layer in bf16 at M=8192) and `gemv_15b` / `gemv_7b`
(config 4: forward over the 28-layer stacks at M in {1, 8, 64}, HBM GB/s).

    python bench.py [--steps K] [--warmup W] [--dtype f16|bf16] [--no-cpu-baseline]
                    [--no-dequant] [--no-stack] [--no-7b] [--no-gemv]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "kaggle-mltest_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "NF4 dequant-GEMM TFLOP/s (% MFMA peak) at M=2048; dequant HBM GB/s"
PEAK_MFMA_TFLOPS = 2516.6   # MI355X dense fp16 / bf16
PEAK_HBM_GBPS = 8000.0      # MI355X HBM3E
M = 2048
RANK, ALPHA = 16, 32
# (name, out_features N, in_features K) of one Qwen2.5-1.5B decoder layer
LAYER = [("q", 1536, 1536), ("k", 256, 1536), ("v", 256, 1536), ("o", 1536, 1536),
         ("gate", 8960, 1536), ("up", 8960, 1536), ("down", 1536, 8960)]
DEQUANT_BYTES_PER_ELEMENT = 0.5 + 1 / 64 + 2  # packed + uint8 absmax + fp16 out (+ absmax2)


def dequant_bytes(n_elements: int) -> int:
    return n_elements // 2 + n_elements // 64 + 4 * -(-n_elements // 16384) + 2 * n_elements


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--dtype", choices=["f16", "bf16"], default="f16")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-dequant", action="store_true")
    ap.add_argument("--no-stack", action="store_true",
                    help="skip the 28-layer varlen projection stack (config 3)")
    ap.add_argument("--no-7b", action="store_true",
                    help="skip the Qwen2.5-7B bf16 M=8192 layer (config 4)")
    ap.add_argument("--no-gemv", action="store_true",
                    help="skip the small-M forward sweeps over the 28-layer stacks")
    ap.add_argument("--no-swiglu", action="store_true",
                    help="skip the gate|up + SwiGLU epilogue comparison")
    ap.add_argument("--no-int8", action="store_true",
                    help="skip the int8 MLP input-gradient leg (the reference's T4 backward)")
    ap.add_argument("--no-norm-rope", action="store_true",
                    help="skip the RMSNorm / RoPE neighbours of the projection")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only the small-M forward sweeps (gemv_15b, gemv_7b), printed as one "
                         "JSON object: the command the decode-regime profiles are taken with")
    ap.add_argument("--gemv-ms", default="1,8,64",
                    help="token counts M of the small-M sweeps (comma-separated)")
    ap.add_argument("--cpu-reps", type=int, default=5)
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="after timing, copy this many MiB device-to-device 3 times: the "
                         "known-size kernel that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE")
    return ap.parse_args()


# ----------------------------------------------------------------------------- workload

class Workload:
    """One Qwen2.5-1.5B layer on the projection-stack driver: weights,
    inputs, every output buffer and the prebuilt C-ABI arguments of one step."""

    def __init__(self, dtype, dev):
        from solution.stack import QWEN2_15B, ProjectionStack

        self.stack = ProjectionStack.synthetic(QWEN2_15B, 1, M, dtype, dev, seed_base=100,
                                               rank=RANK, alpha=ALPHA)
        self.lib = self.stack.lib

    # flops of one step, counted from the shapes
    @staticmethod
    def flops():
        gemm = sum(2 * M * n * k for _, n, k in LAYER)
        k, n_q, n_v = 1536, 1536, 256
        # forward: x A^T then (.) B^T, for q and v
        lora_fwd = 2 * M * RANK * (k + n_q) + 2 * M * RANK * (k + n_v)
        # backward: da = dY B, dB = dY^T t, dA = da^T x, dX += da A, for q and v
        lora_bwd = 2 * M * RANK * (2 * n_q + 2 * k) + 2 * M * RANK * (2 * n_v + 2 * k)
        return {"gemm_fwd": gemm, "gemm_dx": gemm, "lora_fwd": lora_fwd, "lora_bwd": lora_bwd,
                "total": 2 * gemm + lora_fwd + lora_bwd}

    def gemm_flops(self):
        f = {}
        for gname, names in (("qkv", ["q", "k", "v"]), ("o", ["o"]), ("gu", ["gate", "up"]),
                             ("down", ["down"])):
            n = sum(dict((a, b) for a, b, _ in LAYER)[nm] for nm in names)
            k = dict((a, c) for a, _, c in LAYER)[names[0]]
            lora = 2 * M * RANK * (1536 + 256) if gname == "qkv" else 0
            f[f"fwd_{gname}"] = 2 * M * n * k + lora
            f[f"dx_{gname}"] = 2 * M * n * k + (2 * M * RANK * 1536 * 2 if gname == "qkv" else 0)
        return f

    def step(self, ev=None):
        """Queue one forward+backward on torch's current stream.  `ev`: dict name -> (start,
        end) events recorded around each fused GEMM launch."""
        self.stack.step(ev)


def _time_graph(torch, fn, reps, warmup=1):
    """Mean ms of one replay of a HIP graph captured from `fn` (its launches queued on the
    capture stream): launch-bound sequences measured without per-launch host overhead."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    del g
    return e0.elapsed_time(e1) / reps


def _time_steps(torch, fn, steps, warmup):
    """Mean ms of `fn` over `steps` runs after `warmup`, HIP events on the current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


# ------------------------------------------------------------- gate|up with SwiGLU epilogue

def swiglu_leg(dtype, dev, reps=20, warmup=3):
    """The MLP's gate|up step at M=2048 (Qwen2.5-1.5B: I 8960, K 1536) with the SwiGLU step in
    the GEMM epilogue vs the stacked GEMM writing [M, 2I] followed by the SwiGLU kernel; forward
    (H) and backward (recompute + dG|dU)."""
    import torch

    from solution import kernels
    from solution.quant_state import quantize_4bit

    inter, k = 8960, 1536
    g = torch.Generator(device=dev)
    w = []
    for s in (201, 202):
        g.manual_seed(s)
        packed, qs = quantize_4bit(torch.randn(inter, k, generator=g, device=dev) * 0.02)
        w.append((packed.view(-1), qs))
    gate, up = w
    g.manual_seed(203)
    x = torch.randn(M, k, generator=g, device=dev).to(dtype)
    dh = (torch.randn(M, inter, generator=g, device=dev) * 1e-2).to(dtype)
    h = torch.empty(M, inter, dtype=dtype, device=dev)
    gu = torch.empty(M, 2 * inter, dtype=dtype, device=dev)

    def unfused_fwd():
        kernels.linear_fwd(x, [gate, up], out=gu)
        kernels.swiglu_fwd(gu[:, :inter], gu[:, inter:])

    def unfused_bwd():
        kernels.linear_fwd(x, [gate, up], out=gu)
        kernels.swiglu_bwd(dh, gu[:, :inter], gu[:, inter:], gu[:, :inter], gu[:, inter:])

    t = {"fused_fwd": lambda: kernels.linear_swiglu_fwd(x, gate, up, out=h),
         "unfused_fwd": unfused_fwd,
         "fused_bwd": lambda: kernels.linear_swiglu_bwd(x, gate, up, dh, out=gu),
         "unfused_bwd": unfused_bwd}
    res = {n: round(_time_steps(torch, fn, reps, warmup) * 1e3, 2) for n, fn in t.items()}
    gflop = 2 * M * 2 * inter * k / 1e9
    return {"mlp_swiglu": {
        "workload": "Qwen2.5-1.5B gate|up (2 x 8960 x 1536) + SwiGLU, M=2048; fused = SwiGLU in "
                    "the GEMM epilogue (no [M, 2I] round trip), unfused = stacked GEMM + kernel",
        "us": res, "gflop": round(gflop, 3),
        "fused_fwd_tflops": round(gflop / res["fused_fwd"] * 1e3, 1),
        "speedup_fwd": round(res["unfused_fwd"] / res["fused_fwd"], 3),
        "speedup_bwd": round(res["unfused_bwd"] / res["fused_bwd"], 3)}}


# ---------------------------------------------- int8 input gradients (off the parity path)

PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA


def int8_leg(dev, reps=20):
    """The MLP input gradient at M=2048 on the Qwen2.5-1.5B shapes (dh2 [M, 1536] -> dy2) two
    ways, each captured in a HIP graph: the fp16 path (fused NF4 dX GEMM of down, SwiGLU
    backward, fused NF4 dX GEMM of gate|up) and the int8 path of the reference's T4 backward
    (int8 rows, int8 weights made from the NF4 bytes, two int8 GEMMs, SwiGLU backward
    requantized); plus each int8 GEMM alone against the 5.0 POP/s dense int8 peak."""
    import torch

    from solution import kernels
    from solution.int8_mlp import ColumnScales, mlp_input_grad_int8
    from solution.quant_state import quantize_4bit

    hidden, inter = 1536, 8960
    g = torch.Generator(device=dev)
    w = []
    for s, shape in ((401, (inter, hidden)), (402, (inter, hidden)), (403, (hidden, inter))):
        g.manual_seed(s)
        packed, qs = quantize_4bit(torch.randn(*shape, generator=g, device=dev) * 0.02)
        w.append((packed.view(-1), qs))
    gate, up, down = w
    g.manual_seed(404)
    x = torch.randn(M, hidden, generator=g, device=dev).half()
    dh2 = (torch.randn(M, hidden, generator=g, device=dev) * 1e-2).half()
    gu = kernels.linear_fwd(x, [gate, up])
    d_act = torch.empty(M, inter, dtype=torch.float16, device=dev)
    dgu = torch.empty(M, 2 * inter, dtype=torch.float16, device=dev)
    dy = torch.empty(M, hidden, dtype=torch.float16, device=dev)

    def fp16_path():
        kernels.linear_dx(dh2, [down], out=d_act)
        kernels.swiglu_bwd(d_act, gu[:, :inter], gu[:, inter:], dgu[:, :inter], dgu[:, inter:])
        kernels.linear_dx(dgu, [gate, up], out=dy)

    scales = ColumnScales().get(gate, up, down)
    cs_gu, cs_d = scales
    dh8, sdh = kernels.int8_rows(dh2)
    wd8 = kernels.int8_weight_t([down], cs_d)
    acc = kernels.int8_gemm(dh8, wd8)
    q8, sq = kernels.int8_swiglu_bwd(acc, sdh, cs_d, gu)
    wgu8 = kernels.int8_weight_t([gate, up], cs_gu)
    t = {"fp16_path": _time_graph(torch, fp16_path, reps),
         "int8_path": _time_graph(torch, lambda: mlp_input_grad_int8(dh2, gu, gate, up, down,
                                                                       scales), reps),
         "int8_gemm_down": _time_graph(torch, lambda: kernels.int8_gemm(dh8, wd8), reps),
         "int8_gemm_gate_up": _time_graph(torch, lambda: kernels.int8_gemm(
             q8, wgu8, sq, cs_gu, out_dtype=torch.float16), reps),
         "int8_weights": _time_graph(torch, lambda: (kernels.int8_weight_t([down], cs_d),
                                                     kernels.int8_weight_t([gate, up], cs_gu)),
                                     reps)}
    ops = 2 * M * inter * hidden
    tops = {n: round(ops / (t[n] * 1e-3) / 1e12, 1) for n in ("int8_gemm_down", "int8_gemm_gate_up")}
    return {"int8_mlp_dx": {
        "workload": "Qwen2.5-1.5B MLP input gradient (down 1536x8960, gate|up 2x8960x1536), "
                    "M=2048, HIP graph replay; int8 = the reference's T4 int8 backward "
                    "(off the fp16 parity path, its own tolerance)",
        "us": {n: round(v * 1e3, 2) for n, v in t.items()},
        "speedup_int8_vs_fp16": round(t["fp16_path"] / t["int8_path"], 3),
        "int8_gemm_tops": tops, "peak_int8_tops": PEAK_INT8_TOPS,
        "int8_gemm_frac": {n: round(v / PEAK_INT8_TOPS, 4) for n, v in tops.items()}}}


# ------------------------------------------------- the projection's neighbours (norm, RoPE)

def norm_rope_leg(dtype, dev, reps=20):
    """RMSNorm (fp32 residual stream + o_proj output, LoRA dropout inputs with bit-packed masks)
    and RoPE forward and backward at M=2048 on the Qwen2.5-1.5B shapes (hidden 1536, 12 query heads, 2 key/value heads of 128): GB/s of
    algorithmic bytes against the 8 TB/s HBM peak, each kernel replayed 20 times in a HIP
    graph (these launches are a few microseconds each)."""
    import torch

    from solution import kernels

    h, nh, nkv, hd = 1536, 12, 2, 128
    g = torch.Generator(device=dev).manual_seed(301)
    r = lambda *s: torch.randn(*s, generator=g, device=dev).to(dtype)  # noqa: E731
    d, dy, dq, dv = (r(M, h) for _ in range(4))
    # the residual stream and its gradient in fp32, as the reference's decoder layer keeps them
    x, dres = (torch.randn(M, h, generator=g, device=dev) for _ in range(2))
    w = torch.rand(h, generator=g, device=dev) + 0.5
    keep = lambda: torch.rand(M, h, generator=g, device=dev) > 0.1  # noqa: E731
    kq, kv = keep(), keep()
    _, rstd, _, _, packed = kernels.add_rmsnorm(x, w, 1e-6, d=d, keep_q=kq, keep_v=kv)
    qkv = r(M, (nh + 2 * nkv) * hd)
    ang = torch.rand(M, hd // 2, generator=g, device=dev)
    cos, sin = torch.cat([ang.cos()] * 2, 1), torch.cat([ang.sin()] * 2, 1)
    gq, gk, gv = (r(M, nh, hd) for _ in range(3))
    e = 2  # bytes per element
    legs = {
        # mode 1: one-byte keep masks in, packed bits out; mode 2: packed bits in
        "rmsnorm_fwd": (lambda: kernels.add_rmsnorm(x, w, 1e-6, d=d, keep_q=kq, keep_v=kv,
                                                    scale_q=1.1, scale_v=1.1),
                        M * h * (4 + e + 2 + 3 * e) + M * h // 4 + M * 4 + h * 4),
        "rmsnorm_fwd_packed": (lambda: kernels.add_rmsnorm(x, w, 1e-6, d=d, packed=packed,
                                                           scale_q=1.1, scale_v=1.1),
                               M * h * (4 + e + 3 * e) + M * h // 4 + M * 4 + h * 4),
        "rmsnorm_bwd": (lambda: kernels.rmsnorm_bwd(x, w, rstd, dy=dy, d=d, dres=dres, dq=dq, dv=dv,
                                                    packed=packed),
                        M * h * (4 * e + 4 + 4 + 4) + M * h // 4 + M * 4 + h * 4),
        "rope_fwd": (lambda: kernels.qkv_rope(qkv, cos, sin, nh, nkv, hd),
                     M * ((nh + 2 * nkv) * hd * e + 2 * hd * 4 + 3 * nh * hd * e + 2 * nkv * hd * e)),
        "rope_bwd": (lambda: kernels.qkv_rope_bwd(gq, gk, gv, cos, sin, nkv),
                     M * (3 * nh * hd * e + 2 * hd * 4 + (nh + 2 * nkv) * hd * e)),
    }
    out = {}
    for name, (fn, nbytes) in legs.items():
        ms = _time_graph(torch, lambda fn=fn: [fn() for _ in range(reps)], 3) / reps
        gbps = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"us": round(ms * 1e3, 2), "gbps": round(gbps, 1),
                     "frac": round(gbps / PEAK_HBM_GBPS, 4), "bytes": nbytes}
    return {"norm_rope": dict(out, workload="RMSNorm + RoPE fwd/bwd around the q|k|v projection, "
                                           "Qwen2.5-1.5B shapes, M=2048, HIP graph replay")}


# -------------------------------------------------------------------- varlen stack (config 3)

def varlen_stack_leg(dtype, dev, steps=5, warmup=2, gemv=True, gemv_ms=(1, 8, 64)):
    """the 28-layer Qwen2.5-1.5B projection stack (7 NF4 weights per layer,
    seeds 1000 + 7 l + i) forward and backward on an unpadded batch of 4 sequences with lengths
    drawn uniformly from [64, 512] (seed 5), concatenated through cu_seqlens."""
    import torch

    from solution.stack import QWEN2_15B, ProjectionStack

    g = torch.Generator().manual_seed(5)
    lens = torch.randint(64, 513, (4,), generator=g)
    cu = torch.zeros(5, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0)
    st = ProjectionStack.synthetic(QWEN2_15B, 28, int(cu[-1]), dtype, dev, seed_base=1000,
                                   seed_stride=7, rank=RANK, alpha=ALPHA)
    m = st.set_tokens(cu)
    ms = _time_steps(torch, st.step, steps, warmup)
    fl = st.flops()["total"]
    tf = fl / (ms * 1e-3) / 1e12
    out = {"varlen_stack": {
        "workload": "28-layer Qwen2.5-1.5B projection stack fwd+bwd, varlen tokens",
        "cu_seqlens": [int(v) for v in cu], "tokens": m, "ms_per_step": round(ms, 3),
        "gflop_per_step": round(fl / 1e9, 2), "tflops": round(tf, 2),
        "frac": round(tf / PEAK_MFMA_TFLOPS, 4), "steps": steps}}
    if gemv:
        out["gemv_15b"] = gemv_sweep(st, torch, "28-layer Qwen2.5-1.5B stack, fp16", gemv_ms)
    del st
    torch.cuda.empty_cache()
    return out


# ------------------------------------------------------------ 7B bf16 and GEMV sweep (config 4)

def qwen7b_legs(dev, steps=5, warmup=2, gemv=True, layers=28, gemv_ms=(1, 8, 64)):
    """one Qwen2.5-7B layer (hidden 3584, intermediate 18944, kv 512) in
    bf16 at M = 8192, forward+backward; and the small-M dequant-GEMV regime (M in {1, 8, 64},
    forward) over the 28-layer 7B stack (3.3 GB of NF4 weights, far above the Infinity Cache),
    reported as HBM GB/s (NF4 weight bytes + activation bytes) against 8 TB/s."""
    import torch

    from solution.stack import GEMMS, QWEN2_7B, ProjectionStack

    st = ProjectionStack.synthetic(QWEN2_7B, layers if gemv else 1, 8192, torch.bfloat16, dev,
                                   seed_base=2000, seed_stride=7, rank=RANK, alpha=ALPHA)
    st.set_tokens([0, 8192])
    ev = {n: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for n in GEMMS}
    fl = st.flops()["total"] / len(st.per_layer)
    ms = _time_steps(torch, lambda: (st.forward(layers=[0]), st.backward(layers=[0])), steps,
                     warmup)
    st.forward(ev, layers=[0])
    st.backward(ev, layers=[0])
    torch.cuda.synchronize()
    per = {n: round(ev[n][0].elapsed_time(ev[n][1]) * 1e3, 1) for n in GEMMS}
    tf = fl / (ms * 1e-3) / 1e12
    out = {"qwen7b_m8192": {
        "workload": "Qwen2.5-7B decoder-layer NF4 projections fwd+bwd, bf16, M=8192",
        "ms_per_step": round(ms, 3), "gflop_per_step": round(fl / 1e9, 1),
        "tflops": round(tf, 2), "frac": round(tf / PEAK_MFMA_TFLOPS, 4),
        "gemm_us_per_launch": per}}
    if gemv:
        out["gemv_7b"] = gemv_sweep(st, torch, "28-layer Qwen2.5-7B stack, bf16", gemv_ms)
    del st
    torch.cuda.empty_cache()
    return out


def gemv_only(dev, ms_list):
    """The two small-M sweeps alone, on stacks sized for the largest M (no M=2048 / 8192
    buffers)."""
    import torch

    from solution.stack import QWEN2_7B, QWEN2_15B, ProjectionStack

    out = {}
    for leg, shape, dtype, seed, what in (
            ("gemv_15b", QWEN2_15B, torch.float16, 1000, "28-layer Qwen2.5-1.5B stack, fp16"),
            ("gemv_7b", QWEN2_7B, torch.bfloat16, 2000, "28-layer Qwen2.5-7B stack, bf16")):
        st = ProjectionStack.synthetic(shape, 28, max(ms_list), dtype, dev, seed_base=seed,
                                       seed_stride=7, rank=RANK, alpha=ALPHA)
        out[leg] = gemv_sweep(st, torch, what, ms_list)
        del st
        torch.cuda.empty_cache()
    return out


def gemv_sweep(st, torch, what, ms_list=(1, 8, 64), reps=5):
    """Forward of every layer of `st` at M tokens, captured once in a HIP graph and replayed
    (decode runs launch-bound otherwise): GB/s = (NF4 weight bytes + activations read and
    written) / replay time."""
    res = {"workload": f"forward of the {what} at M in {list(ms_list)} (decode regime), "
                       f"HIP graph replay"}
    wbytes = st.weight_bytes()
    sh, es = st.shape, st.x.element_size()
    for m in ms_list:
        st.set_tokens([0, m])
        act = len(st.per_layer) * m * es * (
            (sh.hidden + st.n_qkv) + 2 * sh.hidden + (sh.hidden + 2 * sh.inter) +
            (sh.inter + sh.hidden) + 2 * 2 * st.rank)
        ms = _time_graph(torch, st.forward, reps)
        eager = _time_steps(torch, st.forward, reps, 1)
        gbps = (wbytes + act) / (ms * 1e-3) / 1e9
        res[str(m)] = {"us_per_layer": round(ms * 1e3 / len(st.per_layer), 2),
                       "gbps": round(gbps, 1), "frac": round(gbps / PEAK_HBM_GBPS, 4),
                       "us_per_layer_eager_launches": round(eager * 1e3 / len(st.per_layer), 2)}
    res["nf4_weight_bytes"] = wbytes
    return res


# ------------------------------------------------------------------------------ dequant leg

def dequant_leg(dtype, dev, reps=5):
    """Standalone dequant over the 28-layer Qwen2.5-1.5B stack (28 x 7 weights, 3.3 GB of
    algorithmic traffic, far above the 256 MB Infinity Cache): one stacked launch per group
    (q|k|v, o, gate|up, down) as the reference's _dequant does.  Returns a dict."""
    import torch

    from solution import _lib
    from solution.quant_state import quantize_4bit, weight_desc

    lib = _lib.load()
    dt = _lib.DTYPE_CODE[dtype]
    shapes = {name: (n, k) for name, n, k in LAYER}
    groups = [["q", "k", "v"], ["o"], ["gate", "up"], ["down"]]
    grouped, batched, keep = [], [], []
    total_bytes = write_bytes = 0
    for layer in range(28):
        # every layer's weights quantized on their own (seeds 1000 + 7 layer + i): packed bytes,
        # absmax codes and absmax2 scales all distinct, the whole stack the working set
        base = {}
        for i, (name, n, k) in enumerate(LAYER):
            g = torch.Generator(device=dev).manual_seed(1000 + 7 * layer + i)
            packed, qs = quantize_4bit(torch.randn(n, k, generator=g, device=dev) * 0.02)
            base[name] = (packed.view(-1), qs)
            keep += [packed, qs]
        layer_descs, layer_outs = [], []
        for names in groups:
            descs, rows = [], 0
            for nm in names:
                p, qs = base[nm]
                descs.append(weight_desc(p, qs))
                rows += int(qs.shape[0])
            cols = shapes[names[0]][1]
            out = torch.empty((rows, cols), dtype=dtype, device=dev)
            keep.append(out)
            arr = (_lib.NF4Weight * len(descs))(*descs)
            grouped.append((arr, len(descs), out.data_ptr()))
            total_bytes += dequant_bytes(rows * cols)
            write_bytes += 2 * rows * cols
            off = 0
            for d, nm in zip(descs, names):  # the same outputs, weight by weight
                layer_descs.append(d)
                layer_outs.append(out.data_ptr() + off * out.element_size())
                off += int(base[nm][1].shape[0]) * cols
        batched.append(((_lib.NF4Weight * 7)(*layer_descs),
                        (ctypes.c_void_p * 7)(*layer_outs)))

    def run_grouped():
        s = torch.cuda.current_stream().cuda_stream
        for arr, nw, out in grouped:
            st = lib.nf4_dequant_multi(arr, nw, out, dt, s)
            if st:
                raise RuntimeError(f"nf4_dequant_multi status {st}")

    def run_batched():
        s = torch.cuda.current_stream().cuda_stream
        for arr, outs in batched:
            st = lib.nf4_dequant_batch(arr, 7, outs, dt, s)
            if st:
                raise RuntimeError(f"nf4_dequant_batch status {st}")

    # every weight of the stack in one launch through a device descriptor table
    pairs, outs = [], []
    for arr, out_ptrs in batched:
        for i in range(7):
            pairs.append(arr[i])
            outs.append(out_ptrs[i])
    nbytes = lib.nf4_dequant_table_bytes((_lib.NF4Weight * len(pairs))(*pairs), len(pairs))
    host = torch.empty(nbytes, dtype=torch.uint8)
    blocks = ctypes.c_int64(0)
    st = lib.nf4_dequant_table_pack((_lib.NF4Weight * len(pairs))(*pairs), len(pairs),
                                    (ctypes.c_void_p * len(outs))(*outs), dt, host.data_ptr(),
                                    nbytes, ctypes.byref(blocks))
    if st:
        raise RuntimeError(f"nf4_dequant_table_pack status {st}")
    table = host.to(dev)

    def run_table():
        st = lib.nf4_dequant_table(table.data_ptr(), len(pairs), blocks.value, dt,
                                   torch.cuda.current_stream().cuda_stream)
        if st:
            raise RuntimeError(f"nf4_dequant_table status {st}")

    table_ms = _time_steps(torch, run_table, max(reps, 10), 2)
    batch_ms = _time_graph(torch, run_batched, reps)
    group_ms = _time_graph(torch, run_grouped, reps)
    gbps = total_bytes / (table_ms * 1e-3) / 1e9
    # the box's own ceilings for this traffic mix: torch's fill (write only) and copy on 2 GiB
    big = torch.empty(2 << 30, dtype=torch.uint8, device=dev)
    big2 = torch.empty_like(big)
    fill_ms = _time_steps(torch, lambda: big.fill_(1), 5, 2)
    copy_ms = _time_steps(torch, lambda: big2.copy_(big), 5, 2)
    del big, big2
    return {"gbps": round(gbps, 1), "frac": round(gbps / PEAK_HBM_GBPS, 4),
            "bytes_per_pass": total_bytes, "read_bytes": total_bytes - write_bytes,
            "write_bytes": write_bytes, "us_per_pass": round(table_ms * 1e3, 1),
            "launches_per_pass": 1, "workgroups": int(blocks.value),
            "working_set": "28-layer Qwen2.5-1.5B stack (196 weights, each quantized on its own: "
                           "distinct packed bytes, absmax codes and absmax2 scales)",
            "timing": "one nf4_dequant_table launch over all 196 weights, HIP events, mean of 10",
            "gbps_per_layer_launches": round(total_bytes / (batch_ms * 1e-3) / 1e9, 1),
            "per_layer_launches": "one nf4_dequant_batch launch per layer (7 weights), 28 "
                                  "launches in a HIP graph",
            "gbps_grouped_launches": round(total_bytes / (group_ms * 1e-3) / 1e9, 1),
            "grouped": "4 nf4_dequant_multi launches per layer (q|k|v, o, gate|up, down) as the "
                       "reference's _dequant groups them",
            "box_write_gbps": round((2 << 30) / (fill_ms * 1e-3) / 1e9, 1),
            "box_copy_gbps": round(2 * (2 << 30) / (copy_ms * 1e-3) / 1e9, 1),
            "box_note": "torch fill_ (write only) and copy_ (read + write) of 2 GiB on the same "
                        "box: the dequant moves 0.52 B read + 2 B written per element, so the "
                        "write rate bounds it"}


# ---------------------------------------------------------------------------- CPU baseline

def cpu_baseline(dtype_name, reps):
    """The CPU oracle (numpy dequant + torch fp32 GEMMs on the bit-exact weight) running the
    same step on the host cores: one warm-up, then the median of `reps`."""
    import concurrent.futures as cf

    import numpy as np
    import torch

    from oracle import nf4_oracle as o

    # every host core this process may use: the cores the scheduler gives it (the GPU box
    # grants one GPU's job a share of the host, which os.cpu_count() does not show) and at most
    # the OMP_NUM_THREADS the box sets for it
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = max(1, min(avail or 1, omp if omp > 0 else (avail or 1)))
    torch.set_num_threads(threads)
    rng = np.random.default_rng(0)
    states = {}
    for i, (name, n, k) in enumerate(LAYER):
        w = np.random.default_rng(100 + i).standard_normal((n, k)).astype(np.float32) * 0.02
        states[name] = o.quantize_nf4(w)
    half = lambda *s: torch.from_numpy(rng.standard_normal(s).astype(np.float16))  # noqa: E731
    x, attn, x2, act = half(M, 1536), half(M, 1536), half(M, 1536), half(M, 8960)
    dy_qkv, dy_o, dy_gu, dy_d = (half(M, 2048) * 1e-3, half(M, 1536) * 1e-3,
                                 half(M, 17920) * 1e-3, half(M, 1536) * 1e-3)
    a_q, a_v = half(RANK, 1536) * 0.02, half(RANK, 1536) * 0.02
    b_q, b_v = half(1536, RANK) * 0.01, half(256, RANK) * 0.01
    bias = half(2048) * 0.1
    s = ALPHA / RANK
    pool = cf.ThreadPoolExecutor(max_workers=min(7, threads))

    def deq():
        futs = {nm: pool.submit(o.dequantize, p, st, dtype_name) for nm, (p, st) in
                states.items()}
        out = {}
        for nm, f in futs.items():
            w = f.result()
            out[nm] = torch.from_numpy(w.view(np.int16)).view(torch.bfloat16).float() \
                if dtype_name == "bf16" else torch.from_numpy(w).float()
        return out

    def step():
        w = deq()  # forward dequant
        wqkv = torch.cat([w["q"], w["k"], w["v"]])
        lor = [(0, 1536, x, a_q, b_q, s), (1792, 256, x, a_v, b_v, s)]
        o.linear_fwd(x, wqkv, bias, lor)
        o.linear_fwd(attn, w["o"])
        o.linear_fwd(x2, torch.cat([w["gate"], w["up"]]))
        o.linear_fwd(act, w["down"])
        w = deq()  # backward dequant
        wqkv = torch.cat([w["q"], w["k"], w["v"]])
        o.linear_dx(dy_d, w["down"])
        o.linear_dx(dy_gu, torch.cat([w["gate"], w["up"]]))
        o.linear_dx(dy_o, w["o"])
        o.linear_dx(dy_qkv, wqkv, lor)
        o.lora_grads(dy_qkv[:, :1536], x, a_q, b_q, s)
        o.lora_grads(dy_qkv[:, 1792:], x, a_v, b_v, s)

    step()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    pool.shutdown()
    sec = float(np.median(times))
    tflops = Workload.flops()["total"] / sec / 1e12
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(tflops, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": (f"the full step (M=2048, 7 projections fwd+bwd, LoRA q/v, both dequants) "
                       f"in the CPU oracle: numpy dequant (7 weights in parallel) + torch fp32 "
                       f"GEMMs, median of {reps} after 1 warm-up: {sec:.2f} s/step; "
                       f"torch threads {threads}, os.cpu_count() {os.cpu_count()}, CPU {cpu}")}


# ------------------------------------------------------------------ measured device ceilings

PROBE_LIB = ROOT / "kaggle-mltest_amd" / "probe" / "libnf4_probe.so"


def _probe_lib():
    """The bench's measurement probes (kaggle-mltest_amd/probe/nf4_probe.hip), a library of
    their own beside the NF4 one."""
    lib = ctypes.CDLL(str(PROBE_LIB))
    lib.nf4_probe_mfma.restype = ctypes.c_int
    lib.nf4_probe_mfma.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int,
                                   ctypes.c_void_p, ctypes.c_void_p]
    lib.nf4_probe_read.restype = ctypes.c_int
    lib.nf4_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                   ctypes.c_void_p, ctypes.c_void_p]
    return lib

def measured_peaks(dtype, dev):
    """What this box sustains, for fractions of measured peaks beside the data-sheet ones: the
    MFMA rate of back-to-back v_mfma_f32_32x32x16 on register operands (nf4_probe_mfma, 2048
    workgroups of 4 waves x 4 independent accumulators; operands drawn from N(0, 1), whose bit
    patterns set the power draw), the HBM read rate (nf4_probe_read over 4 GiB) and write rate
    (torch fill_ of 4 GiB).  Best of 3 timed launches each."""
    import torch

    from solution import _lib

    lib = _probe_lib()
    dt = _lib.DTYPE_CODE[dtype]
    s = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    ops = torch.randn(128 * 8, generator=torch.Generator().manual_seed(7)).to(dtype).to(dev)
    wgs, iters = 2048, 4000
    out = torch.empty(wgs * 256, dtype=torch.float32, device=dev)

    def best(fn, n=3):
        fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(n):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1))
        return min(ts)

    def mfma():
        if lib.nf4_probe_mfma(ops.data_ptr(), wgs, iters, dt, out.data_ptr(), s()):
            raise RuntimeError("nf4_probe_mfma failed")
    mfma_ms = best(mfma)
    flops = 2.0 * 32 * 32 * 16 * 4 * iters * 4 * wgs
    big = torch.empty(4 << 30, dtype=torch.uint8, device=dev)
    big.fill_(1)
    red = torch.empty(2048 * 256, dtype=torch.int32, device=dev)

    def read():
        if lib.nf4_probe_read(big.data_ptr(), big.numel(), 2048, red.data_ptr(), s()):
            raise RuntimeError("nf4_probe_read failed")
    read_ms = best(read)
    fill_ms = best(lambda: big.fill_(2))
    del big
    return {"mfma_tflops": round(flops / (mfma_ms * 1e-3) / 1e12, 1),
            "hbm_read_gbps": round((4 << 30) / (read_ms * 1e-3) / 1e9, 1),
            "hbm_write_gbps": round((4 << 30) / (fill_ms * 1e-3) / 1e9, 1),
            "how": "nf4_probe_mfma (2048 workgroups x 4 waves x 4 accumulator chains of "
                   "v_mfma_f32_32x32x16, N(0,1) operands), nf4_probe_read and torch fill_ over "
                   "4 GiB; best of 3"}


def mix_gbps(peaks, read_bytes, write_bytes):
    """The measured HBM ceiling for a kernel moving read_bytes and write_bytes: the time the
    measured read and write rates take for them, serially."""
    t = read_bytes / peaks["hbm_read_gbps"] + write_bytes / peaks["hbm_write_gbps"]
    return (read_bytes + write_bytes) / t


# ------------------------------------------------------------------------------------- main

TRAFFIC_PROFILE = ROOT / "profiles" / "gemm_traffic_m2048.md"


def measured_traffic(kernel: str, dtype_name: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary (fp16 runs, calibrated against a device copy of known size), or None."""
    if dtype_name != "f16" or not TRAFFIC_PROFILE.exists():
        return None
    for line in TRAFFIC_PROFILE.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            vals = dict(kv.split("=") for kv in line.split(":", 1)[1].split())
            return int(vals[kernel]) if kernel in vals else None
    return None


DEQUANT_TRAFFIC_PROFILE = ROOT / "profiles" / "dequant_table_traffic.md"


def measured_dequant_traffic(dtype_name: str):
    """HBM bytes per nf4_dequant_table launch over the 28-layer stack from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (fp16, calibrated against a copy of known size),
    or None."""
    if dtype_name != "f16" or not DEQUANT_TRAFFIC_PROFILE.exists():
        return None
    for line in DEQUANT_TRAFFIC_PROFILE.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            vals = dict(kv.split("=") for kv in line.split(":", 1)[1].split())
            return int(vals["dequant_table"]) if "dequant_table" in vals else None
    return None


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this path has no multi-GPU mode "
              "(run without --gpus or with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    import torch

    dev = torch.device("cuda:0")
    dtype = torch.float16 if args.dtype == "f16" else torch.bfloat16
    gemv_ms = tuple(int(v) for v in args.gemv_ms.split(","))
    if args.gemv_only:
        print(json.dumps(gemv_only(dev, gemv_ms)), flush=True)
        return
    wl = Workload(dtype, dev)
    names = ["fwd_qkv", "fwd_o", "fwd_gu", "fwd_down", "dx_down", "dx_gu", "dx_o", "dx_qkv"]
    for _ in range(args.warmup):
        wl.step()
    torch.cuda.synchronize()

    def event_pairs(keys, n):
        return [{k: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                 for k in keys} for _ in range(n)]

    # untimed pass: every GEMM bracketed by HIP events (the events themselves cost ~5 % of a
    # step), which names the dominant GEMM and gives the per-GEMM table
    prof_steps = 10
    evp = event_pairs(names, prof_steps)
    for i in range(prof_steps):
        wl.step(evp[i])
    torch.cuda.synchronize()
    per = {n: sum(e[n][0].elapsed_time(e[n][1]) for e in evp) / prof_steps for n in names}
    dom = max(per, key=per.get)

    # timed region: K steps; HIP events on the launch stream (torch's current stream) around
    # the dominant GEMM only
    evs = event_pairs([dom], args.steps)
    t0 = time.perf_counter()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(args.steps):
        wl.step(evs[i])
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end) / args.steps
    dom_ms = sum(e[dom][0].elapsed_time(e[dom][1]) for e in evs) / args.steps
    fl = Workload.flops()
    gf = wl.gemm_flops()
    value = fl["total"] / (ms * 1e-3) / 1e12
    achieved = gf[dom] / (dom_ms * 1e-3) / 1e12
    gemm_ms = sum(per.values())
    gemm_tf = sum(gf.values()) / (gemm_ms * 1e-3) / 1e12

    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": args.dtype, "data": "synthetic",
        "config": {"workload": "Qwen2.5-1.5B decoder-layer NF4 projections fwd+bwd "
                               "(q|k|v+bias+LoRA r16 on q,v; o; gate|up; down), M=2048",
                   "global_batch": 4, "seq_len": 512, "tokens": M,
                   "gflop_per_step": round(fl["total"] / 1e9, 3), "parallelism": "none (1 GPU)"},
        "mfma_peak_frac": round(value / PEAK_MFMA_TFLOPS, 4),
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2),
                     "peak": PEAK_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_MFMA_TFLOPS, 4),
                     "traffic": measured_traffic(dom, args.dtype),
                     "us_per_launch": round(dom_ms * 1e3, 2),
                     "gflop_per_launch": round(gf[dom] / 1e9, 3)},
        "gemm_us_per_launch": {n: round(v * 1e3, 2) for n, v in per.items()},
        "gemm_table": f"HIP events around every GEMM in an untimed {prof_steps}-step pass",
        "gemm_tflops_per_launch": {n: round(gf[n] / (per[n] * 1e-3) / 1e12, 1) for n in names},
        "gemm_only_tflops": round(gemm_tf, 2),
        "wall_s": round(wall, 3),
    }
    peaks = measured_peaks(dtype, dev)
    out["measured_peaks"] = peaks
    out["mfma_peak_frac_measured"] = round(value / peaks["mfma_tflops"], 4)
    out["roofline"]["peak_measured"] = peaks["mfma_tflops"]
    out["roofline"]["frac_measured"] = round(achieved / peaks["mfma_tflops"], 4)
    if not args.no_dequant:
        dq = dequant_leg(dtype, dev)
        bound = mix_gbps(peaks, dq["read_bytes"], dq["write_bytes"])
        out["dequant"] = dict(dq, roofline={"bound": "hbm", "achieved": dq["gbps"],
                                            "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                                            "frac": dq["frac"],
                                            "peak_measured": round(bound, 1),
                                            "frac_measured": round(dq["gbps"] / bound, 4),
                                            "traffic": measured_dequant_traffic(args.dtype)})
    if not args.no_swiglu:
        out.update(swiglu_leg(dtype, dev))
    if not args.no_int8 and args.dtype == "f16":
        out.update(int8_leg(dev))
    if not args.no_norm_rope:
        out.update(norm_rope_leg(dtype, dev))
    if not args.no_stack:
        out.update(varlen_stack_leg(dtype, dev, gemv=not args.no_gemv, gemv_ms=gemv_ms))
    if not args.no_7b:
        out.update(qwen7b_legs(dev, gemv=not args.no_gemv, gemv_ms=gemv_ms))
    for leg in ("gemv_15b", "gemv_7b"):  # weight streaming: bounded by the measured read rate
        for key, v in out.get(leg, {}).items():
            if isinstance(v, dict) and "gbps" in v:
                v["frac_measured"] = round(v["gbps"] / peaks["hbm_read_gbps"], 4)
    if args.copy_mib > 0:
        src = torch.empty(args.copy_mib << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        out["copy_calibration_bytes"] = src.numel()
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.dtype, args.cpu_reps)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
