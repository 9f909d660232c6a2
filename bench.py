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
the host cores as a baseline.

    python bench.py [--steps K] [--warmup W] [--dtype f16|bf16] [--no-cpu-baseline]
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
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="after timing, copy this many MiB device-to-device 3 times: the "
                         "known-size kernel that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE")
    return ap.parse_args()


# ----------------------------------------------------------------------------- workload

class Workload:
    """Weights, inputs and every output buffer of one step, plus prebuilt C-ABI arguments."""

    def __init__(self, dtype, dev):
        import torch

        from solution import _lib
        from solution.quant_state import quantize_4bit, weight_desc

        self.torch, self.dev, self.dtype = torch, dev, dtype
        self.lib = _lib.load()
        self.dt = _lib.DTYPE_CODE[dtype]
        self.W = {}
        for i, (name, n, k) in enumerate(LAYER):
            g = torch.Generator(device=dev).manual_seed(100 + i)
            w = torch.randn(n, k, generator=g, device=dev) * 0.02
            packed, qs = quantize_4bit(w)
            self.W[name] = (packed.view(-1), qs)
        del w

        def rnd(shape, seed, std=1.0):
            g = torch.Generator(device=dev).manual_seed(seed)
            return (torch.randn(shape, generator=g, device=dev) * std).to(dtype)

        H, I, QKV = 1536, 8960, 2048
        self.x = rnd((M, H), 1)            # input of q|k|v (and LoRA)
        self.attn = rnd((M, H), 11)        # input of o
        self.x2 = rnd((M, H), 12)          # input of gate|up
        self.act = rnd((M, I), 13)         # input of down
        self.bias_qkv = rnd((QKV,), 14, 0.1)
        g = torch.Generator(device=dev).manual_seed(3)
        bound = 1.0 / H ** 0.5
        self.a_q = ((torch.rand(RANK, H, generator=g, device=dev) * 2 - 1) * bound).to(dtype)
        self.a_v = ((torch.rand(RANK, H, generator=g, device=dev) * 2 - 1) * bound).to(dtype)
        g = torch.Generator(device=dev).manual_seed(4)
        self.b_q = (torch.randn(1536, RANK, generator=g, device=dev) * 0.01).to(dtype)
        self.b_v = (torch.randn(256, RANK, generator=g, device=dev) * 0.01).to(dtype)
        self.scale = ALPHA / RANK
        self.dy_qkv = rnd((M, QKV), 2, 1e-3)
        self.dy_o = rnd((M, H), 21, 1e-3)
        self.dy_gu = rnd((M, 2 * I), 22, 1e-3)
        self.dy_d = rnd((M, H), 23, 1e-3)

        e = lambda *s: torch.empty(s, dtype=dtype, device=dev)  # noqa: E731
        self.t_q, self.t_v = e(M, RANK), e(M, RANK)
        self.y_qkv, self.y_o, self.y_gu, self.y_d = e(M, QKV), e(M, H), e(M, 2 * I), e(M, H)
        self.dx_d, self.dx_gu, self.dx_o, self.dx_qkv = e(M, I), e(M, H), e(M, H), e(M, H)
        self.da_q, self.da_v = e(M, RANK), e(M, RANK)
        f = lambda *s: torch.empty(s, dtype=torch.float32, device=dev)  # noqa: E731
        self.gb_q, self.gb_v, self.ga_q, self.ga_v = f(1536, RANK), f(256, RANK), f(RANK, H), \
            f(RANK, H)

        arr = lambda names: _lib.NF4Weight * len(names)  # noqa: E731
        self.groups = {}
        for gname, names in (("qkv", ["q", "k", "v"]), ("o", ["o"]), ("gu", ["gate", "up"]),
                             ("down", ["down"])):
            descs = arr(names)(*[weight_desc(*self.W[nm]) for nm in names])
            self.groups[gname] = descs
        lib, dt = self.lib, self.dt
        self.ws = {}
        for gname, descs in self.groups.items():
            nw = len(descs)
            fb = lib.nf4_linear_fwd_workspace(M, descs, nw, dt)
            db = lib.nf4_linear_dx_workspace(M, descs, nw, dt)
            self.ws[gname] = (torch.empty(max(fb, 1), dtype=torch.uint8, device=dev), fb,
                              torch.empty(max(db, 1), dtype=torch.uint8, device=dev), db)
        wb = lib.nf4_lora_wgrad_workspace(M, 1536, RANK)
        self.wg_ws = (torch.empty(wb, dtype=torch.uint8, device=dev), wb)
        P = lambda t: t.data_ptr()  # noqa: E731
        L = _lib.NF4Lora
        self.fwd_loras = (L * 2)(L(0, RANK, self.scale, P(self.t_q), P(self.b_q), None, None),
                                 L(2, RANK, self.scale, P(self.t_v), P(self.b_v), None, None))
        self.dx_loras = (L * 2)(L(0, RANK, self.scale, None, None, P(self.a_q), P(self.da_q)),
                                L(2, RANK, self.scale, None, None, P(self.a_v), P(self.da_v)))

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
        lib, dt, s = self.lib, self.dt, self.torch.cuda.current_stream().cuda_stream
        P = lambda t: t.data_ptr()  # noqa: E731
        chk = self._chk

        def timed(name, fn):
            if ev is not None:
                ev[name][0].record()
            chk(fn(), name)
            if ev is not None:
                ev[name][1].record()

        H, I, QKV = 1536, 8960, 2048
        chk(lib.nf4_lora_xa(P(self.x), M, H, H, P(self.a_q), RANK, P(self.t_q), dt, s), "xa")
        chk(lib.nf4_lora_xa(P(self.x), M, H, H, P(self.a_v), RANK, P(self.t_v), dt, s), "xa")
        G, W = self.groups, self.ws
        timed("fwd_qkv", lambda: lib.nf4_linear_fwd(
            P(self.x), M, H, G["qkv"], 3, P(self.bias_qkv), self.fwd_loras, 2, P(self.y_qkv), QKV,
            dt, P(W["qkv"][0]), W["qkv"][1], s))
        timed("fwd_o", lambda: lib.nf4_linear_fwd(
            P(self.attn), M, H, G["o"], 1, None, None, 0, P(self.y_o), H, dt, P(W["o"][0]),
            W["o"][1], s))
        timed("fwd_gu", lambda: lib.nf4_linear_fwd(
            P(self.x2), M, H, G["gu"], 2, None, None, 0, P(self.y_gu), 2 * I, dt, P(W["gu"][0]),
            W["gu"][1], s))
        timed("fwd_down", lambda: lib.nf4_linear_fwd(
            P(self.act), M, I, G["down"], 1, None, None, 0, P(self.y_d), H, dt,
            P(W["down"][0]), W["down"][1], s))
        # backward
        timed("dx_down", lambda: lib.nf4_linear_dx(
            P(self.dy_d), M, H, G["down"], 1, None, 0, P(self.dx_d), I, 0, dt, P(W["down"][2]),
            W["down"][3], s))
        timed("dx_gu", lambda: lib.nf4_linear_dx(
            P(self.dy_gu), M, 2 * I, G["gu"], 2, None, 0, P(self.dx_gu), H, 0, dt,
            P(W["gu"][2]), W["gu"][3], s))
        timed("dx_o", lambda: lib.nf4_linear_dx(
            P(self.dy_o), M, H, G["o"], 1, None, 0, P(self.dx_o), H, 0, dt, P(W["o"][2]),
            W["o"][3], s))
        dq = self.dy_qkv
        chk(lib.nf4_lora_da(P(dq), M, 1536, QKV, P(self.b_q), RANK, self.scale, P(self.da_q),
                            dt, s), "da")
        chk(lib.nf4_lora_da(P(dq) + 1792 * dq.element_size(), M, 256, QKV, P(self.b_v), RANK,
                            self.scale, P(self.da_v), dt, s), "da")
        wg, wb = P(self.wg_ws[0]), self.wg_ws[1]
        chk(lib.nf4_lora_wgrad(P(dq), M, 1536, QKV, P(self.t_q), RANK, self.scale,
                               P(self.gb_q), 0, dt, wg, wb, s), "wgrad")
        chk(lib.nf4_lora_wgrad(P(dq) + 1792 * dq.element_size(), M, 256, QKV, P(self.t_v), RANK,
                               self.scale, P(self.gb_v), 0, dt, wg, wb, s), "wgrad")
        chk(lib.nf4_lora_wgrad(P(self.x), M, H, H, P(self.da_q), RANK, 1.0, P(self.ga_q), 1, dt,
                               wg, wb, s), "wgrad")
        chk(lib.nf4_lora_wgrad(P(self.x), M, H, H, P(self.da_v), RANK, 1.0, P(self.ga_v), 1, dt,
                               wg, wb, s), "wgrad")
        timed("dx_qkv", lambda: lib.nf4_linear_dx(
            P(dq), M, QKV, G["qkv"], 3, self.dx_loras, 2, P(self.dx_qkv), H, 0, dt,
            P(W["qkv"][2]), W["qkv"][3], s))

    def _chk(self, st, what):
        if st != 0:
            raise RuntimeError(f"{what}: status {st} ({self.lib.nf4_status_string(st).decode()})")


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
    base = {}
    for i, (name, n, k) in enumerate(LAYER):
        g = torch.Generator(device=dev).manual_seed(1000 + i)
        packed, qs = quantize_4bit(torch.randn(n, k, generator=g, device=dev) * 0.02)
        base[name] = (packed.view(-1), qs)
    groups = [["q", "k", "v"], ["o"], ["gate", "up"], ["down"]]
    launches, keep = [], []
    total_bytes = 0
    for layer in range(28):
        for names in groups:
            descs, rows = [], 0
            for nm in names:
                p, qs = base[nm]
                p2 = p.clone()  # a distinct copy per layer: the working set is the whole stack
                keep.append(p2)
                descs.append(weight_desc(p2, qs))
                rows += int(qs.shape[0])
            cols = int(base[names[0]][1].shape[1])
            out = torch.empty((rows, cols), dtype=dtype, device=dev)
            keep.append(out)
            arr = (_lib.NF4Weight * len(descs))(*descs)
            launches.append((arr, len(descs), out.data_ptr()))
            total_bytes += dequant_bytes(rows * cols)
    s = torch.cuda.current_stream().cuda_stream

    def run():
        for arr, nw, out in launches:
            st = lib.nf4_dequant_multi(arr, nw, out, dt, s)
            if st:
                raise RuntimeError(f"nf4_dequant_multi status {st}")

    run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        run()
    e1.record()
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) / 1e3 / reps
    gbps = total_bytes / sec / 1e9
    return {"gbps": round(gbps, 1), "frac": round(gbps / PEAK_HBM_GBPS, 4),
            "bytes_per_pass": total_bytes, "us_per_pass": round(sec * 1e6, 1),
            "launches_per_pass": len(launches), "working_set": "28-layer Qwen2.5-1.5B stack"}


# ---------------------------------------------------------------------------- CPU baseline

def cpu_baseline(dtype_name, reps):
    """The CPU oracle (numpy dequant + torch fp32 GEMMs on the bit-exact weight) running the
    same step on the host cores: one warm-up, then the median of `reps`."""
    import concurrent.futures as cf

    import numpy as np
    import torch

    from oracle import nf4_oracle as o

    threads = min(16, os.cpu_count() or 1)
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


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this path has no multi-GPU mode "
              "(run without --gpus or with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    import torch

    dev = torch.device("cuda:0")
    dtype = torch.float16 if args.dtype == "f16" else torch.bfloat16
    wl = Workload(dtype, dev)
    names = ["fwd_qkv", "fwd_o", "fwd_gu", "fwd_down", "dx_down", "dx_gu", "dx_o", "dx_qkv"]
    for _ in range(args.warmup):
        wl.step()
    torch.cuda.synchronize()

    # timed region: K steps, per-GEMM HIP events on the launch stream (torch's current stream)
    evs = [{n: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for n in names} for _ in range(args.steps)]
    t0 = time.perf_counter()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(args.steps):
        wl.step(evs[i])
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end) / args.steps
    per = {n: sum(e[n][0].elapsed_time(e[n][1]) for e in evs) / args.steps for n in names}
    fl = Workload.flops()
    gf = wl.gemm_flops()
    value = fl["total"] / (ms * 1e-3) / 1e12
    dom = max(per, key=per.get)
    achieved = gf[dom] / (per[dom] * 1e-3) / 1e12
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
                     "us_per_launch": round(per[dom] * 1e3, 2),
                     "gflop_per_launch": round(gf[dom] / 1e9, 3)},
        "gemm_us_per_launch": {n: round(v * 1e3, 2) for n, v in per.items()},
        "gemm_tflops_per_launch": {n: round(gf[n] / (per[n] * 1e-3) / 1e12, 1) for n in names},
        "gemm_only_tflops": round(gemm_tf, 2),
        "wall_s": round(wall, 3),
    }
    if not args.no_dequant:
        dq = dequant_leg(dtype, dev)
        out["dequant"] = dict(dq, roofline={"bound": "hbm", "achieved": dq["gbps"],
                                            "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                                            "frac": dq["frac"], "traffic": None})
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
