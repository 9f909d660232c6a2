"""The NF4 projection part of the reference's fused decoder layer, on the HIP kernels.

Mirror of the projection sites of /root/reference/solution/layer.py: `_code` (454-460),
`_dequant` (463-493: up to three weights stacked row-wise, q|k|v or gate|up), and the q|k|v
projection with its two LoRA adapters, forward (871-878) and backward (1072-1090), here one
autograd function, `NF4Projection`, over any stack of NF4 weights with LoRA adapters on any of
its segments:

    forward   Y = x W_stack^T + bias,   Y[:, seg] += s * (x A^T) B^T
    backward  dX = dY W_stack + sum_seg (s dY_seg B) A,
              dB = s dY_seg^T (x A^T),  dA = (s dY_seg B)^T x

The LoRA product is folded into the same GEMM launch as the weight product (one extra rank-r
reduction slab), instead of the reference's separate mm's and fp32 add in the RoPE kernel.
LoRA dropout is taken as p = 0 (the LoRA input is x itself).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import kernels

_CODE: dict = {}


def _code(quant_state):
    """The NF4 code table as fp32 on the weight's device, one copy per table (layer.py:454-460)."""
    code = quant_state.code
    key = (code.device, code.data_ptr())
    if key not in _CODE:
        _CODE[key] = code.to(torch.float32).contiguous()
    return _CODE[key]


def _pairs(layers):
    """[(packed uint8 flat, quant_state)] of layers (objects with .weight.quant_state) or of
    (packed, quant_state) pairs."""
    out = []
    for layer in layers:
        if isinstance(layer, tuple):
            out.append((layer[0].reshape(-1), layer[1]))
        else:
            out.append((layer.weight.reshape(-1), layer.weight.quant_state))
    return out


def _dequant(layers, dtype, streamed=None):
    """The stacked weights of up to eight NF4 layers ([sum of out_features, in_features]) in
    one launch (layer.py:463-493).  `streamed` is accepted for signature parity and must be
    None: weights stay resident in HBM here."""
    if streamed is not None:
        raise ValueError("host-streamed weights are not part of this path")
    return kernels.dequant(_pairs(layers), dtype)


@dataclass
class LoraAdapter:
    seg: int                  # index of the segment the adapter adds to
    scale: float              # alpha / r


@dataclass
class ProjectionSpec:
    weights: list             # [(packed, quant_state)] stacked along the output dim
    loras: list = field(default_factory=list)   # [LoraAdapter]

    def offsets(self):
        offs, o = [], 0
        for _, qs in self.weights:
            offs.append(o)
            o += int(qs.shape[0])
        return offs


def _aligned_rows(t: torch.Tensor) -> torch.Tensor:
    if t.stride(-1) != 1 or t.stride(0) % 8 or t.data_ptr() % 16:
        return t.contiguous()
    return t


def _run_jobs(fn, jobs, like):
    """Run (rank, nf4_lora_job) jobs through a multi launch, grouped by rank, at most 4 per
    launch (one launch for the q and v adapters of a layer)."""
    by_rank = {}
    for r, j in jobs:
        by_rank.setdefault(r, []).append(j)
    for r, js in by_rank.items():
        for k in range(0, len(js), 4):
            fn(js[k:k + 4], like.shape[0], r, like.dtype, like)


class NF4Projection(torch.autograd.Function):
    """apply(x [M, K], bias or None, spec, A_0, B_0, A_1, B_1, ...) -> Y [M, sum rows]."""

    @staticmethod
    def forward(ctx, x, bias, spec, *lora_params):
        dtype = x.dtype
        x = _aligned_rows(x)
        structs, saved, jobs = [], [], []
        for ad, a, b in zip(spec.loras, lora_params[0::2], lora_params[1::2]):
            a16 = a.detach().to(dtype).contiguous()
            b16 = b.detach().to(dtype).contiguous()
            t = torch.empty((x.shape[0], a16.shape[0]), dtype=dtype, device=x.device)
            jobs.append((a16.shape[0], kernels.lora_job(x, a16, t)))
            structs.append(kernels.make_lora(ad.seg, a16.shape[0], ad.scale, t=t, b=b16))
            saved += [t, a16, b16]
        _run_jobs(kernels.lora_xa_multi, jobs, x)  # t = x A^T for every adapter
        b = None if bias is None else bias.detach().to(dtype).contiguous()
        y = kernels.linear_fwd(x, spec.weights, b, structs)
        ctx.spec = spec
        ctx.has_bias = bias is not None
        ctx.param_dtypes = [p.dtype for p in lora_params]
        ctx.save_for_backward(x, *saved)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, *saved = ctx.saved_tensors
        spec = ctx.spec
        dy = _aligned_rows(dy.to(x.dtype))
        offs = spec.offsets()
        # `live` holds every tensor the launches below reach only through raw pointers in
        # their argument structs, until the last launch is queued: a tensor freed earlier
        # goes back to torch's allocator, which may hand its memory to the next allocation
        # while a queued kernel still reads it
        grads, structs, da_jobs, wg_jobs, pairs, live = [], [], [], [], [], []
        for i, ad in enumerate(spec.loras):
            t, a16, b16 = saved[3 * i: 3 * i + 3]
            r = a16.shape[0]
            rows = int(spec.weights[ad.seg][1].shape[0])
            dy_s = dy[:, offs[ad.seg]: offs[ad.seg] + rows]
            if dy_s.data_ptr() % 16:
                dy_s = dy_s.contiguous()
            da = torch.empty((x.shape[0], r), dtype=x.dtype, device=x.device)
            live.append(da)
            grad_b = torch.empty((rows, r), dtype=torch.float32, device=x.device)
            grad_a = torch.empty((r, x.shape[1]), dtype=torch.float32, device=x.device)
            da_jobs.append((r, kernels.lora_job(dy_s, b16, da, ad.scale)))
            wg_jobs += [(r, kernels.lora_job(dy_s, t, grad_b, ad.scale)),
                        (r, kernels.lora_job(x, da, grad_a, 1.0, transpose_out=True))]
            pairs.append((grad_a, grad_b, dy_s))
            structs.append(kernels.make_lora(ad.seg, r, ad.scale, a=a16, da=da))
        _run_jobs(kernels.lora_da_multi, da_jobs, x)         # da = s dY_seg B
        _run_jobs(kernels.lora_wgrad_multi, wg_jobs, x)      # dB = s dY_seg^T t, dA = da^T x
        for i, (grad_a, grad_b, _) in enumerate(pairs):
            grads += [grad_a.to(ctx.param_dtypes[2 * i]), grad_b.to(ctx.param_dtypes[2 * i + 1])]
        dx = kernels.linear_dx(dy, spec.weights, structs) if ctx.needs_input_grad[0] else None
        dbias = kernels.bias_grad(dy) if ctx.has_bias and ctx.needs_input_grad[1] else None
        return (dx, dbias, None, *grads)


def project(x, spec: ProjectionSpec, bias=None, lora_params=()):
    """Y = NF4Projection over a [..., K] input."""
    shape = x.shape
    y = NF4Projection.apply(x.reshape(-1, shape[-1]), bias, spec, *lora_params)
    return y.view(*shape[:-1], y.shape[-1])
