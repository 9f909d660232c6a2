"""The NF4 projection part of the reference's fused decoder layer, on the HIP kernels.

Mirror of the projection sites of /root/reference/solution/layer.py: `_code` (454-460),
`_dequant` (463-493: up to three weights stacked row-wise, q|k|v or gate|up), and the q|k|v
projection with its two LoRA adapters, forward (871-878) and backward (1072-1090), here one
autograd function, `NF4Projection`, over any stack of NF4 weights with LoRA adapters on any of
its segments:

    forward   Y = x W_stack^T + bias,   Y[:, seg] += s * (xd A^T) B^T
    backward  dX = dY W_stack (+ sum over adapters with xd = x of (s dY_seg B) A),
              dB = s dY_seg^T (xd A^T),  dA = (s dY_seg B)^T xd,
              d(xd) = (s dY_seg B) A       for an adapter with its own input xd

The LoRA input xd of an adapter is x itself (dropout p = 0), or its own tensor: LoRA's
dropout output, which the reference's norm kernel writes (drop_q, drop_v; layer.py:859-878)
and whose gradient its norm backward masks (layer.py:1072-1090, 135-164: dd_q = da_q A_q).
The LoRA product is folded into the same GEMM launch as the weight product (one extra rank-r
reduction slab), instead of the reference's separate mm's and fp32 add in the RoPE kernel; for
an adapter on x its down-projection t = x A^T is left to the projection call too (inside the
GEMM launch on the small-M skinny path), and its input-gradient term is folded into the dX
GEMM the same way, while an adapter with its own input gets t from its own launch and returns
d(xd) unfolded (nf4_lora_ax_multi) for the norm backward.
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


def _norm(x, d, weight, eps, dtype, drop=None):
    """(y16, 1/rms) of RMSNorm(x (+ d)) in the GEMM dtype, and with `drop` also LoRA's dropout
    outputs (layer.py:683-715, on nf4_add_rmsnorm):
      drop = (keep_q, keep_v, rows, scale_q, scale_v) -> (y16, rstd, drop_q, drop_v, packed),
        keep masks over the padded batch read at row rows[token] (rows None: the token's own
        row), packed the masks 8 per byte for the backward pass;
      drop = (packed, scale_q, scale_v) -> (y16, rstd, drop_q, drop_v).
    x is the residual stream (fp32 or the GEMM dtype), d the o_proj output or None."""
    if drop is None:
        return kernels.add_rmsnorm(x, weight, eps, d=d, dtype=dtype)
    if len(drop) == 5:
        keep_q, keep_v, rows, scale_q, scale_v = drop
        return kernels.add_rmsnorm(x, weight, eps, d=d, dtype=dtype, keep_q=keep_q,
                                   keep_v=keep_v, rows=rows, scale_q=scale_q, scale_v=scale_v)
    packed, scale_q, scale_v = drop
    return kernels.add_rmsnorm(x, weight, eps, d=d, dtype=dtype, packed=packed, scale_q=scale_q,
                               scale_v=scale_v)


def _norm_bwd(dy, dq, dv, packed, x, d, weight, rstd, dres, scale_q, scale_v):
    """dX of _norm (layer.py:718-730, on nf4_rmsnorm_bwd): the output's gradient dy plus LoRA's
    dropout branches dq, dv (the d(xd) of NF4Projection) masked with the packed keep bits and
    scaled, plus the residual gradient dres; dX in x's dtype (fp32 for the fp32 residual
    stream, as the reference's)."""
    return kernels.rmsnorm_bwd(x, weight, rstd, dy=dy, d=d, dres=dres, dq=dq, dv=dv,
                               packed=packed if dq is not None else None, scale_q=scale_q,
                               scale_v=scale_v)


@dataclass
class LoraAdapter:
    seg: int                  # index of the segment the adapter adds to
    scale: float              # alpha / r
    own_input: bool = False   # the adapter reads its own input xd (LoRA dropout) instead of x


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


def _xd_slots(spec):
    """Per entry of the flat LoRA parameter list: the adapter when the entry is its input xd,
    else None."""
    out = []
    for ad in spec.loras:
        out += [None, None] + ([ad] if ad.own_input else [])
    return out


def _adapter_params(spec, lora_params):
    """[(adapter, A, B, xd or None)] from the flat parameter list: A, B per adapter, then its
    input xd when the adapter has one."""
    out, i = [], 0
    for ad in spec.loras:
        a, b = lora_params[i], lora_params[i + 1]
        i += 2
        xd = None
        if ad.own_input:
            xd = lora_params[i]
            i += 1
        out.append((ad, a, b, xd))
    if i != len(lora_params):
        raise ValueError("LoRA parameters: A, B (and xd for an adapter with own_input) each")
    return out


class NF4Projection(torch.autograd.Function):
    """apply(x [M, K], bias or None, spec, A_0, B_0[, xd_0], A_1, B_1[, xd_1], ...) -> Y
    [M, sum rows]; xd_i ([M, K], the adapter's dropout output) when spec.loras[i].own_input."""

    @staticmethod
    def forward(ctx, x, bias, spec, *lora_params):
        dtype = x.dtype
        x = _aligned_rows(x)
        structs, saved, jobs, xd_dtypes = [], [], [], []
        for ad, a, b, xd in _adapter_params(spec, lora_params):
            a16 = a.detach().to(dtype).contiguous()
            b16 = b.detach().to(dtype).contiguous()
            xin = x
            if xd is not None:
                if tuple(xd.shape) != tuple(x.shape):
                    raise ValueError("a LoRA input has the projection input's shape")
                xd_dtypes.append(xd.dtype)
                xin = _aligned_rows(xd.detach().to(dtype))
            t = torch.empty((x.shape[0], a16.shape[0]), dtype=dtype, device=x.device)
            if xd is None:  # t = x A^T: the projection's own call computes it
                if a16.data_ptr() % 16:
                    a16 = a16.clone()
                structs.append(kernels.make_lora(ad.seg, a16.shape[0], ad.scale, t=t, b=b16, a=a16))
            else:
                jobs.append((a16.shape[0], kernels.lora_job(xin, a16, t)))
                structs.append(kernels.make_lora(ad.seg, a16.shape[0], ad.scale, t=t, b=b16))
            saved += [t, a16, b16] + ([xin] if xd is not None else [])
        _run_jobs(kernels.lora_xa_multi, jobs, x)  # t = xd A^T for the adapters with own input
        b = None if bias is None else bias.detach().to(dtype).contiguous()
        y = kernels.linear_fwd(x, spec.weights, b, structs)
        ctx.spec = spec
        ctx.has_bias = bias is not None
        ctx.param_dtypes = [p.dtype for p in lora_params]
        ctx.xd_dtypes = xd_dtypes
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
        structs, da_jobs, wg_jobs, ax_jobs, per_ad, live = [], [], [], [], [], []
        k = 0
        for ad in spec.loras:
            t, a16, b16 = saved[k: k + 3]
            k += 3
            xin = x
            if ad.own_input:
                xin = saved[k]
                k += 1
            r = a16.shape[0]
            rows = int(spec.weights[ad.seg][1].shape[0])
            dy_s = dy[:, offs[ad.seg]: offs[ad.seg] + rows]
            if dy_s.data_ptr() % 16:
                dy_s = dy_s.contiguous()  # a copy only the job structs point to
            da = torch.empty((x.shape[0], r), dtype=x.dtype, device=x.device)
            live += [dy_s, da]
            grad_b = torch.empty((rows, r), dtype=torch.float32, device=x.device)
            grad_a = torch.empty((r, x.shape[1]), dtype=torch.float32, device=x.device)
            da_jobs.append((r, kernels.lora_job(dy_s, b16, da, ad.scale)))
            wg_jobs += [(r, kernels.lora_job(dy_s, t, grad_b, ad.scale)),
                        (r, kernels.lora_job(xin, da, grad_a, 1.0, transpose_out=True))]
            dxd = None
            if ad.own_input:
                dxd = torch.empty_like(xin)
                ax_jobs.append((r, kernels.lora_ax_job(da, a16, dxd)))
            else:
                structs.append(kernels.make_lora(ad.seg, r, ad.scale, a=a16, da=da))
            per_ad.append((grad_a, grad_b, dxd))
        _run_jobs(kernels.lora_da_multi, da_jobs, x)         # da = s dY_seg B
        _run_jobs(kernels.lora_wgrad_multi, wg_jobs, x)      # dB = s dY_seg^T t, dA = da^T xd
        _run_jobs(kernels.lora_ax_multi, ax_jobs, x)         # d(xd) = da A (own inputs)
        grads, p, q = [], 0, 0
        for ad, (grad_a, grad_b, dxd) in zip(spec.loras, per_ad):
            grads += [grad_a.to(ctx.param_dtypes[p]), grad_b.to(ctx.param_dtypes[p + 1])]
            p += 2
            if ad.own_input:
                grads.append(dxd.to(ctx.xd_dtypes[q]))
                p += 1
                q += 1
        dx = kernels.linear_dx(dy, spec.weights, structs) if ctx.needs_input_grad[0] else None
        dbias = kernels.bias_grad(dy) if ctx.has_bias and ctx.needs_input_grad[1] else None
        return (dx, dbias, None, *grads)


def project(x, spec: ProjectionSpec, bias=None, lora_params=()):
    """Y = NF4Projection over a [..., K] input (the adapters' own inputs [..., K] too)."""
    shape = x.shape
    flat = [t.reshape(-1, shape[-1]) if a is not None else t
            for t, a in zip(lora_params, _xd_slots(spec))]
    y = NF4Projection.apply(x.reshape(-1, shape[-1]), bias, spec, *flat)
    return y.view(*shape[:-1], y.shape[-1])
