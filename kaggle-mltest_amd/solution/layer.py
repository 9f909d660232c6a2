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


class NF4Projection(torch.autograd.Function):
    """apply(x [M, K], bias or None, spec, A_0, B_0, A_1, B_1, ...) -> Y [M, sum rows]."""

    @staticmethod
    def forward(ctx, x, bias, spec, *lora_params):
        dtype = x.dtype
        x = _aligned_rows(x)
        structs, saved = [], []
        for ad, a, b in zip(spec.loras, lora_params[0::2], lora_params[1::2]):
            a16 = a.detach().to(dtype).contiguous()
            b16 = b.detach().to(dtype).contiguous()
            t = kernels.lora_xa(x, a16)
            structs.append(kernels.make_lora(ad.seg, a16.shape[0], ad.scale, t=t, b=b16))
            saved += [t, a16, b16]
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
        grads, structs = [], []
        for i, ad in enumerate(spec.loras):
            t, a16, b16 = saved[3 * i: 3 * i + 3]
            rows = int(spec.weights[ad.seg][1].shape[0])
            dy_s = dy[:, offs[ad.seg]: offs[ad.seg] + rows]
            if dy_s.data_ptr() % 16:
                dy_s = dy_s.contiguous()
            da = kernels.lora_da(dy_s, b16, ad.scale)
            grad_b = kernels.lora_wgrad(dy_s, t, ad.scale, transpose_out=False)
            grad_a = kernels.lora_wgrad(x, da, 1.0, transpose_out=True)
            grads += [grad_a.to(ctx.param_dtypes[2 * i]), grad_b.to(ctx.param_dtypes[2 * i + 1])]
            structs.append(kernels.make_lora(ad.seg, a16.shape[0], ad.scale, a=a16, da=da))
        dx = kernels.linear_dx(dy, spec.weights, structs) if ctx.needs_input_grad[0] else None
        dbias = kernels.bias_grad(dy) if ctx.has_bias and ctx.needs_input_grad[1] else None
        return (dx, dbias, None, *grads)


def project(x, spec: ProjectionSpec, bias=None, lora_params=()):
    """Y = NF4Projection over a [..., K] input."""
    shape = x.shape
    y = NF4Projection.apply(x.reshape(-1, shape[-1]), bias, spec, *lora_params)
    return y.view(*shape[:-1], y.shape[-1])
