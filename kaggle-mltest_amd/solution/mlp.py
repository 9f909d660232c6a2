"""Qwen2 MLP that keeps only its input for the backward pass and recomputes gate|up there,
on the HIP kernels.  Mirror of /root/reference/solution/mlp.py (`RecomputedMLP`, 42-74, same
apply() signature; `patch_qwen2_mlp_recompute`, 123-157).

gate and up run as ONE dequant-GEMM launch over the pair with the SwiGLU step in its epilogue
(nf4_linear_swiglu_fwd: the [M, 2I] gate|up product never reaches memory); the backward
recomputes them the same way with the SwiGLU gradient in the epilogue (nf4_linear_swiglu_bwd),
and the input gradient dgate W_gate + dup W_up is ONE transposed dequant-GEMM over the stacked
pair, summed in fp32 (the reference adds two fp16 products).  Below FUSED_MIN_TOKENS rows
(decode) the unfused sequence runs: the stacked small-M GEMM, then the SwiGLU kernels.
The reference's recompute budget (mlp.py:92-120) is a 15 GB-GPU memory policy and is not
mirrored: this MLP always recomputes.

`INT8_BACKWARD` (off by default, as RecomputedMLP's backward is fp16 in the reference) routes the
input gradient through the int8 GEMMs of `int8_mlp` instead, the way the reference's fused
decoder layer runs its MLP backward on the T4 (layer.py:530-534, 992-1013).  `INT8_FORWARD` (off
by default, as in the reference, layer.py:531-533) computes gate|up in the forward through one
int8 GEMM and the SwiGLU step (layer.py:900-912); the backward still recomputes gate|up in the
GEMM dtype, as the reference's recomputing layers do (layer.py:986-990).
"""

from __future__ import annotations

import torch

from . import _lib, kernels
from .quant_state import nf4_state_ok

# int8 input gradients (int8_mlp.mlp_input_grad_int8) in RecomputedMLP.backward
INT8_BACKWARD = False
# int8 gate|up product (int8_mlp.gate_up_fwd_int8) in RecomputedMLP.forward
INT8_FORWARD = False


# Token count from which the gate|up GEMM carries the SwiGLU epilogue (its tiles are the large
# forward tiles; the decode-size GEMM paths keep the separate SwiGLU step).
FUSED_MIN_TOKENS = 65


class RecomputedMLP(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, gate_w, gate_qs, up_w, up_qs, down_w, down_qs):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        if x2.stride(0) % 8 or x2.data_ptr() % 16:
            x2 = x2.contiguous()
        gate_w, up_w, down_w = gate_w.reshape(-1), up_w.reshape(-1), down_w.reshape(-1)
        inter = int(gate_qs.shape[0])
        if INT8_FORWARD and _int8_ok(gate_qs, down_qs):
            from .int8_mlp import gate_up_fwd_int8

            gu, hidden = gate_up_fwd_int8(x2, (gate_w, gate_qs), (up_w, up_qs))
            del gu
        elif x2.shape[0] >= FUSED_MIN_TOKENS:
            hidden = kernels.linear_swiglu_fwd(x2, (gate_w, gate_qs), (up_w, up_qs))
        else:
            gu = kernels.linear_fwd(x2, [(gate_w, gate_qs), (up_w, up_qs)])
            hidden = kernels.swiglu_fwd(gu[:, :inter], gu[:, inter:])
            del gu
        out = kernels.linear_fwd(hidden, [(down_w, down_qs)])
        ctx.save_for_backward(x2, gate_w, up_w, down_w)
        ctx.qs, ctx.shape = (gate_qs, up_qs, down_qs), shape
        return out.view(*shape[:-1], out.shape[-1])

    @staticmethod
    def backward(ctx, grad):
        x2, gate_w, up_w, down_w = ctx.saved_tensors
        gate_qs, up_qs, down_qs = ctx.qs
        inter = int(gate_qs.shape[0])
        grad = grad.reshape(-1, grad.shape[-1]).to(x2.dtype)
        if grad.stride(0) % 8 or grad.data_ptr() % 16:
            grad = grad.contiguous()
        if INT8_BACKWARD and _int8_ok(gate_qs, down_qs):
            from .int8_mlp import mlp_input_grad_int8

            gate, up, down = (gate_w, gate_qs), (up_w, up_qs), (down_w, down_qs)
            gu = kernels.linear_fwd(x2, [gate, up])
            dx = mlp_input_grad_int8(grad, gu, gate, up, down,
                                     scales=_SCALES.get(gate, up, down, x2.dtype))
            return dx.view(ctx.shape), None, None, None, None, None, None
        d_hidden = kernels.linear_dx(grad, [(down_w, down_qs)])
        if x2.shape[0] >= FUSED_MIN_TOKENS:
            gu = kernels.linear_swiglu_bwd(x2, (gate_w, gate_qs), (up_w, up_qs), d_hidden)
        else:
            gu = kernels.linear_fwd(x2, [(gate_w, gate_qs), (up_w, up_qs)])
            # the gradient of gate|up overwrites gate|up (each element is read, then written)
            kernels.swiglu_bwd(d_hidden, gu[:, :inter], gu[:, inter:], gu[:, :inter],
                               gu[:, inter:])
        del d_hidden
        dx = kernels.linear_dx(gu, [(gate_w, gate_qs), (up_w, up_qs)])
        return dx.view(ctx.shape), None, None, None, None, None, None


def _int8_ok(gate_qs, down_qs) -> bool:
    from .int8_mlp import int8_eligible

    return int8_eligible(int(gate_qs.shape[1]), int(gate_qs.shape[0]), int(gate_qs.blocksize)) \
        and int(down_qs.blocksize) <= 128 and 128 % int(down_qs.blocksize) == 0


class _Scales:
    """The int8 column scales of each MLP, made once per weight triple (the weights are
    frozen; the reference caches them per module for the run, layer.py:598-615)."""

    def __init__(self):
        self._cols = None

    def get(self, gate, up, down, dtype):
        if self._cols is None:
            from .int8_mlp import ColumnScales

            self._cols = ColumnScales()
        return self._cols.get(gate, up, down, dtype)


_SCALES = _Scales()


def _usable(layer, in_features):
    """A frozen bias-free NF4 bitsandbytes layer (mlp.py:77-89)."""
    from bitsandbytes.nn import Linear4bit

    if type(layer) is not Linear4bit or layer.bias is not None or layer.weight.requires_grad:
        return False
    qs = getattr(layer.weight, "quant_state", None)
    return nf4_state_ok(layer.weight, qs, in_features) and int(qs.blocksize) % 64 == 0 and \
        int(qs.shape[1]) % int(qs.blocksize) == 0


def patch_qwen2_mlp_recompute():
    """Qwen2MLP.forward through RecomputedMLP under fp16 autocast (mlp.py:123-157).  Needs
    bitsandbytes (the layers it serves are Linear4bit) and a loadable libnf4_mi355x.so; raises
    without either (apply() logs that and leaves Qwen2MLP.forward as it was)."""
    import bitsandbytes  # noqa: F401 - the layers this patch serves are bitsandbytes layers
    from transformers.models.qwen2 import modeling_qwen2

    _lib.load()

    cls = modeling_qwen2.Qwen2MLP
    if getattr(cls.forward, "_nf4_recompute", False):
        return
    previous = cls.forward

    def forward(self, x):
        if not x.is_cuda or not torch.is_autocast_enabled("cuda") or \
                torch.get_autocast_dtype("cuda") not in kernels.GEMM_DTYPES or \
                getattr(getattr(self, "config", None), "hidden_act", "silu") != "silu" or \
                not torch.is_grad_enabled() or \
                x.dtype not in (torch.float16, torch.bfloat16, torch.float32) or x.numel() == 0:
            return previous(self, x)
        if not _usable(self.gate_proj, x.shape[-1]) or not _usable(self.up_proj, x.shape[-1]) or \
                not _usable(self.down_proj, self.gate_proj.out_features):
            return previous(self, x)
        dtype = torch.get_autocast_dtype("cuda")
        half = getattr(x, "_soup_half", None)
        if half is None or half.dtype != dtype or half.shape != x.shape:
            half = x.to(dtype)
        for layer in (self.gate_proj, self.up_proj, self.down_proj):
            if not layer.compute_type_is_set:
                layer.set_compute_type(x)
                layer.compute_type_is_set = True
        return RecomputedMLP.apply(
            half, self.gate_proj.weight.view(-1), self.gate_proj.weight.quant_state,
            self.up_proj.weight.view(-1), self.up_proj.weight.quant_state,
            self.down_proj.weight.view(-1), self.down_proj.weight.quant_state)

    forward._nf4_recompute = True
    cls.forward = forward
