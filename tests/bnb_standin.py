"""A minimal stand-in for the parts of bitsandbytes 0.50.2 that the patch surface touches, so the
routing of `patch_linear4bit`, `patch_bnb_matmul_4bit` and `patch_qwen2_mlp_recompute` can run
without bitsandbytes (absent here and on the GPU box).

What the patches read (/root/reference/solution/nf4.py:148-216, mlp.py:77-157):
  bitsandbytes.matmul_4bit(A, B, quant_state, out=None, bias=None)
  bitsandbytes.autograd._functions.matmul_4bit
  bitsandbytes.nn.Linear4bit / bitsandbytes.nn.modules.Linear4bit (one class) with
      .weight (uint8 packed bytes carrying .quant_state), .bias, .compute_dtype,
      .compute_type_is_set, .set_compute_type(x)
  bitsandbytes.nn.modules.fix_4bit_weight_quant_state_from_module(module)

The stand-in's own `Linear4bit.forward` and `matmul_4bit` play bitsandbytes' original path: they
count their calls (so a test can tell which path ran) and compute the product on the CPU from
the oracle's dequantized weight, returning it in the input's dtype on the input's device.
"""

from __future__ import annotations

import sys
import types

import torch

from oracle import nf4_oracle as o
from tests.gpu_util import to_oracle_state


class Calls:
    def __init__(self):
        self.forward = 0
        self.matmul = 0
        self.fix_state = 0


def _original_product(x, packed, quant_state, bias):
    p, st = to_oracle_state(packed, quant_state)
    w = torch.from_numpy(o.dequantize_f32(p, st))
    y = x.detach().float().cpu() @ w.t()
    if bias is not None:
        y = y + bias.detach().float().cpu()
    return y.to(x.dtype).to(x.device)


def install(monkeypatch) -> tuple[types.ModuleType, Calls]:
    """Put a fresh stand-in `bitsandbytes` into sys.modules (undone by monkeypatch) and return
    (module, call counters)."""
    calls = Calls()
    bnb = types.ModuleType("bitsandbytes")
    nn = types.ModuleType("bitsandbytes.nn")
    modules = types.ModuleType("bitsandbytes.nn.modules")
    autograd = types.ModuleType("bitsandbytes.autograd")
    functions = types.ModuleType("bitsandbytes.autograd._functions")

    class Linear4bit(torch.nn.Module):
        def __init__(self, packed, quant_state, bias=None, compute_dtype=None):
            super().__init__()
            w = torch.nn.Parameter(packed.reshape(-1, 1), requires_grad=False)
            w.quant_state = quant_state
            self.weight = w
            self.bias = bias
            self.in_features = int(quant_state.shape[1])
            self.out_features = int(quant_state.shape[0])
            self.compute_dtype = compute_dtype
            self.compute_type_is_set = compute_dtype is not None

        def set_compute_type(self, x):
            if self.compute_dtype is None:
                self.compute_dtype = x.dtype

        def forward(self, x):
            calls.forward += 1
            return _original_product(x, self.weight, self.weight.quant_state, self.bias)

    def fix_4bit_weight_quant_state_from_module(module):
        calls.fix_state += 1

    def matmul_4bit(A, B, quant_state, out=None, bias=None):
        calls.matmul += 1
        y = _original_product(A, B, quant_state, bias)
        if out is not None:
            out.copy_(y)
            return out
        return y

    modules.Linear4bit = Linear4bit
    modules.fix_4bit_weight_quant_state_from_module = fix_4bit_weight_quant_state_from_module
    nn.Linear4bit = Linear4bit
    nn.modules = modules
    functions.matmul_4bit = matmul_4bit
    autograd._functions = functions
    bnb.nn = nn
    bnb.autograd = autograd
    bnb.matmul_4bit = matmul_4bit
    for name, mod in (("bitsandbytes", bnb), ("bitsandbytes.nn", nn),
                      ("bitsandbytes.nn.modules", modules), ("bitsandbytes.autograd", autograd),
                      ("bitsandbytes.autograd._functions", functions)):
        monkeypatch.setitem(sys.modules, name, mod)
    return bnb, calls
