"""NF4 dequantization and the 4-bit linear layer on the gfx950 HIP kernels.

Mirror of /root/reference/solution/nf4.py: the same names and signatures (`dequantize_nf4`,
`NF4Linear`, `patch_linear4bit`, `patch_bnb_matmul_4bit`, `_supported`, `_nf4_state_ok`,
`_gemm_dtype`, `_base_uses_fused_kernel_for`), the same routing rules, and the same fall-back to
bitsandbytes' original function for anything this path does not cover.  Underneath, the
reference's Triton dequant + cuBLAS GEMM becomes one fused dequant-GEMM launch
(`nf4_linear_fwd` / `nf4_linear_dx` in libnf4_mi355x.so): the fp16 weight is never written
to HBM.

Differences from the reference, by design:
* the double-quantized absmax is rebuilt inside the kernels from the uint8 codes (no cached
  fp32 absmax, nf4.py:41-55), bit for bit the same value;
* fp16 and bf16 GEMMs are one fused launch; an fp32 GEMM (the reference's path when neither
  autocast nor a half compute dtype is set) dequantizes to fp32 with the HIP kernel and
  multiplies with torch's fp32 GEMM, as the reference's NF4Linear does in fp32;
* a library that cannot be loaded, or an error status from it, sends the call to
  bitsandbytes' original function instead of raising (the reference's patches never raise:
  __init__.py:49-53, nf4.py:172-181).
"""

from __future__ import annotations

import torch

from . import _lib, kernels
from ._lib import NF4LibraryError
from .quant_state import nf4_state_ok

DEQUANT_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
LINEAR_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _gemm_rows(t):
    """t [M, C] as the fused GEMMs read their activations: unit column stride, a row stride
    that is a multiple of 8 elements and a 16-byte aligned start.  Anything else is copied
    into a fresh [M, C rounded up to 8] buffer (zero padding) and returned as its [M, C] view,
    so an output width that is not a multiple of 8 (e.g. 100) still has an input gradient."""
    if t.stride(-1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0:
        return t
    m, c = t.shape
    c8 = -(-c // 8) * 8
    buf = t.new_zeros((m, c8)) if c8 != c else t.new_empty((m, c8))
    buf[:, :c] = t
    return buf[:, :c]


def dequantize_nf4(packed, quant_state, dtype=torch.float16):
    """The [N, K] weight of a 4-bit NF4 layer in `dtype` (nf4.py:69-77)."""
    if dtype not in DEQUANT_DTYPES:
        raise TypeError(f"cannot dequantize to {dtype}")
    return kernels.dequant([(packed.reshape(-1), quant_state)], dtype).view(
        tuple(quant_state.shape))


class NF4Linear(torch.autograd.Function):
    """`x @ dequant(W).T + bias`, forward and backward, with the weight dequantized inside the
    GEMM main loop.  Like the reference (nf4.py:80-102) only the packed weight is kept for the
    backward pass; the weight gets no gradient."""

    @staticmethod
    def forward(ctx, x, packed, quant_state, bias):
        if x.dtype not in LINEAR_DTYPES:
            raise TypeError(f"NF4Linear computes in fp16, bf16 or fp32, got {x.dtype}")
        shape = x.shape
        packed = packed.reshape(-1)
        if x.dtype == torch.float32:
            # fp32: the weight dequantized to fp32 by the HIP kernel, torch's fp32 GEMM
            # (nf4.py:86-87 with x in fp32)
            w = dequantize_nf4(packed, quant_state, torch.float32)
            out = torch.nn.functional.linear(x, w, None if bias is None else bias.float())
        else:
            x2 = _gemm_rows(x.reshape(-1, shape[-1]))
            b = None if bias is None else bias.to(x.dtype).contiguous()
            out = kernels.linear_fwd(x2, [(packed, quant_state)], b)
            out = out.view(*shape[:-1], out.shape[-1])
        ctx.quant_state = quant_state
        ctx.has_bias_grad = bias is not None and ctx.needs_input_grad[3]
        ctx.bias_dtype = None if bias is None else bias.dtype
        ctx.save_for_backward(packed)
        return out

    @staticmethod
    def backward(ctx, grad):
        (packed,) = ctx.saved_tensors
        grad_x = grad_bias = None
        g2 = grad.reshape(-1, grad.shape[-1])
        if grad.dtype == torch.float32:
            if ctx.needs_input_grad[0]:
                w = dequantize_nf4(packed, ctx.quant_state, torch.float32)
                grad_x = torch.matmul(grad, w)
            if ctx.has_bias_grad:
                grad_bias = g2.sum(0).to(ctx.bias_dtype)
            return grad_x, None, None, grad_bias
        g2 = _gemm_rows(g2)
        if ctx.needs_input_grad[0]:
            dx = kernels.linear_dx(g2, [(packed, ctx.quant_state)])
            grad_x = dx.view(*grad.shape[:-1], dx.shape[-1])
        if ctx.has_bias_grad:
            grad_bias = kernels.bias_grad(g2).to(ctx.bias_dtype)
        return grad_x, None, None, grad_bias


def _base_uses_fused_kernel_for(m, k, quant_state, dtype, device_index):
    """True where bitsandbytes' own backend would run its fused small-batch 4-bit GEMM
    (nf4.py:105-118); there the reference keeps bitsandbytes' numerics."""
    try:
        from bitsandbytes.backends.cuda import ops as cuda_ops
    except Exception:  # noqa: BLE001 - no such backend: nothing to defer to
        return False
    n = quant_state.shape[0]
    try:
        if m > cuda_ops._gemm_4bit_custom_max_m or k % quant_state.blocksize != 0:
            return False
        return bool(cuda_ops._gemm_4bit_use_custom_fn(device_index, dtype, m, n, k))
    except Exception:  # noqa: BLE001 - a different bitsandbytes: be conservative
        return True


def _base_uses_fused_kernel(x, quant_state, dtype=None):
    k = x.shape[-1]
    return _base_uses_fused_kernel_for(x.numel() // k, k, quant_state, dtype or x.dtype,
                                       x.device.index)


def _nf4_state_ok(packed, quant_state, in_features):
    return nf4_state_ok(packed, quant_state, in_features)


def _fused_ok(quant_state) -> bool:
    """The layouts the fused GEMM covers: each 64-wide step of a weight row inside one absmax
    block (a power-of-two blocksize >= 64 dividing in_features; a power-of-two double-quant
    group when nested).  bitsandbytes writes powers of two only."""
    bs, k = int(quant_state.blocksize), int(quant_state.shape[1])
    if bs < 64 or bs & (bs - 1) or k % bs:
        return False
    inner = getattr(quant_state, "state2", None)
    if getattr(quant_state, "nested", False) and inner is not None:
        bs2 = int(inner.blocksize)
        return bs2 > 0 and not bs2 & (bs2 - 1)
    return True


def _supported(x, packed, quant_state):
    """nf4.py:134-137 (fp16 / fp32 inputs), plus bf16."""
    return (x.is_cuda and x.numel() > 0 and x.dtype in LINEAR_DTYPES
            and _nf4_state_ok(packed, quant_state, x.shape[-1]))


def _routable(gemm_dtype, quant_state) -> bool:
    """Whether this path runs a GEMM in `gemm_dtype` on this weight: fp16 / bf16 through the
    fused kernels (the layouts `_fused_ok` covers), fp32 through the dequant kernel and torch's
    fp32 GEMM (any even blocksize)."""
    if gemm_dtype == torch.float32:
        return True
    return gemm_dtype in kernels.GEMM_DTYPES and _fused_ok(quant_state)


def _gemm_dtype(module, x):
    """The dtype the base run's GEMM runs in: autocast's when it is on, the layer's compute
    dtype otherwise (nf4.py:140-145)."""
    if torch.is_autocast_enabled(x.device.type):
        return torch.get_autocast_dtype(x.device.type)
    return module.compute_dtype or x.dtype


def patch_linear4bit():
    """Linear4bit.forward through NF4Linear (nf4.py:148-195).  Needs bitsandbytes and a
    loadable libnf4_mi355x.so; raises without either (apply() logs that and goes on, leaving
    bitsandbytes' forward in place)."""
    from bitsandbytes.nn import modules as bnb_modules

    _lib.load()
    cls = bnb_modules.Linear4bit
    if getattr(cls.forward, "_nf4_patched", False):
        return
    original = cls.forward
    fix_state = bnb_modules.fix_4bit_weight_quant_state_from_module

    def forward(self, x):
        if type(self) is not cls and type(self).forward is not forward:
            return original(self, x)
        fix_state(self)
        quant_state = self.weight.quant_state
        if not x.is_cuda or not _supported(x, self.weight, quant_state):
            return original(self, x)
        if not self.compute_type_is_set:
            self.set_compute_type(x)
            self.compute_type_is_set = True
        gemm_dtype = _gemm_dtype(self, x)
        base_dtype = self.compute_dtype or x.dtype
        if not _routable(gemm_dtype, quant_state) or \
                _base_uses_fused_kernel(x, quant_state, base_dtype):
            return original(self, x)
        half = getattr(x, "_soup_half", None)
        xg = half if half is not None and half.dtype == gemm_dtype and half.shape == x.shape \
            else x.to(gemm_dtype)
        bias = self.bias
        if bias is not None:
            if bias.dtype != base_dtype:  # as Linear4bit.forward does to its bias
                bias.data = bias.data.to(base_dtype)
            bias = bias.to(gemm_dtype)
        try:
            return NF4Linear.apply(xg, self.weight.view(-1), quant_state, bias)
        except NF4LibraryError:  # unsupported layout or a HIP error: bitsandbytes' path
            return original(self, x)

    forward._nf4_patched = True
    cls.forward = forward


def patch_bnb_matmul_4bit():
    """bitsandbytes.matmul_4bit through NF4Linear (nf4.py:198-216).  Needs bitsandbytes and a
    loadable libnf4_mi355x.so."""
    import bitsandbytes
    from bitsandbytes.autograd import _functions as bnb_autograd

    _lib.load()
    if getattr(bitsandbytes.matmul_4bit, "_nf4_patched", False):
        return
    original = bitsandbytes.matmul_4bit

    def matmul_4bit(A, B, quant_state, out=None, bias=None):
        if out is not None or not _supported(A, B, quant_state) or \
                not _routable(A.dtype, quant_state) or _base_uses_fused_kernel(A, quant_state):
            return original(A, B, quant_state, out=out, bias=bias)
        try:
            return NF4Linear.apply(A, B.view(-1), quant_state, bias)
        except NF4LibraryError:  # unsupported layout or a HIP error: bitsandbytes' path
            return original(A, B, quant_state, out=out, bias=bias)

    matmul_4bit._nf4_patched = True
    bitsandbytes.matmul_4bit = matmul_4bit
    bnb_autograd.matmul_4bit = matmul_4bit
