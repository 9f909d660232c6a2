"""bitsandbytes-layout NF4 weights: the QuantState container, a quantizer, and the C-ABI
weight descriptor.

`QuantState` carries the attribute names bitsandbytes 0.50.2 uses and the reference reads
(/root/reference/solution/nf4.py:46-53, 112-131; layer.py:456, 468-469), so a real bitsandbytes
QuantState and this one are interchangeable for every function of this package.

`quantize_4bit` follows bitsandbytes' `quantize_4bit(A, blocksize=64, compress_statistics=True,
quant_type="nf4")`: per block of `blocksize` elements the absmax, values scaled by its fp32
reciprocal and mapped to the nearest NF4 code (high nibble first); with compress_statistics the
absmax is double-quantized - its mean subtracted (`offset`), then 8-bit block-wise quantization
with one fp32 scale per 256 blocks on the dynamic map.  It runs on whatever device `A` is on.
"""

from __future__ import annotations

import ctypes
import math

import torch

from ._lib import NF4Weight

# QLoRA's NormalFloat4 table (bitsandbytes get_4bit_type("nf4")), fp32.
NF4_CODE = (
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0)


def dynamic_map(max_exponent_bits: int = 7, total_bits: int = 8) -> torch.Tensor:
    """The signed 8-bit dynamic map of block-wise quantization (Dettmers et al. 2022): per
    decade i the midpoints of linspace(0.1, 1, 2**i + 1) times 10**(i - 6), both signs, plus 0
    and 1; sorted, fp32, 256 entries."""
    values: list[float] = []
    for i in range(max_exponent_bits):
        count = 2 ** (i + total_bits - 1 - max_exponent_bits) + 1
        bounds = torch.linspace(0.1, 1, count, dtype=torch.float32)
        means = (bounds[:-1] + bounds[1:]) / 2.0
        scale = 10.0 ** (i - (max_exponent_bits - 1))
        values += (scale * means).tolist() + (-scale * means).tolist()
    values += [0.0, 1.0]
    values += [0.0] * (2 ** total_bits - len(values))
    return torch.tensor(sorted(values), dtype=torch.float32)


class QuantState:
    """What bitsandbytes keeps next to a packed 4-bit weight."""

    def __init__(self, absmax, shape=None, code=None, blocksize=None, quant_type=None,
                 dtype=None, offset=None, state2=None):
        self.absmax = absmax
        self.shape = shape
        self.code = code
        self.blocksize = blocksize
        self.quant_type = quant_type
        self.dtype = dtype
        self.offset = offset
        self.state2 = state2
        self.nested = state2 is not None

    def to(self, device):
        self.absmax = self.absmax.to(device)
        self.code = self.code.to(device)
        if self.nested:
            self.offset = self.offset.to(device)
            self.state2.absmax = self.state2.absmax.to(device)
            self.state2.code = self.state2.code.to(device)
        for attr in ("_nf4_desc", "_nf4_refs"):
            if hasattr(self, attr):
                delattr(self, attr)
        return self


def _nearest(x: torch.Tensor, code: torch.Tensor) -> torch.Tensor:
    """Index of the nearest entry of the sorted `code` (ties to the lower index)."""
    hi = torch.searchsorted(code, x.contiguous()).clamp(1, code.numel() - 1)
    lo = hi - 1
    d_lo = (x.double() - code[lo].double()).abs()
    d_hi = (code[hi].double() - x.double()).abs()
    return torch.where(d_hi < d_lo, hi, lo)


def quantize_4bit(A: torch.Tensor, blocksize: int = 64, compress_statistics: bool = True,
                  quant_type: str = "nf4") -> tuple[torch.Tensor, QuantState]:
    """(packed uint8 [ceil(n/2), 1], QuantState) of `A` in NF4."""
    if quant_type != "nf4":
        raise ValueError("only NF4 is implemented")
    if blocksize % 2:
        raise ValueError("blocksize must be even")
    dev = A.device
    shape = tuple(A.shape)
    flat = A.detach().reshape(-1).float()
    n = flat.numel()
    nb = -(-n // blocksize)
    padded = torch.zeros(nb * blocksize, dtype=torch.float32, device=dev)
    padded[:n] = flat
    blocks = padded.view(nb, blocksize)
    absmax = blocks.abs().amax(1)
    inv = torch.where(absmax > 0, 1.0 / absmax, torch.zeros_like(absmax))
    normed = (blocks * inv[:, None]).reshape(-1)[:n]
    code = torch.tensor(NF4_CODE, dtype=torch.float32, device=dev)
    mids = ((code.double()[:-1] + code.double()[1:]) / 2.0).float()
    q = torch.searchsorted(mids, normed.contiguous()).to(torch.uint8)
    if n % 2:
        q = torch.cat([q, torch.zeros(1, dtype=torch.uint8, device=dev)])
    packed = ((q[0::2] << 4) | q[1::2]).view(-1, 1)
    if not compress_statistics:
        return packed, QuantState(absmax=absmax, shape=torch.Size(shape), code=code,
                                  blocksize=blocksize, quant_type="nf4", dtype=A.dtype)
    offset = absmax.double().mean().float()  # fp64 accumulation: independent of the order
    x2 = absmax - offset
    nb2 = -(-nb // 256)
    pad2 = torch.zeros(nb2 * 256, dtype=torch.float32, device=dev)
    pad2[:nb] = x2
    b2 = pad2.view(nb2, 256)
    absmax2 = b2.abs().amax(1)
    inv2 = torch.where(absmax2 > 0, 1.0 / absmax2, torch.zeros_like(absmax2))
    normed2 = (b2 * inv2[:, None]).reshape(-1)[:nb]
    code2 = dynamic_map().to(dev)
    qabs = _nearest(normed2, code2).to(torch.uint8)
    state2 = QuantState(absmax=absmax2, code=code2, blocksize=256, quant_type=None,
                        dtype=torch.float32)
    return packed, QuantState(absmax=qabs, shape=torch.Size(shape), code=code,
                              blocksize=blocksize, quant_type="nf4", dtype=A.dtype,
                              offset=offset, state2=state2)


def nf4_state_ok(packed: torch.Tensor, quant_state, in_features: int | None = None) -> bool:
    """The checks of the reference's `_nf4_state_ok` (nf4.py:127-132)."""
    return (quant_state is not None and quant_state.quant_type == "nf4"
            and len(quant_state.shape) == 2
            and (in_features is None or quant_state.shape[1] == in_features)
            and quant_state.blocksize % 2 == 0
            and (not quant_state.nested or quant_state.state2.blocksize == 256)
            and packed.dtype == torch.uint8 and packed.is_contiguous())


def _device_f32(t, device) -> torch.Tensor:
    return t.to(device=device, dtype=torch.float32).contiguous()


def weight_desc(packed: torch.Tensor, quant_state) -> NF4Weight:
    """The C-ABI descriptor of one weight.  Device copies of the tables (fp32 code maps, the
    offset as a host float) are made once and cached on the QuantState, as the reference caches
    its rebuilt absmax there (nf4.py:43-54); the descriptor references `packed` directly."""
    qs = quant_state
    dev = packed.device
    refs = getattr(qs, "_nf4_refs", None)
    if refs is None or refs[0] != dev:
        code = _device_f32(qs.code, dev)
        if qs.nested:
            absmax = qs.absmax.to(device=dev, dtype=torch.uint8).contiguous()
            absmax2 = _device_f32(qs.state2.absmax, dev)
            code2 = _device_f32(qs.state2.code, dev)
            offset = float(qs.offset)  # one host sync per weight and process
            bs2 = int(qs.state2.blocksize)
        else:
            absmax = _device_f32(qs.absmax, dev)
            absmax2 = code2 = None
            offset, bs2 = 0.0, 0
        refs = (dev, code, absmax, absmax2, code2, offset, bs2)
        qs._nf4_refs = refs
    _, code, absmax, absmax2, code2, offset, bs2 = refs
    rows, cols = int(qs.shape[0]), int(qs.shape[1])
    return NF4Weight(
        packed=packed.data_ptr(), absmax=absmax.data_ptr(),
        absmax2=absmax2.data_ptr() if absmax2 is not None else None,
        code2=code2.data_ptr() if code2 is not None else None,
        code=code.data_ptr(), offset=offset, nested=1 if qs.nested else 0, rows=rows, cols=cols,
        blocksize=int(qs.blocksize), blocksize2=bs2)


def weight_array(descs: list[NF4Weight]):
    arr = (NF4Weight * len(descs))(*descs)
    return arr


def packed_bytes(n_elements: int) -> int:
    return math.ceil(n_elements / 2)


__all__ = ["NF4_CODE", "QuantState", "dynamic_map", "quantize_4bit", "nf4_state_ok",
           "weight_desc", "weight_array", "packed_bytes", "ctypes"]
