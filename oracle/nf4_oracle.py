"""CPU oracle for the NF4 quantized-linear path.  TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import this
module, and only as the checker.  The product path (the HIP library and its Python host layer in
`kaggle-mltest_amd/`) never calls it and never falls back to it.

What it restates, and where the reference does it
-------------------------------------------------
The reference keeps weights in the bitsandbytes 0.50.2 ``QuantState`` layout and dequantizes them
with its own Triton kernel (``/root/reference/solution/nf4.py:26-55``):

* element ``i`` of the row-major flattened weight lives in byte ``i // 2``, high nibble for even
  ``i`` (nf4.py:33-35; layer.py:65-69);
* the double-quantized absmax is rebuilt as ``fp32(code2[q] * absmax2[b // 256]) + offset``
  (bnb ``dequantize_blockwise`` then ``+ offset``, nf4.py:47-51): two fp32 roundings, no FMA;
* the weight is ``fp16(fp32(code[nib]) * absmax_fp32[i // blocksize])``, one rounding to nearest
  even (nf4.py:36-38, bnb ``kDequantizeBlockwise``);
* the forward GEMM is ``F.linear(x, W, bias)`` and the input gradient ``grad @ W``
  (nf4.py:84-102), the LoRA update ``s * (drop(x) @ A^T) @ B^T`` with its gradients
  (layer.py:875-878, 1072-1090), and the recomputed MLP (mlp.py:42-74).

bitsandbytes itself is absent from this machine and from the GPU box, so its quantizer is restated
from the published method (Dettmers et al. 2022 block-wise dynamic quantization; QLoRA 2023 NF4
with double quantization): ``create_normal_map`` and ``create_dynamic_map`` below follow the
constructions bitsandbytes publishes in ``bitsandbytes/functional.py``.

Pinning (what makes this oracle trustworthy, checked in ``tests/test_oracle.py``)
----------------------------------------------------------------------------------
* ``NF4_CODE`` literals: against the closed-form normal-quantile construction (scipy ``norm.ppf``),
  sortedness, ``code[7] == 0``, the ``+-1`` ends.
* ``create_dynamic_map``: against its closed form per decade (``10**(i-6)`` times the midpoints
  of ``linspace(0.1, 1, 2**i + 1)``), size 256, sortedness, symmetry, ``0`` and ``1`` present.
* ``dequantize``: against an element-by-element Python loop, against torch's own fp32 -> fp16 /
  bf16 conversion (a library routine), and against hand-computed special cases.
* ``absmax_fp32``: against a loop over blocks with explicit fp32 scalar arithmetic.
* quantize -> dequantize: error bounded by half the widest NF4 gap times the block absmax.
* GEMM / LoRA references: a library routine (torch CPU fp32 matmul) on the bit-exact weight, and
  the hand-written LoRA backward formulas against torch autograd of the forward formula.
* Parity unpinned: bitsandbytes' own quantizer tie-breaking (its 8-bit binary search in
  ``dQuantize`` and NF4 decision tree), which no file on this machine holds.  Dequantization is
  table-driven and does not depend on it.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

# bitsandbytes' NF4 table (``get_4bit_type("nf4")``), the 16 fp32 values of QLoRA's NormalFloat4.
NF4_CODE = np.array([
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0], dtype=np.float32)


# ------------------------------------------------------------------------------------ code maps

def create_normal_map(offset: float = 0.9677083) -> np.ndarray:
    """The NF4 table rebuilt from its definition: 8 positive normal quantiles on
    ``linspace(offset, 0.5, 9)[:-1]``, 7 negative ones on ``linspace(offset, 0.5, 8)[:-1]``, plus
    zero, sorted and divided by the largest value (bitsandbytes ``create_normal_map`` with
    ``use_extra_value=True``).  Returns the 16 distinct values in fp32."""
    from scipy.stats import norm

    pos = norm.ppf(np.linspace(offset, 0.5, 9, dtype=np.float32)[:-1].astype(np.float64))
    neg = -norm.ppf(np.linspace(offset, 0.5, 8, dtype=np.float32)[:-1].astype(np.float64))
    values = np.sort(np.concatenate([pos, [0.0], neg]).astype(np.float32))
    return (values / values.max()).astype(np.float32)


def create_dynamic_map(signed: bool = True, max_exponent_bits: int = 7,
                       total_bits: int = 8) -> np.ndarray:
    """The 8-bit dynamic map that double quantization stores the absmax with (bitsandbytes
    ``create_dynamic_map``, Dettmers et al. 2022): for decade ``i`` the midpoints of
    ``linspace(0.1, 1, 2**(i + non_sign_bits - max_exponent_bits) + 1)`` scaled by
    ``10**(i - (max_exponent_bits - 1))``, mirrored when signed, plus 0 and 1, sorted."""
    import torch  # bitsandbytes builds the map with torch's fp32 linspace and fp32 products

    data: list[float] = []
    non_sign_bits = total_bits - 1
    additional = 2 ** (non_sign_bits - max_exponent_bits) - 1

    def decade(count: int, i: int) -> None:
        bounds = torch.linspace(0.1, 1, count, dtype=torch.float32)
        means = (bounds[:-1] + bounds[1:]) / 2.0
        scale = 10.0 ** (-(max_exponent_bits - 1) + i)
        data.extend((scale * means).tolist())
        if signed:
            data.extend((-scale * means).tolist())

    for i in range(max_exponent_bits):
        decade(2 ** (i + non_sign_bits - max_exponent_bits) + 1 if signed else
               2 ** (i + non_sign_bits - max_exponent_bits + 1) + 1, i)
    if additional > 0:
        decade(additional + 1, max_exponent_bits - 1)
    data += [0.0, 1.0]
    data += [0.0] * (2 ** total_bits - len(data))
    return np.sort(np.array(data, dtype=np.float32))


DYNAMIC_CODE = create_dynamic_map()


# ------------------------------------------------------------------------------- quant state

@dataclass
class OracleState2:
    absmax: np.ndarray          # fp32 [ceil(nblocks / blocksize)]
    code: np.ndarray            # fp32 [256]
    blocksize: int = 256


@dataclass
class OracleQuantState:
    """The bitsandbytes ``QuantState`` fields the path reads (nf4.py:46-53, 112-131)."""
    absmax: np.ndarray          # uint8 [nblocks] when nested, else fp32 [nblocks]
    shape: tuple
    code: np.ndarray = field(default_factory=lambda: NF4_CODE.copy())
    blocksize: int = 64
    quant_type: str = "nf4"
    offset: float = 0.0         # fp32 value
    state2: OracleState2 | None = None
    nested: bool = False


# ---------------------------------------------------------------------------------- quantize

def _nf4_thresholds(code: np.ndarray) -> np.ndarray:
    mids = (code.astype(np.float64)[:-1] + code.astype(np.float64)[1:]) / 2.0
    return mids.astype(np.float32)


def quantize_nf4_codes(x: np.ndarray, code: np.ndarray = NF4_CODE) -> np.ndarray:
    """Nearest NF4 index of each normalised value: above a midpoint goes up (ties go down)."""
    return np.searchsorted(_nf4_thresholds(code), x.astype(np.float32), side="left").astype(
        np.uint8)


def quantize_blockwise_u8(x: np.ndarray, code2: np.ndarray = DYNAMIC_CODE,
                          blocksize: int = 256) -> tuple[np.ndarray, np.ndarray]:
    """Block-wise 8-bit quantization of ``x`` (fp32, flat): per block the absmax, values scaled by
    its fp32 reciprocal, each mapped to the nearest entry of ``code2`` (ties to the lower index).
    bitsandbytes' GPU kernel reaches the nearest entry by binary search; exact ties are the only
    place the two may differ (parity unpinned there)."""
    x = x.astype(np.float32).reshape(-1)
    n = x.size
    nb = -(-n // blocksize)
    pad = np.zeros(nb * blocksize, np.float32)
    pad[:n] = x
    blocks = pad.reshape(nb, blocksize)
    absmax2 = np.abs(blocks).max(1).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = np.where(absmax2 > 0, np.float32(1.0) / absmax2, np.float32(0.0)).astype(np.float32)
    normed = (blocks * inv[:, None]).astype(np.float32).reshape(-1)[:n]
    hi = np.clip(np.searchsorted(code2, normed, side="left"), 1, code2.size - 1)
    lo = hi - 1
    d_lo = np.abs(normed.astype(np.float64) - code2[lo])
    d_hi = np.abs(code2[hi].astype(np.float64) - normed)
    q = np.where(d_hi < d_lo, hi, lo).astype(np.uint8)
    return q, absmax2


def quantize_nf4(w: np.ndarray, blocksize: int = 64, compress_statistics: bool = True,
                 code: np.ndarray = NF4_CODE) -> tuple[np.ndarray, OracleQuantState]:
    """bitsandbytes ``quantize_4bit(w, blocksize, compress_statistics, quant_type="nf4")`` in the
    same storage layout: packed uint8 [ceil(n/2)], high nibble first."""
    shape = tuple(int(s) for s in w.shape)
    flat = w.astype(np.float32).reshape(-1)
    n = flat.size
    nb = -(-n // blocksize)
    pad = np.zeros(nb * blocksize, np.float32)
    pad[:n] = flat
    blocks = pad.reshape(nb, blocksize)
    absmax = np.abs(blocks).max(1).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = np.where(absmax > 0, np.float32(1.0) / absmax, np.float32(0.0)).astype(np.float32)
    normed = (blocks * inv[:, None]).astype(np.float32).reshape(-1)[:n]
    q = quantize_nf4_codes(normed, code)
    if n % 2:
        q = np.concatenate([q, np.zeros(1, np.uint8)])
    packed = ((q[0::2] << 4) | q[1::2]).astype(np.uint8)
    if compress_statistics:
        # the mean of the block absmax, accumulated in fp64 and rounded once to fp32
        offset = np.float32(absmax.astype(np.float64).mean())
        q2, absmax2 = quantize_blockwise_u8((absmax - offset).astype(np.float32))
        state = OracleQuantState(absmax=q2, shape=shape, code=code.copy(), blocksize=blocksize,
                                 offset=float(offset), nested=True,
                                 state2=OracleState2(absmax=absmax2, code=DYNAMIC_CODE.copy()))
    else:
        state = OracleQuantState(absmax=absmax, shape=shape, code=code.copy(),
                                 blocksize=blocksize)
    return packed, state


# -------------------------------------------------------------------------------- dequantize

def absmax_fp32(state: OracleQuantState) -> np.ndarray:
    """Per-block absmax in fp32: ``fp32(code2[q] * absmax2[b // 256]) + offset`` for a nested
    state (bnb ``dequantize_blockwise`` + offset, nf4.py:47-51), the stored fp32 otherwise."""
    if not state.nested:
        return state.absmax.astype(np.float32)
    s2 = state.state2
    idx = np.arange(state.absmax.size) // s2.blocksize
    prod = (s2.code[state.absmax.astype(np.int64)].astype(np.float32)
            * s2.absmax[idx].astype(np.float32)).astype(np.float32)
    return (prod + np.float32(state.offset)).astype(np.float32)


def f32_to_bf16_bits(v: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 with round-to-nearest-even, returned as uint16 bit patterns."""
    bits = v.astype(np.float32).view(np.uint32).astype(np.uint64)
    bias = 0x7FFF + ((bits >> 16) & 1)
    return ((bits + bias) >> 16).astype(np.uint16)


def nibbles(packed: np.ndarray, n: int) -> np.ndarray:
    """The 4-bit index of each of the ``n`` elements: byte i//2, high nibble for even i."""
    p = packed.reshape(-1).astype(np.uint8)
    out = np.empty(p.size * 2, np.uint8)
    out[0::2] = p >> 4
    out[1::2] = p & 0xF
    return out[:n]


def dequantize_f32(packed: np.ndarray, state: OracleQuantState) -> np.ndarray:
    """The fp32 products ``code[nib] * absmax`` (before the one rounding to the output type)."""
    n = int(np.prod(state.shape))
    a = absmax_fp32(state)
    nib = nibbles(packed, n)
    scale = a[np.arange(n) // state.blocksize]
    return (state.code[nib].astype(np.float32) * scale).astype(np.float32).reshape(state.shape)


def dequantize(packed: np.ndarray, state: OracleQuantState, dtype: str = "f16") -> np.ndarray:
    """The dequantized weight: ``"f16"`` -> float16, ``"bf16"`` -> uint16 bf16 bits,
    ``"f32"`` -> float32 (nf4.py:69-77 with ``dtype``)."""
    v = dequantize_f32(packed, state)
    if dtype == "f16":
        with np.errstate(over="ignore"):  # beyond fp16 range rounds to +-inf, as on the GPU
            return v.astype(np.float16)
    if dtype == "bf16":
        return f32_to_bf16_bits(v)
    if dtype == "f32":
        return v
    raise ValueError(dtype)


def _round_to(v: np.ndarray, dtype: str) -> np.ndarray:
    """fp32 values rounded (RNE) to ``dtype`` and returned as fp32."""
    v = np.asarray(v, dtype=np.float32)
    if dtype == "f16":
        return v.astype(np.float16).astype(np.float32)
    bits = f32_to_bf16_bits(v).astype(np.uint32) << 16
    return bits.view(np.float32)


def dequantize_scaled_codes(packed: np.ndarray, state: OracleQuantState,
                            dtype: str = "f16") -> np.ndarray:
    """The weight as the small-M (decode) GEMV multiplies it: the 16 codes rounded to the GEMM
    dtype, each times its block's fp32 absmax in fp32, rounded once to ``dtype`` - what a
    one-hot activation row returns.  Returns float16, or bf16 bits as uint16.  It differs
    from ``dequantize`` (one rounding of the fp32 product code * absmax) only where the code
    itself is not exact in ``dtype``; bitsandbytes' own decode GEMV forms no rounded weight at
    all (fp32 code * fp32 absmax * x)."""
    n = int(np.prod(state.shape))
    a = absmax_fp32(state)
    nib = nibbles(packed, n)
    code = _round_to(state.code.astype(np.float32), dtype)
    v = (code[nib] * a[np.arange(n) // state.blocksize]).astype(np.float32)
    if dtype == "f16":
        return v.astype(np.float16).reshape(state.shape)
    return f32_to_bf16_bits(v).reshape(state.shape)


def dequantize_loop(packed: np.ndarray, state: OracleQuantState) -> np.ndarray:
    """Element-by-element restatement (tiny inputs only): fp16 output."""
    n = int(np.prod(state.shape))
    out = np.empty(n, np.float16)
    p = packed.reshape(-1)
    for i in range(n):
        byte = int(p[i // 2])
        nib = (byte >> 4) if i % 2 == 0 else (byte & 0xF)
        b = i // state.blocksize
        if state.nested:
            q = int(state.absmax[b])
            a = np.float32(state.state2.code[q]) * np.float32(state.state2.absmax[b // 256])
            a = np.float32(np.float32(a) + np.float32(state.offset))
        else:
            a = np.float32(state.absmax[b])
        out[i] = np.float16(np.float32(state.code[nib]) * a)
    return out.reshape(state.shape)


# ------------------------------------------------------------------------ GEMM / LoRA (fp32)

def _t(a):
    import torch

    if isinstance(a, np.ndarray):
        if a.dtype == np.uint16:  # bf16 bits
            return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).float()
        return torch.from_numpy(np.ascontiguousarray(a)).float()
    return a.float().cpu()  # differentiable: references may be run under autograd


def linear_fwd(x, w, bias=None, loras=()):
    """fp32 ``x @ W^T + bias + sum_seg s * (xd @ A^T) @ B^T`` on the bit-exact weight
    (nf4.py:84-91; layer.py:871-878).  ``loras``: (col0, ncols, xd, A [r,K], B [ncols,r], s),
    where the LoRA output lands in columns ``col0 : col0 + ncols``."""
    x, w = _t(x), _t(w)
    y = x @ w.t()
    if bias is not None:
        y = y + _t(bias)
    for col0, ncols, xd, a, b, s in loras:
        y[..., col0:col0 + ncols] += float(s) * ((_t(xd) @ _t(a).t()) @ _t(b).t())
    return y


def linear_dx(dy, w, loras=()):
    """fp32 ``dX = dY @ W + sum_seg (s * dY_seg @ B) @ A`` (nf4.py:96-99; layer.py:1077,
    1086-1088)."""
    dy, w = _t(dy), _t(w)
    dx = dy @ w
    for col0, ncols, _xd, a, b, s in loras:
        dx = dx + (float(s) * dy[..., col0:col0 + ncols] @ _t(b)) @ _t(a)
    return dx


def lora_grads(dy_seg, xd, a, b, s):
    """fp32 LoRA gradients (layer.py:1072-1081): ``dl = s*dY``, ``dB = dl^T (xd A^T)``,
    ``dA = (dl B)^T xd``.  Returns (dA [r,K], dB [N,r])."""
    dy_seg, xd, a, b = _t(dy_seg), _t(xd), _t(a), _t(b)
    dl = float(s) * dy_seg.reshape(-1, dy_seg.shape[-1])
    xd = xd.reshape(-1, xd.shape[-1])
    t = xd @ a.t()
    grad_b = dl.t() @ t
    grad_a = (dl @ b).t() @ xd
    return grad_a, grad_b


def silu(v):
    return v / (1.0 + (-v).exp())


def mlp_fwd(x, wg, wu, wd):
    """fp32 SwiGLU MLP ``down(silu(gate(x)) * up(x))`` (mlp.py:44-57)."""
    x = _t(x)
    g, u = x @ _t(wg).t(), x @ _t(wu).t()
    return (silu(g) * u) @ _t(wd).t()


# --------------------------------------------------- the projection's neighbours (fp32)

def pack_keep_bits(keep_q, keep_v) -> np.ndarray:
    """0/1 keep masks [rows, cols] (cols a multiple of 8) -> uint8 [rows, 2 * cols / 8]: per row
    q's bytes then v's, bit k of byte j = element 8 j + k (layer.py:76-81, 118-125)."""
    out = []
    for keep in (keep_q, keep_v):
        k = (np.asarray(keep) != 0).astype(np.uint32)
        rows, cols = k.shape
        b = (k.reshape(rows, cols // 8, 8) << np.arange(8, dtype=np.uint32)).sum(-1)
        out.append(b.astype(np.uint8))
    return np.concatenate(out, axis=1)


def unpack_keep_bits(packed, cols):
    """The inverse of pack_keep_bits: (keep_q, keep_v) as uint8 0/1 [rows, cols]
    (layer.py:84-90)."""
    p = np.asarray(packed, dtype=np.uint8)
    nb = cols // 8
    res = []
    for half in (p[:, :nb], p[:, nb:2 * nb]):
        bits = (half[:, :, None].astype(np.uint32) >> np.arange(8, dtype=np.uint32)) & 1
        res.append(bits.reshape(p.shape[0], cols).astype(np.uint8))
    return res[0], res[1]


def add_rmsnorm(x, w, eps, d=None, keep_q=None, keep_v=None, scale_q=1.0, scale_v=1.0):
    """fp32 ``h = x (+ d)``, ``rstd = 1/sqrt(mean(h^2) + eps)``, ``y = w * (h * rstd)`` and
    LoRA's dropout inputs ``y * keep * scale`` (layer.py:92-132).  Returns (y, rstd, oq, ov)."""
    h = _t(x)
    if d is not None:
        h = h + _t(d)
    rstd = 1.0 / (h.pow(2).mean(-1, keepdim=True) + float(eps)).sqrt()
    y = _t(w) * (h * rstd)
    oq = ov = None
    if keep_q is not None:
        oq = y * _t(keep_q) * float(scale_q)
        ov = y * _t(keep_v) * float(scale_v)
    return y, rstd.squeeze(-1), oq, ov


def rmsnorm_bwd(x, w, rstd, dy=None, d=None, dres=None, dq=None, dv=None, keep_q=None,
                keep_v=None, scale_q=1.0, scale_v=1.0):
    """fp32 gradient of add_rmsnorm (layer.py:135-164): ``g = dy + dq*keep_q*s_q +
    dv*keep_v*s_v``, ``h^ = (x + d) * rstd``, ``dx = rstd (g w - h^ mean(g w h^)) + dres``."""
    h = _t(x)
    if d is not None:
        h = h + _t(d)
    g = _zeros_like(h)
    if dy is not None:
        g = g + _t(dy)
    if dq is not None:
        g = g + _t(dq) * _t(keep_q) * float(scale_q) + _t(dv) * _t(keep_v) * float(scale_v)
    r = _t(rstd).reshape(-1, 1)
    hh = h * r
    gw = g * _t(w)
    dx = r * (gw - hh * (gw * hh).mean(-1, keepdim=True))
    if dres is not None:
        dx = dx + _t(dres)
    return dx


def _zeros_like(t):
    import torch

    return torch.zeros_like(t)


def _rotate(lo, hi, cos, sin, half):
    return (lo * cos[:, None, :half] - hi * sin[:, None, :half],
            hi * cos[:, None, half:] + lo * sin[:, None, half:])


def qkv_rope(qkv, cos, sin, n_heads, n_kv, head_dim):
    """fp32 rotary embedding of the finished q|k|v projection (layer.py:167-218 without its
    LoRA add): q, k rotated, k and v expanded to every query head.  Returns (q, k, v, kc, vc)
    with q, k, v [tokens, n_heads, head_dim] and kc, vc [tokens, n_kv, head_dim]."""
    import torch

    qkv, cos, sin = _t(qkv), _t(cos), _t(sin)
    t, half, groups = qkv.shape[0], head_dim // 2, n_heads // n_kv
    q = qkv[:, :n_heads * head_dim].reshape(t, n_heads, head_dim)
    k = qkv[:, n_heads * head_dim:(n_heads + n_kv) * head_dim].reshape(t, n_kv, head_dim)
    v = qkv[:, (n_heads + n_kv) * head_dim:(n_heads + 2 * n_kv) * head_dim].reshape(t, n_kv, head_dim)
    qr = torch.cat(_rotate(q[..., :half], q[..., half:], cos, sin, half), -1)
    kr = torch.cat(_rotate(k[..., :half], k[..., half:], cos, sin, half), -1)
    return (qr, kr.repeat_interleave(groups, 1), v.repeat_interleave(groups, 1), kr, v)


def qkv_rope_bwd(dq, dk, dv, cos, sin, n_kv):
    """fp32 gradient of qkv_rope into the [tokens, q|k|v] layout (layer.py:221-263): the
    transposed rotation; the expanded copies' gradients summed per key/value head."""
    import torch

    dq, dk, dv, cos, sin = _t(dq), _t(dk), _t(dv), _t(cos), _t(sin)
    t, n_heads, head_dim = dq.shape
    half, groups = head_dim // 2, n_heads // n_kv

    def back(g):
        lo, hi = g[..., :half], g[..., half:]
        return torch.cat((lo * cos[:, None, :half] + hi * sin[:, None, half:],
                          hi * cos[:, None, half:] - lo * sin[:, None, :half]), -1)

    gk = dk.reshape(t, n_kv, groups, head_dim).sum(2)
    gv = dv.reshape(t, n_kv, groups, head_dim).sum(2)
    return torch.cat((back(dq).reshape(t, -1), back(gk).reshape(t, -1), gv.reshape(t, -1)), 1)


# ----------------------------------------------------------------- int8 input gradients
#
# The reference's int8 MLP backward (layer.py:299-442, 515-618, 992-1013), restated in numpy
# float32 with every product / quotient rounded on its own; integer GEMMs in int64 (exact).

def round_i8(v: np.ndarray) -> np.ndarray:
    """Ties away from zero, clamped to [-127, 127] (layer.py:299-303):
    ``floor(v + 0.5)`` for v >= 0, ``-floor(0.5 - v)`` otherwise, in fp32."""
    v = np.asarray(v, dtype=np.float32)
    half = np.float32(0.5)
    r = np.where(v >= 0, np.floor(v + half), -np.floor(half - v)).astype(np.float32)
    return np.clip(r, -127, 127).astype(np.int8)


def int8_rows(x) -> tuple[np.ndarray, np.ndarray]:
    """One int8 row per row (row_quant_kernel, layer.py:372-382): top = max(max|x|, 1e-20),
    q = round(x * fp32(127 / top)), s = fp32(top / 127)."""
    x = _np32(x)
    top = np.maximum(np.abs(x).max(axis=1), np.float32(1e-20)).astype(np.float32)
    inv = (np.float32(127.0) / top).astype(np.float32)
    q = round_i8((x * inv[:, None]).astype(np.float32))
    return q, (top / np.float32(127.0)).astype(np.float32)


def _np32(x) -> np.ndarray:
    if hasattr(x, "detach"):
        x = x.detach().cpu().float().numpy()
    return np.asarray(x, dtype=np.float32)


def stack_f32(weights) -> np.ndarray:
    """fp32 products code[nib] * absmax of stacked weights [(packed, OracleQuantState)]."""
    return np.concatenate([dequantize_f32(p, st).reshape(st.shape) for p, st in weights])


def col_scales(weights, dtype: str = "f16") -> np.ndarray:
    """Per input column, max(largest |W|, 1e-20) / 127 with W dequantized to ``dtype``
    (_col_scales, layer.py:598-615)."""
    w = np.concatenate([_as_f32(dequantize(p, st, dtype), dtype).reshape(st.shape)
                        for p, st in weights])
    top = np.abs(w).max(axis=0).astype(np.float32)
    return (np.maximum(top, np.float32(1e-20)) / np.float32(127.0)).astype(np.float32)


def _as_f32(w: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return (w.astype(np.uint32) << 16).view(np.float32)
    return w.astype(np.float32)


def int8_weight_t(weights, scale: np.ndarray) -> np.ndarray:
    """The stack as int8, transposed: q[c][r] = round(fp32(W[r][c] / scale[c])) with W the fp32
    product (nf4_int8_t_kernel, layer.py:338-369)."""
    w = stack_f32(weights)
    return np.ascontiguousarray(round_i8((w / scale[None, :]).astype(np.float32)).T)


def int8_weight_rows(weights) -> tuple[np.ndarray, np.ndarray]:
    """The stack as int8 rows with one scale per row (nf4_int8_rows_kernel, layer.py:306-335)."""
    return int8_rows(stack_f32(weights))


def int8_matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Exact ``a [M, K] . b [N, K]^T`` of int8 operands (torch._int_mm), as int64: evaluated in
    float64, which holds every partial sum exactly (|sum| <= 127^2 K < 2^53 for K < 5e8)."""
    assert a.shape[1] * 127 * 127 < 2 ** 53
    return (a.astype(np.float64) @ b.astype(np.float64).T).astype(np.int64)


def int8_scale(acc: np.ndarray, sa: np.ndarray, sb: np.ndarray) -> np.ndarray:
    """fp32(acc) * sa[m] * sb[n], left to right (layer.py:1012)."""
    f = acc.astype(np.float32)
    return ((f * sa[:, None].astype(np.float32)).astype(np.float32) *
            sb[None, :].astype(np.float32)).astype(np.float32)


def int8_swiglu_bwd(acc: np.ndarray, sd: np.ndarray, cs: np.ndarray, gu) -> tuple:
    """gate_up_act_bwd_i8_kernel (layer.py:414-442): dh = fp32(acc) * sd[m] * cs[j]; with g, u
    the saved gate | up halves and sig = 1 / (1 + exp(-g)): d_gate = dh u sig (1 + g (1 - sig)),
    d_up = dh g sig; q = round(grad * fp32(127 / peak)) per row over both halves (peak = max(
    largest |grad|, 1e-20)), sq = peak / 127.  Returns (q [M, 2I] int8, sq, d_gate, d_up)."""
    gu = _np32(gu)
    inter = acc.shape[1]
    g, u = gu[:, :inter], gu[:, inter:]
    f32 = np.float32
    dh = ((acc.astype(f32) * sd[:, None].astype(f32)).astype(f32) * cs[None, :].astype(f32)).astype(f32)
    sig = (f32(1.0) / (f32(1.0) + np.exp(-g).astype(f32))).astype(f32)
    du = ((dh * g).astype(f32) * sig).astype(f32)
    dg = (((dh * u).astype(f32) * sig).astype(f32) *
          (f32(1.0) + (g * (f32(1.0) - sig)).astype(f32)).astype(f32)).astype(f32)
    peak = np.maximum(np.maximum(np.abs(dg).max(axis=1), np.abs(du).max(axis=1)), f32(1e-20))
    peak = peak.astype(f32)
    inv = (f32(127.0) / peak).astype(f32)
    q = np.concatenate([round_i8((dg * inv[:, None]).astype(f32)),
                        round_i8((du * inv[:, None]).astype(f32))], axis=1)
    return q, (peak / f32(127.0)).astype(f32), dg, du


def mlp_dx_int8(dh2, gu, gate_up, down, dtype: str = "f16"):
    """The int8 MLP input gradient (layer.py:992-1013, without the 512-token chunking, which
    only bounds the T4's memory): dh2 -> int8 rows, . int8 W_down^T (column scales), SwiGLU
    backward requantized, . int8 W_gate|up^T, scaled.  Returns fp32 dy2 before the rounding
    to the GEMM dtype."""
    cs_gu, cs_d = col_scales(gate_up, dtype), col_scales(down, dtype)
    dh8, sdh = int8_rows(dh2)
    acc = int8_matmul(dh8, int8_weight_t(down, cs_d))
    q8, sq, _, _ = int8_swiglu_bwd(acc, sdh, cs_d, gu)
    return int8_scale(int8_matmul(q8, int8_weight_t(gate_up, cs_gu)), sq, cs_gu)


def gate_up_fwd_int8(x, gate_up, dtype: str = "f16"):
    """The int8 gate|up forward (layer.py:900-912 with gate_up_act_fwd_i8_kernel, 383-405;
    without the 512-token chunking, which only bounds the T4's int32 buffer): x -> int8 rows
    (sx), the stacked weights -> int8 rows (sw, nf4_int8_rows_kernel), the exact int32 product,
    gu = round_dtype(fp32(acc) * sx[m] * sw[n]), and act = g / (1 + exp(-g)) * u in fp32 from
    the rounded halves, rounded once.  Returns (gu [M, 2I], act [M, I]) as fp32 arrays holding
    dtype values."""
    x8, sx = int8_rows(x)
    w8, sw = int8_weight_rows(gate_up)
    gu = _round_to(int8_scale(int8_matmul(x8, w8), sx, sw), dtype)
    inter = gu.shape[1] // 2
    g, u = gu[:, :inter], gu[:, inter:]
    f32 = np.float32
    with np.errstate(over="ignore"):
        act = (g / (f32(1.0) + np.exp(-g).astype(f32))).astype(f32)
    return gu, _round_to((act * u).astype(f32), dtype)


def rel_errors(out, ref) -> tuple[float, float]:
    """(max |out-ref| / max |ref|, mean |out-ref| / mean |ref|): the reference's ``_rel``
    (layer.py:1253-1254) and its mean counterpart."""
    out, ref = _t(out).detach(), _t(ref).detach()
    d = (out - ref).abs()
    return (d.max().item() / (ref.abs().max().item() + 1e-12),
            d.mean().item() / (ref.abs().mean().item() + 1e-12))


def nf4_max_gap() -> float:
    """Half the widest gap between neighbouring NF4 values (the worst rounding, in units of
    the block absmax)."""
    return float(np.max(np.diff(NF4_CODE.astype(np.float64))) / 2.0)


__all__ = [n for n in dir() if not n.startswith("_") and n not in ("annotations", "math",
                                                                      "np", "field",
                                                                      "dataclass")]
