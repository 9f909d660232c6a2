"""Tensor-level wrappers of the C ABI: allocate outputs and workspaces with torch (device
memory and streams only), pass raw pointers, launch on torch's current stream, raise on a
nonzero status.  No arithmetic happens here."""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import DTYPE_CODE, NF4Lora, NF4LoraJob, check, load, stream_of
from .quant_state import weight_array, weight_desc

GEMM_DTYPES = (torch.float16, torch.bfloat16)

# tilings of the tiled GEMMs (NF4_TILE_* of the C header)
TILE_256, TILE_128, TILE_128_KSPLIT2 = 0, 1, 3


def _code(dtype: torch.dtype, allowed=GEMM_DTYPES) -> int:
    if dtype not in allowed:
        raise TypeError(f"dtype {dtype} is not supported here (expected one of {allowed})")
    return DTYPE_CODE[dtype]


def _descs(weights):
    """[(packed, quant_state), ...] -> ctypes array of descriptors."""
    return weight_array([weight_desc(p, qs) for p, qs in weights])


def _check_device(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("the NF4 kernels run on the GPU: every tensor must be on a cuda device")


def dequant(weights, dtype=torch.float16, out: torch.Tensor | None = None) -> torch.Tensor:
    """Stacked [sum rows, cols] dequantized weight(s) (nf4_dequant_multi)."""
    packed0 = weights[0][0]
    _check_device(packed0)
    rows = sum(int(qs.shape[0]) for _, qs in weights)
    cols = int(weights[0][1].shape[1])
    if out is None:
        out = torch.empty((rows, cols), dtype=dtype, device=packed0.device)
    arr = _descs(weights)
    st = load().nf4_dequant_multi(arr, len(weights), out.data_ptr(),
                                  _code(dtype, (torch.float16, torch.bfloat16, torch.float32)),
                                  stream_of(out))
    check(st, "nf4_dequant_multi")
    return out


def dequant_batch(weights, dtype=torch.float16, outs=None) -> list:
    """Each weight dequantized into its own [rows, cols] tensor, all in one launch
    (nf4_dequant_batch, at most 8 weights)."""
    packed0 = weights[0][0]
    _check_device(packed0)
    if outs is None:
        outs = [torch.empty(tuple(int(d) for d in qs.shape), dtype=dtype, device=packed0.device)
                for _, qs in weights]
    arr = _descs(weights)
    ptrs = (ctypes.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
    st = load().nf4_dequant_batch(arr, len(weights), ptrs,
                                  _code(dtype, (torch.float16, torch.bfloat16, torch.float32)),
                                  stream_of(outs[0]))
    check(st, "nf4_dequant_batch")
    return outs


class DequantTable:
    """Any number of weights dequantized by one launch (nf4_dequant_table): the descriptor
    table is packed once on the host and kept in device memory; `run()` launches on torch's
    current stream.  `outs` default to fresh [rows, cols] tensors; the weights and outputs must
    stay alive (and in place) as long as the table is used - this object keeps references."""

    def __init__(self, weights, dtype=torch.float16, outs=None):
        packed0 = weights[0][0]
        _check_device(packed0)
        if outs is None:
            outs = [torch.empty(tuple(int(d) for d in qs.shape), dtype=dtype,
                                device=packed0.device) for _, qs in weights]
        self.weights, self.outs, self.dtype = list(weights), list(outs), dtype
        self._code = _code(dtype, (torch.float16, torch.bfloat16, torch.float32))
        arr = _descs(weights)
        lib = load()
        nbytes = lib.nf4_dequant_table_bytes(arr, len(weights))
        host = torch.empty(max(nbytes, 16), dtype=torch.uint8)
        ptrs = (ctypes.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
        blocks = ctypes.c_int64(0)
        check(lib.nf4_dequant_table_pack(arr, len(weights), ptrs, self._code, host.data_ptr(),
                                         nbytes, ctypes.byref(blocks)), "nf4_dequant_table_pack")
        self.blocks = int(blocks.value)
        self.table = host.to(packed0.device)
        self.refs = [w for pair in weights for w in pair]

    def run(self):
        check(load().nf4_dequant_table(self.table.data_ptr(), len(self.weights), self.blocks,
                                       self._code, stream_of(self.table)), "nf4_dequant_table")
        return self.outs


def _workspace(nbytes: int, device) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def _lora_array(loras):
    if not loras:
        return None, 0
    arr = (NF4Lora * len(loras))(*loras)
    return arr, len(loras)


def linear_fwd(x: torch.Tensor, weights, bias: torch.Tensor | None = None, loras=(),
               out: torch.Tensor | None = None, tile: int | None = None,
               splits: int = 1) -> torch.Tensor:
    """Y[M, sum rows] = x[M, K] @ W_stack^T (+ bias) (+ LoRA terms).  `loras`: NF4Lora structs
    whose pointers stay alive for the call (make_lora's structs hold their tensors; a struct
    built otherwise needs the caller to keep them).  `tile` (TILE_*) and `splits` pin the
    tiling; None lets the library choose."""
    _check_device(x, bias)
    dt = _code(x.dtype)
    m, k = x.shape
    n = sum(int(qs.shape[0]) for _, qs in weights)
    if out is None:
        out = torch.empty((m, n), dtype=x.dtype, device=x.device)
    arr = _descs(weights)
    lib = load()
    if tile is None:
        ws_bytes = lib.nf4_linear_fwd_workspace(m, arr, len(weights), dt)
    else:
        ws_bytes = 4 * splits * m * n if splits > 1 else 0
    ws = _workspace(ws_bytes, x.device)
    larr, nl = _lora_array(loras)
    args = (x.data_ptr() if m else None, m, x.stride(0), arr, len(weights),
            bias.data_ptr() if bias is not None else None, larr, nl, out.data_ptr(),
            out.stride(0), dt, ws.data_ptr() if ws is not None else None, ws_bytes, stream_of(x))
    if tile is None:
        check(lib.nf4_linear_fwd(*args), "nf4_linear_fwd")
    else:
        check(lib.nf4_linear_fwd_tiled(*args, int(tile), int(splits)), "nf4_linear_fwd_tiled")
    return out


def linear_dx(dy: torch.Tensor, weights, loras=(), out: torch.Tensor | None = None,
              accumulate: bool = False, tile: int | None = None,
              splits: int = 1) -> torch.Tensor:
    """dX[M, K] (+)= dY[M, sum rows] @ W_stack (+ LoRA terms); `tile` / `splits` as in
    linear_fwd."""
    _check_device(dy)
    dt = _code(dy.dtype)
    m = dy.shape[0]
    k = int(weights[0][1].shape[1])
    if out is None:
        out = torch.empty((m, k), dtype=dy.dtype, device=dy.device)
        accumulate = False
    offs = _offsets(weights)
    if tile is None and len(weights) > 1 and any(o % 8 for o in offs):
        return _linear_dx_by_segment(dy, weights, loras, out, accumulate, offs)
    arr = _descs(weights)
    lib = load()
    if tile is None:
        ws_bytes = lib.nf4_linear_dx_workspace(m, arr, len(weights), dt)
    else:
        ws_bytes = 4 * splits * m * k if splits > 1 else 0
    ws = _workspace(ws_bytes, dy.device)
    larr, nl = _lora_array(loras)
    args = (dy.data_ptr() if m else None, m, dy.stride(0), arr, len(weights), larr, nl,
            out.data_ptr(), out.stride(0), int(accumulate), dt,
            ws.data_ptr() if ws is not None else None, ws_bytes, stream_of(dy))
    if tile is None:
        check(lib.nf4_linear_dx(*args), "nf4_linear_dx")
    else:
        check(lib.nf4_linear_dx_tiled(*args, int(tile), int(splits)), "nf4_linear_dx_tiled")
    return out


def _offsets(weights):
    offs, o = [], 0
    for _, qs in weights:
        offs.append(o)
        o += int(qs.shape[0])
    return offs


def _linear_dx_by_segment(dy, weights, loras, out, accumulate, offs):
    """linear_dx over stacked segments of which one starts off a multiple of 8 dY columns: the
    stacked launch reads each segment's dY columns as 16-byte chunks, so each segment runs as
    its own launch over its dY columns (copied when they are not 16-byte aligned), the first
    writing dX and the others adding to it; a LoRA struct goes with its segment's launch."""
    by_seg = {}
    for lo in loras:
        by_seg.setdefault(int(lo.seg), []).append(lo)
    for i, (w, off) in enumerate(zip(weights, offs)):
        rows = int(w[1].shape[0])
        dy_s = dy[:, off: off + rows]
        if dy_s.data_ptr() % 16 or dy_s.stride(0) % 8:  # to rows of a multiple of 8 values
            pad = torch.empty((dy.shape[0], -(-rows // 8) * 8), dtype=dy.dtype, device=dy.device)
            pad[:, :rows].copy_(dy_s)
            dy_s = pad[:, :rows]
        seg_loras = [NF4Lora(seg=0, rank=lo.rank, scale=lo.scale, t=lo.t, b=lo.b, a=lo.a, da=lo.da)
                     for lo in by_seg.get(i, [])]
        linear_dx(dy_s, [w], seg_loras, out=out, accumulate=accumulate or i > 0)
    return out


def lora_xa(xd: torch.Tensor, a: torch.Tensor) -> torch.Tensor:
    """t[M, r] = xd[M, K] @ A[r, K]^T."""
    _check_device(xd, a)
    m, k = xd.shape
    r = a.shape[0]
    t = torch.empty((m, r), dtype=xd.dtype, device=xd.device)
    st = load().nf4_lora_xa(xd.data_ptr(), m, k, xd.stride(0), a.data_ptr(), r, t.data_ptr(),
                            _code(xd.dtype), stream_of(xd))
    check(st, "nf4_lora_xa")
    return t


def lora_da(dy: torch.Tensor, b: torch.Tensor, scale: float) -> torch.Tensor:
    """da[M, r] = scale * dY[M, N] @ B[N, r]  (dY may be a column slice: rows stride(0) apart)."""
    _check_device(dy, b)
    m, n = dy.shape
    r = b.shape[1]
    da = torch.empty((m, r), dtype=dy.dtype, device=dy.device)
    st = load().nf4_lora_da(dy.data_ptr(), m, n, dy.stride(0), b.data_ptr(), r, float(scale),
                            da.data_ptr(), _code(dy.dtype), stream_of(dy))
    check(st, "nf4_lora_da")
    return da


def lora_wgrad(u: torch.Tensor, v: torch.Tensor, scale: float, transpose_out: bool) -> torch.Tensor:
    """scale * U[M, P]^T @ V[M, r] in fp32: [P, r], or [r, P] when transpose_out."""
    _check_device(u, v)
    m, p = u.shape
    r = v.shape[1]
    out = torch.empty((r, p) if transpose_out else (p, r), dtype=torch.float32, device=u.device)
    lib = load()
    ws_bytes = lib.nf4_lora_wgrad_workspace(m, p, r)
    ws = _workspace(ws_bytes, u.device)
    st = lib.nf4_lora_wgrad(u.data_ptr() if m else None, m, p, u.stride(0),
                            v.data_ptr() if m else None, r, float(scale), out.data_ptr(),
                            int(transpose_out), _code(u.dtype),
                            ws.data_ptr() if ws is not None else None, ws_bytes, stream_of(u))
    check(st, "nf4_lora_wgrad")
    return out


def _pair(gate, up):
    if tuple(gate[1].shape) != tuple(up[1].shape):
        raise ValueError("gate and up weights must have the same shape")
    return _descs([gate, up])


def linear_swiglu_fwd(x: torch.Tensor, gate, up, out: torch.Tensor | None = None,
                      tile: int | None = None) -> torch.Tensor:
    """H[M, I] = silu(x @ Wg^T) * (x @ Wu^T), the SwiGLU step in the gate|up GEMM's epilogue.
    `gate`, `up`: (packed, quant_state) pairs of equal shape [I, K]; `tile` pins the tiling."""
    _check_device(x)
    m = x.shape[0]
    inter = int(gate[1].shape[0])
    if out is None:
        out = torch.empty((m, inter), dtype=x.dtype, device=x.device)
    arr = _pair(gate, up)
    if tile is not None:
        st = load().nf4_linear_swiglu_tiled(x.data_ptr() if m else None, m, x.stride(0), arr,
                                            out.data_ptr(), out.stride(0), None, 0,
                                            _code(x.dtype), stream_of(x), 0, int(tile))
        check(st, "nf4_linear_swiglu_tiled")
        return out
    st = load().nf4_linear_swiglu_fwd(x.data_ptr() if m else None, m, x.stride(0), arr,
                                      out.data_ptr(), out.stride(0), _code(x.dtype), stream_of(x))
    check(st, "nf4_linear_swiglu_fwd")
    return out


def linear_swiglu_bwd(x: torch.Tensor, gate, up, d_hidden: torch.Tensor,
                      out: torch.Tensor | None = None, tile: int | None = None) -> torch.Tensor:
    """dGU[M, 2I] (dgate | dup) from d_hidden [M, I] and gate/up recomputed from x inside the
    GEMM; the input of linear_dx over the stacked (gate, up) pair."""
    _check_device(x, d_hidden)
    m = x.shape[0]
    inter = int(gate[1].shape[0])
    if tuple(d_hidden.shape) != (m, inter) or d_hidden.stride(1) != 1:
        raise ValueError("d_hidden must be a row-contiguous [M, I] tensor")
    if out is None:
        out = torch.empty((m, 2 * inter), dtype=x.dtype, device=x.device)
    arr = _pair(gate, up)
    if tile is not None:
        st = load().nf4_linear_swiglu_tiled(x.data_ptr() if m else None, m, x.stride(0), arr,
                                            out.data_ptr(), out.stride(0), d_hidden.data_ptr(),
                                            d_hidden.stride(0), _code(x.dtype), stream_of(x), 1,
                                            int(tile))
        check(st, "nf4_linear_swiglu_tiled")
        return out
    st = load().nf4_linear_swiglu_bwd(x.data_ptr() if m else None, m, x.stride(0), arr,
                                      d_hidden.data_ptr(), d_hidden.stride(0), out.data_ptr(),
                                      out.stride(0), _code(x.dtype), stream_of(x))
    check(st, "nf4_linear_swiglu_bwd")
    return out


def swiglu_fwd(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up for two [M, I] views with equal row stride (e.g. halves of gate|up)."""
    _check_device(gate, up)
    rows, cols = gate.shape
    if up.stride(0) != gate.stride(0) or gate.stride(1) != 1 or up.stride(1) != 1:
        raise ValueError("gate and up must be row-contiguous views with one row stride")
    out = torch.empty((rows, cols), dtype=gate.dtype, device=gate.device)
    st = load().nf4_swiglu_fwd(gate.data_ptr(), up.data_ptr(), gate.stride(0), out.data_ptr(),
                               out.stride(0), rows, cols, _code(gate.dtype), stream_of(gate))
    check(st, "nf4_swiglu_fwd")
    return out


def swiglu_bwd(grad: torch.Tensor, gate: torch.Tensor, up: torch.Tensor,
               dgate: torch.Tensor, dup: torch.Tensor) -> None:
    """dgate, dup (row-strided like gate/up; may be gate/up themselves) from grad [M, I]."""
    _check_device(grad, gate, up)
    rows, cols = gate.shape
    st = load().nf4_swiglu_bwd(grad.data_ptr(), grad.stride(0), gate.data_ptr(), up.data_ptr(),
                               gate.stride(0), dgate.data_ptr(), dup.data_ptr(), rows, cols,
                               _code(gate.dtype), stream_of(gate))
    check(st, "nf4_swiglu_bwd")


def bias_grad(dy: torch.Tensor) -> torch.Tensor:
    """Column sums of dY [M, N] in fp32."""
    _check_device(dy)
    m, n = dy.shape
    out = torch.empty(n, dtype=torch.float32, device=dy.device)
    st = load().nf4_bias_grad(dy.data_ptr() if m else None, m, n, dy.stride(0), out.data_ptr(),
                              _code(dy.dtype), stream_of(dy))
    check(st, "nf4_bias_grad")
    return out


def _p(t):
    return None if t is None else t.data_ptr()


def _rows(t, cols):
    if t is not None and (t.dim() != 2 or t.shape[1] != cols or not t.is_contiguous()):
        raise ValueError("norm operands are contiguous [rows, cols] tensors")


def _gemm_dtype(x, *others, dtype=None):
    """The GEMM dtype of a norm call: `dtype`, else the first 16-bit operand's, else x's."""
    if dtype is None:
        for t in (*others, x):
            if t is not None and t.dtype in (torch.float16, torch.bfloat16):
                dtype = t.dtype
                break
    if dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("the norm kernels compute float16 or bfloat16 outputs")
    if x.dtype not in (dtype, torch.float32):
        raise ValueError("the residual stream x is float32 or the GEMM dtype")
    return dtype


def _as_u8(keep):
    keep = keep.contiguous()
    return keep.view(torch.uint8) if keep.dtype == torch.bool else keep.to(torch.uint8)


def add_rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, d: torch.Tensor | None = None,
                dtype=None, keep_q: torch.Tensor | None = None, keep_v: torch.Tensor | None = None,
                rows: torch.Tensor | None = None, packed: torch.Tensor | None = None,
                scale_q: float = 1.0, scale_v: float = 1.0):
    """RMSNorm of the residual stream x (+ d) (layer.py:92-132, 683-715): returns (y, rstd), y in
    the GEMM dtype (`dtype`, default d's or x's) and rstd fp32 [rows].  x is fp32 or the GEMM
    dtype, d the GEMM dtype.  With LoRA dropout also the dropout inputs y * keep * scale:
      keep_q, keep_v (bool or 0/1 uint8 [*, cols], read at row rows[r], or r when rows is None)
        -> (y, rstd, oq, ov, packed), packed the masks 8 per byte ([rows, 2 * cols / 8] uint8,
           q's bytes then v's; bit k of byte j = element 8 j + k);
      packed -> (y, rstd, oq, ov)."""
    _check_device(x, d, w, keep_q, keep_v, rows, packed)
    dtype = _gemm_dtype(x, d, dtype=dtype)
    n, cols = x.shape
    _rows(x, cols)
    _rows(d, cols)
    y = torch.empty((n, cols), dtype=dtype, device=x.device)
    rstd = torch.empty(n, dtype=torch.float32, device=x.device)
    w = w.to(torch.float32).contiguous()
    mode, oq, ov, kq, kv = 0, None, None, None, None
    if keep_q is not None:
        if keep_v is None or packed is not None:
            raise ValueError("give keep_q and keep_v (mode 1) or packed (mode 2)")
        kq, kv = _as_u8(keep_q), _as_u8(keep_v)
        if kq.shape[-1] != cols or kv.shape != kq.shape:
            raise ValueError("keep masks are [*, cols]")
        if rows is not None:
            rows = rows.to(torch.int64).contiguous()
            if rows.numel() != n:
                raise ValueError("rows holds one mask row per token")
        elif kq.shape[0] < n:
            raise ValueError("keep masks need a row per token")
        packed = torch.empty((n, 2 * (cols // 8)), dtype=torch.uint8, device=x.device)
        mode = 1
    elif packed is not None:
        if tuple(packed.shape) != (n, 2 * (cols // 8)) or packed.dtype != torch.uint8:
            raise ValueError("packed masks are uint8 [rows, 2 * cols / 8]")
        packed = packed.contiguous()
        mode = 2
    if mode:
        oq, ov = torch.empty_like(y), torch.empty_like(y)
    keep_rows = int(kq.shape[0]) if kq is not None else 0
    st = load().nf4_add_rmsnorm(_p(x), DTYPE_CODE[x.dtype], _p(d), _p(w), _p(y), _p(rstd), _p(kq),
                                _p(kv), _p(rows) if mode == 1 else None, keep_rows, _p(packed),
                                mode,
                                float(scale_q), float(scale_v), _p(oq), _p(ov), n, cols,
                                float(eps), _code(dtype), stream_of(x))
    check(st, "nf4_add_rmsnorm")
    if mode == 1:
        return y, rstd, oq, ov, packed
    if mode == 2:
        return y, rstd, oq, ov
    return y, rstd


def rmsnorm_bwd(x: torch.Tensor, w: torch.Tensor, rstd: torch.Tensor, dy=None, d=None, dres=None,
                dq=None, dv=None, packed=None, scale_q: float = 1.0, scale_v: float = 1.0,
                dtype=None) -> torch.Tensor:
    """dX of add_rmsnorm (layer.py:135-164, 718-730) from the output's gradient dy and LoRA's
    dropout branches dq, dv (masked with the packed keep bits of the forward), plus the
    residual gradient dres; dX and dres in x's dtype (fp32 for an fp32 residual stream), the
    other gradients in the GEMM dtype."""
    _check_device(x, w, rstd, dy, d, dres, dq, dv, packed)
    dtype = _gemm_dtype(x, dy, dq, d, dtype=dtype)
    n, cols = x.shape
    for t in (x, dy, d, dres, dq, dv):
        _rows(t, cols)
    if dres is not None and dres.dtype != x.dtype:
        raise ValueError("dres has the residual stream's dtype")
    if (dq is None) != (dv is None) or (dq is not None and packed is None):
        raise ValueError("dq and dv come together, with the packed masks")
    if packed is not None:
        if tuple(packed.shape) != (n, 2 * (cols // 8)) or packed.dtype != torch.uint8:
            raise ValueError("packed masks are uint8 [rows, 2 * cols / 8]")
        packed = packed.contiguous()
    dx = torch.empty_like(x)
    w = w.to(torch.float32).contiguous()
    st = load().nf4_rmsnorm_bwd(_p(dy), _p(dq), _p(dv), _p(packed), float(scale_q),
                                float(scale_v), _p(x), DTYPE_CODE[x.dtype], _p(d), _p(w), _p(rstd),
                                _p(dres), _p(dx), n, cols, _code(dtype), stream_of(x))
    check(st, "nf4_rmsnorm_bwd")
    return dx


def qkv_rope(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, n_heads: int, n_kv: int,
             head_dim: int, caches: bool = True):
    """(q, k, v[, k_cache, v_cache]) from the finished q|k|v projection [tokens, ...]: rotary
    embedding on q and k, k and v expanded to [tokens, n_heads, head_dim]."""
    _check_device(qkv, cos, sin)
    tokens = qkv.shape[0]
    if qkv.stride(1) != 1:
        raise ValueError("qkv rows must be contiguous")
    cos, sin = cos.to(torch.float32).contiguous(), sin.to(torch.float32).contiguous()
    e = lambda h: torch.empty(tokens, h, head_dim, dtype=qkv.dtype, device=qkv.device)  # noqa: E731
    q, k, v = e(n_heads), e(n_heads), e(n_heads)
    kc, vc = (e(n_kv), e(n_kv)) if caches else (None, None)
    st = load().nf4_qkv_rope(_p(qkv), qkv.stride(0), _p(cos), _p(sin), _p(q), _p(k), _p(v), _p(kc),
                             _p(vc), tokens, n_heads, n_kv, head_dim, _code(qkv.dtype),
                             stream_of(qkv))
    check(st, "nf4_qkv_rope")
    return (q, k, v, kc, vc) if caches else (q, k, v)


def qkv_rope_bwd(dq: torch.Tensor, dk: torch.Tensor, dv: torch.Tensor, cos: torch.Tensor,
                 sin: torch.Tensor, n_kv: int) -> torch.Tensor:
    """d(q|k|v) [tokens, (n_heads + 2 n_kv) head_dim] from the gradients of qkv_rope's q, k, v
    ([tokens, n_heads, head_dim] each)."""
    _check_device(dq, dk, dv, cos, sin)
    tokens, n_heads, head_dim = dq.shape
    for t in (dq, dk, dv):
        if tuple(t.shape) != (tokens, n_heads, head_dim) or not t.is_contiguous():
            raise ValueError("dq, dk, dv are contiguous [tokens, n_heads, head_dim] tensors")
    cos, sin = cos.to(torch.float32).contiguous(), sin.to(torch.float32).contiguous()
    out = torch.empty(tokens, (n_heads + 2 * n_kv) * head_dim, dtype=dq.dtype, device=dq.device)
    st = load().nf4_qkv_rope_bwd(_p(dq), _p(dk), _p(dv), _p(cos), _p(sin), _p(out), out.stride(0),
                                 tokens, n_heads, n_kv, head_dim, _code(dq.dtype), stream_of(dq))
    check(st, "nf4_qkv_rope_bwd")
    return out


def make_lora(seg: int, rank: int, scale: float, t=None, b=None, a=None, da=None) -> NF4Lora:
    """The adapter struct of segment `seg`.  It holds raw pointers, so it also keeps references
    to its tensors: a temporary passed here (t=lora_xa(...)) stays allocated while the struct
    lives, instead of returning to torch's cache where the call's own output could reuse it."""
    lo = NF4Lora(seg=seg, rank=rank, scale=float(scale),
                 t=t.data_ptr() if t is not None else None,
                 b=b.data_ptr() if b is not None else None,
                 a=a.data_ptr() if a is not None else None,
                 da=da.data_ptr() if da is not None else None)
    lo._tensors = (t, b, a, da)
    return lo


__all__ = ["dequant", "linear_fwd", "linear_dx", "lora_xa", "lora_da", "lora_wgrad",
           "swiglu_fwd", "swiglu_bwd", "bias_grad", "make_lora", "GEMM_DTYPES", "_lib"]


def lora_job(inp: torch.Tensor, w: torch.Tensor, out: torch.Tensor, scale: float = 1.0,
             transpose_out: bool = False) -> NF4LoraJob:
    """One job of the multi LoRA launches: `inp` [M, cols] (any row stride), `w` the small
    operand, `out` the result.  Like make_lora's struct, the job holds references to its
    tensors, so a temporary passed here stays allocated while the job lives."""
    _check_device(inp, w, out)
    job = NF4LoraJob(in_=inp.data_ptr(), ld=inp.stride(0), cols=inp.shape[1], w=w.data_ptr(),
                     out=out.data_ptr(), scale=float(scale), transpose_out=int(transpose_out))
    job._tensors = (inp, w, out)
    return job


def _jobs(jobs):
    return (NF4LoraJob * len(jobs))(*jobs), len(jobs)


def lora_xa_multi(jobs, m: int, rank: int, dtype, stream_tensor: torch.Tensor):
    """t_j = in_j @ A_j^T for every job, one launch."""
    arr, n = _jobs(jobs)
    check(load().nf4_lora_xa_multi(arr, n, m, rank, _code(dtype), stream_of(stream_tensor)),
          "nf4_lora_xa_multi")


def lora_da_multi(jobs, m: int, rank: int, dtype, stream_tensor: torch.Tensor):
    """da_j = scale_j * in_j @ B_j for every job, one launch."""
    arr, n = _jobs(jobs)
    check(load().nf4_lora_da_multi(arr, n, m, rank, _code(dtype), stream_of(stream_tensor)),
          "nf4_lora_da_multi")


def lora_ax_multi(jobs, m: int, rank: int, dtype, stream_tensor: torch.Tensor):
    """out_j = scale_j * da_j @ A_j ([M, K]) for every job (lora_ax_job), one launch."""
    arr, n = _jobs(jobs)
    check(load().nf4_lora_ax_multi(arr, n, m, rank, _code(dtype), stream_of(stream_tensor)),
          "nf4_lora_ax_multi")


def lora_ax_job(da: torch.Tensor, a: torch.Tensor, out: torch.Tensor, scale: float = 1.0):
    """A job of lora_ax_multi: da [M, rank] (any row stride), A [rank, K] contiguous, out
    [M, K] contiguous."""
    _check_device(da, a, out)
    if not a.is_contiguous() or not out.is_contiguous() or da.stride(-1) != 1:
        raise ValueError("lora_ax: A and out contiguous, da rows contiguous")
    if out.shape[1] != a.shape[1] or da.shape[1] != a.shape[0] or out.shape[0] != da.shape[0]:
        raise ValueError("lora_ax: da [M, r], A [r, K], out [M, K]")
    return NF4LoraJob(in_=da.data_ptr(), ld=da.stride(0), cols=a.shape[1], w=a.data_ptr(),
                      out=out.data_ptr(), scale=float(scale), transpose_out=0)


def lora_wgrad_multi(jobs, m: int, rank: int, dtype, stream_tensor: torch.Tensor):
    """out_j = scale_j * in_j^T @ V_j (fp32) for every job: one launch over M when the rows
    allow it, else row-chunk partials and a final pass through the workspace."""
    arr, n = _jobs(jobs)
    lib = load()
    nbytes = lib.nf4_lora_wgrad_multi_workspace(arr, n, m, rank)
    ws = _workspace(nbytes, stream_tensor.device)
    check(lib.nf4_lora_wgrad_multi(arr, n, m, rank, _code(dtype),
                                   ws.data_ptr() if ws is not None else None, nbytes,
                                   stream_of(stream_tensor)), "nf4_lora_wgrad_multi")


# ------------------------------------------------- int8 input gradients (off the parity path)

def int8_colscale(weights, dtype=torch.float16) -> torch.Tensor:
    """fp32 [cols]: max(largest |W[:, c]|, 1e-20) / 127 over the stacked weights, W rounded to
    `dtype` (the fixed column scales of the transposed int8 weights)."""
    arr = _descs(weights)
    lib = load()
    dev = weights[0][0].device
    cols = int(weights[0][1].shape[1])
    out = torch.empty(cols, dtype=torch.float32, device=dev)
    nb = lib.nf4_int8_colscale_workspace(arr, len(weights))
    ws = _workspace(nb, dev)
    check(lib.nf4_int8_colscale(arr, len(weights), out.data_ptr(), _code(dtype),
                                ws.data_ptr() if ws is not None else None, nb, stream_of(out)),
          "nf4_int8_colscale")
    return out


def int8_weight_t(weights, scale: torch.Tensor) -> torch.Tensor:
    """int8 [cols, sum rows]: the stacked weights transposed, divided by the column scales."""
    arr = _descs(weights)
    rows = sum(int(qs.shape[0]) for _, qs in weights)
    cols = int(weights[0][1].shape[1])
    q = torch.empty((cols, rows), dtype=torch.int8, device=scale.device)
    check(load().nf4_int8_weight_t(arr, len(weights), scale.data_ptr(), q.data_ptr(), rows,
                                   stream_of(q)), "nf4_int8_weight_t")
    return q


def int8_weight_rows(weights):
    """(int8 [sum rows, cols], fp32 [sum rows]): the stacked weights with one scale per row."""
    arr = _descs(weights)
    rows = sum(int(qs.shape[0]) for _, qs in weights)
    cols = int(weights[0][1].shape[1])
    dev = weights[0][0].device
    q = torch.empty((rows, cols), dtype=torch.int8, device=dev)
    s = torch.empty(rows, dtype=torch.float32, device=dev)
    check(load().nf4_int8_weight_rows(arr, len(weights), q.data_ptr(), cols, s.data_ptr(),
                                      stream_of(q)), "nf4_int8_weight_rows")
    return q, s


def int8_rows(x: torch.Tensor):
    """(int8 [M, N], fp32 [M]): one int8 row per row of x with scale largest |x| / 127."""
    _check_device(x)
    m, n = x.shape
    q = torch.empty((m, n), dtype=torch.int8, device=x.device)
    s = torch.empty(m, dtype=torch.float32, device=x.device)
    code = _code(x.dtype, (torch.float16, torch.bfloat16, torch.float32))
    check(load().nf4_int8_rows(x.data_ptr() if m else None, m, n, x.stride(0), q.data_ptr(), n,
                               s.data_ptr(), code, stream_of(x)), "nf4_int8_rows")
    return q, s


def int8_gemm(a: torch.Tensor, b: torch.Tensor, sa: torch.Tensor | None = None,
              sb: torch.Tensor | None = None, out_dtype=None) -> torch.Tensor:
    """a [M, K] . b [N, K]^T over int8: int32 sums (out_dtype None) or
    round(fp32(C) * sa[m] * sb[n]) in out_dtype (float16 / bfloat16)."""
    _check_device(a, b)
    m, k = a.shape
    n = b.shape[0]
    lib = load()
    if out_dtype is None:
        out = torch.empty((m, n), dtype=torch.int32, device=a.device)
        code = _lib.NF4_I32
    else:
        out = torch.empty((m, n), dtype=out_dtype, device=a.device)
        code = _code(out_dtype)
    nb = lib.nf4_int8_gemm_workspace(m, n, k)
    ws = _workspace(nb, a.device)
    check(lib.nf4_int8_gemm(a.data_ptr(), m, a.stride(0), b.data_ptr(), n, b.stride(0), k,
                            sa.data_ptr() if sa is not None else None,
                            sb.data_ptr() if sb is not None else None, out.data_ptr(),
                            out.stride(0), code, ws.data_ptr() if ws is not None else None, nb,
                            stream_of(a)), "nf4_int8_gemm")
    return out


def int8_swiglu_bwd(acc: torch.Tensor, sd: torch.Tensor, cs: torch.Tensor,
                    gu: torch.Tensor):
    """(int8 [M, 2I], fp32 [M]): SwiGLU backward of the int32 sums acc [M, I] (scaled by
    sd[m] cs[j]) with the saved gate | up [M, 2I], requantized with one scale per row."""
    _check_device(acc, sd, cs, gu)
    m, inter = acc.shape
    q = torch.empty((m, 2 * inter), dtype=torch.int8, device=acc.device)
    sq = torch.empty(m, dtype=torch.float32, device=acc.device)
    check(load().nf4_int8_swiglu_bwd(acc.data_ptr(), m, inter, acc.stride(0), sd.data_ptr(),
                                     cs.data_ptr(), gu.data_ptr(), gu.stride(0), q.data_ptr(),
                                     2 * inter, sq.data_ptr(), _code(gu.dtype), stream_of(acc)),
          "nf4_int8_swiglu_bwd")
    return q, sq
