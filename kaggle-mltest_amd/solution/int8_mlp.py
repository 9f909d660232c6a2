"""int8 GEMMs of the SwiGLU MLP on gfx950 int8 MFMA: the reference's T4 int8 backward
(/root/reference/solution/layer.py:515-618, 992-1013) and its int8 gate|up forward (layer.py:
900-912, off by default there: `INT8_FORWARD`), kept off the fp16 parity path and held to the
reference's own int8 tolerance (test_kernels.py:323-357).

Forward (gate_up_fwd_int8):

    y2 [n, H] -> int8 rows x8, sx                          (row_quant, layer.py:555-562)
    W_gate|up -> int8 rows w8, sw (one scale per row)       (_int8_rows, layer.py:565-576)
    gu = round(fp32(x8 . w8^T) * sx[m] * sw[j])  [n, 2I]    (gate_up_act_fwd_i8_kernel)
    act = silu(gate) * up from the rounded halves, rounded once

Input gradient (mlp_input_grad_int8):

    dh2 [n, H]  -> int8 rows dh8, sdh                       (row_quant, layer.py:555-562)
    acc = dh8 . Wd8^T        int32 [n, I]                   (layer.py:1003)
          Wd8 = W_down transposed to int8 with the fixed column scales cs_d
    q8, sq = SwiGLU backward of acc * sdh * cs_d on the saved gate | up, int8 per row
                                                            (gate_up_act_bwd_i8_kernel)
    dy2 = fp32(q8 . Wgu8^T) * sq * cs_gu  -> GEMM dtype     (layer.py:1008-1012)

Column scales are computed once per MLP (the reference caches them per module for the run,
layer.py:598-615); the int8 weights are made from the NF4 bytes at each use, as the fp16 ones
are.  The reference splits the first GEMM into 512-token chunks to bound a 15 GB GPU's memory;
one launch covers every token here (the scaled product is written in the GEMM dtype, no int32
buffer).  RecomputedMLP's forward takes the int8 gate|up path when `mlp.INT8_FORWARD` is set,
its backward the int8 input gradients when `mlp.INT8_BACKWARD` is set."""

from __future__ import annotations

import torch

from . import kernels


def int8_eligible(hidden: int, inter: int, blocksize: int) -> bool:
    """Shapes the int8 kernels tile exactly (layer.py:538-548)."""
    return hidden % 128 == 0 and inter % 128 == 0 and 128 % blocksize == 0


class ColumnScales:
    """Per-MLP cache of (cs_gu, cs_d), keyed by the packed weight tensors."""

    def __init__(self):
        self._cache = {}

    def get(self, gate, up, down, dtype=torch.float16):
        key = (gate[0].data_ptr(), up[0].data_ptr(), down[0].data_ptr(), dtype)
        hit = self._cache.get(key)
        if hit is None:
            hit = (kernels.int8_colscale([gate, up], dtype), kernels.int8_colscale([down], dtype))
            self._cache[key] = hit
        return hit


def gate_up_fwd_int8(y2: torch.Tensor, gate, up, dtype=None) -> tuple:
    """(gu [n, 2I], act [n, I]) in dtype (y2's by default): the gate|up product of y2 [n, H]
    through one int8 GEMM with per-token and per-weight-row scales, and silu(gate) * up
    (layer.py:900-912).  gate, up: (packed, quant_state)."""
    dtype = dtype or y2.dtype
    inter = int(gate[1].shape[0])
    hidden = int(gate[1].shape[1])
    if not int8_eligible(hidden, inter, int(gate[1].blocksize)):
        raise ValueError(f"the int8 gate|up forward needs hidden and inter multiples of 128 "
                         f"(got {hidden}, {inter}) and a block size dividing 128")
    x8, sx = kernels.int8_rows(y2)
    w8, sw = kernels.int8_weight_rows([gate, up])
    gu = kernels.int8_gemm(x8, w8, sx, sw, out_dtype=dtype)
    del x8, w8
    return gu, kernels.swiglu_fwd(gu[:, :inter], gu[:, inter:])


def mlp_input_grad_int8(dh2: torch.Tensor, gu: torch.Tensor, gate, up, down,
                        scales: tuple | None = None, dtype=None) -> torch.Tensor:
    """dy2 [n, H] = d(down(silu(g) u)) / dx for the gradient dh2 [n, H] at the MLP output, the
    saved gate | up product gu [n, 2I] and the NF4 weights (packed, quant_state), through two
    int8 GEMMs.  `scales`: (cs_gu, cs_d) from ColumnScales (computed here when None)."""
    dtype = dtype or gu.dtype
    inter = int(gate[1].shape[0])
    hidden = int(gate[1].shape[1])
    if not int8_eligible(hidden, inter, int(gate[1].blocksize)):
        raise ValueError(f"int8 input gradients need hidden and inter multiples of 128 "
                         f"(got {hidden}, {inter}) and a block size dividing 128")
    cs_gu, cs_d = scales if scales is not None else (kernels.int8_colscale([gate, up], dtype),
                                                      kernels.int8_colscale([down], dtype))
    dh8, sdh = kernels.int8_rows(dh2)
    acc = kernels.int8_gemm(dh8, kernels.int8_weight_t([down], cs_d))
    q8, sq = kernels.int8_swiglu_bwd(acc, sdh, cs_d, gu)
    return kernels.int8_gemm(q8, kernels.int8_weight_t([gate, up], cs_gu), sq, cs_gu,
                             out_dtype=dtype)


__all__ = ["int8_eligible", "ColumnScales", "gate_up_fwd_int8", "mlp_input_grad_int8"]
