"""ctypes binding of libnf4_mi355x.so (C ABI in include/nf4_mi355x.h).

The library is the only compute path: when it is missing or fails to load, every call raises
`NF4LibraryError` - there is no CPU or PyTorch fallback behind it.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import c_float, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

import torch

LIB_PATH = Path(__file__).with_name("libnf4_mi355x.so")

NF4_OK, NF4_ERR_ARG, NF4_ERR_UNSUPPORTED, NF4_ERR_LAUNCH, NF4_ERR_WORKSPACE = range(5)
NF4_F16, NF4_BF16, NF4_F32, NF4_I32 = 0, 1, 2, 3
NF4_MAX_SEGMENTS = 8

DTYPE_CODE = {torch.float16: NF4_F16, torch.bfloat16: NF4_BF16, torch.float32: NF4_F32}


class NF4LibraryError(RuntimeError):
    """The HIP library is missing, failed to load, or returned an error status."""


class NF4Unsupported(NF4LibraryError):
    """The library does not cover this layout or shape (status NF4_ERR_UNSUPPORTED)."""


class NF4Weight(ctypes.Structure):
    _fields_ = [
        ("packed", c_void_p), ("absmax", c_void_p), ("absmax2", c_void_p), ("code2", c_void_p),
        ("code", c_void_p), ("offset", c_float), ("nested", c_int32), ("rows", c_int64),
        ("cols", c_int64), ("blocksize", c_int32), ("blocksize2", c_int32),
    ]


class NF4Lora(ctypes.Structure):
    _fields_ = [
        ("seg", c_int32), ("rank", c_int32), ("scale", c_float), ("t", c_void_p), ("b", c_void_p),
        ("a", c_void_p), ("da", c_void_p),
    ]


# name -> (restype, argtypes)
class NF4LoraJob(ctypes.Structure):
    """struct nf4_lora_job (include/nf4_mi355x.h), 48 bytes."""
    _fields_ = [
        ("in_", c_void_p), ("ld", c_int64), ("cols", c_int64), ("w", c_void_p), ("out", c_void_p),
        ("scale", c_float), ("transpose_out", ctypes.c_int32),
    ]


_SIGNATURES = {
    "nf4_abi_version": (c_int, []),
    "nf4_status_string": (ctypes.c_char_p, [c_int]),
    "nf4_dequant": (c_int, [ctypes.POINTER(NF4Weight), c_void_p, c_int, c_void_p]),
    "nf4_dequant_multi": (c_int, [ctypes.POINTER(NF4Weight), c_int, c_void_p, c_int, c_void_p]),
    "nf4_dequant_batch": (c_int, [ctypes.POINTER(NF4Weight), c_int, ctypes.POINTER(c_void_p),
                                  c_int, c_void_p]),
    "nf4_dequant_table_bytes": (c_size_t, [ctypes.POINTER(NF4Weight), c_int]),
    "nf4_dequant_table_pack": (c_int, [ctypes.POINTER(NF4Weight), c_int, ctypes.POINTER(c_void_p),
                                       c_int, c_void_p, c_size_t, ctypes.POINTER(c_int64)]),
    "nf4_dequant_table": (c_int, [c_void_p, c_int, c_int64, c_int, c_void_p]),
    "nf4_linear_fwd": (c_int, [c_void_p, c_int64, c_int64, ctypes.POINTER(NF4Weight), c_int,
                               c_void_p, ctypes.POINTER(NF4Lora), c_int, c_void_p, c_int64, c_int,
                               c_void_p, c_size_t, c_void_p]),
    "nf4_linear_fwd_workspace": (c_size_t, [c_int64, ctypes.POINTER(NF4Weight), c_int, c_int]),
    "nf4_linear_dx": (c_int, [c_void_p, c_int64, c_int64, ctypes.POINTER(NF4Weight), c_int,
                              ctypes.POINTER(NF4Lora), c_int, c_void_p, c_int64, c_int, c_int,
                              c_void_p, c_size_t, c_void_p]),
    "nf4_linear_dx_workspace": (c_size_t, [c_int64, ctypes.POINTER(NF4Weight), c_int, c_int]),
    "nf4_linear_dx_noalloc": (c_int, [c_void_p, c_int64, c_int64, ctypes.POINTER(NF4Weight),
                                      c_int, ctypes.POINTER(NF4Lora), c_int, c_void_p, c_int64,
                                      c_int, c_int, c_void_p]),
    "nf4_linear_fwd_tiled": (c_int, [c_void_p, c_int64, c_int64, ctypes.POINTER(NF4Weight), c_int,
                                     c_void_p, ctypes.POINTER(NF4Lora), c_int, c_void_p, c_int64,
                                     c_int, c_void_p, c_size_t, c_void_p, c_int, c_int]),
    "nf4_linear_dx_tiled": (c_int, [c_void_p, c_int64, c_int64, ctypes.POINTER(NF4Weight), c_int,
                                    ctypes.POINTER(NF4Lora), c_int, c_void_p, c_int64, c_int,
                                    c_int, c_void_p, c_size_t, c_void_p, c_int, c_int]),
    "nf4_linear_swiglu_fwd": (c_int, [c_void_p, c_int64, c_int64, ctypes.POINTER(NF4Weight),
                                      c_void_p, c_int64, c_int, c_void_p]),
    "nf4_linear_swiglu_bwd": (c_int, [c_void_p, c_int64, c_int64, ctypes.POINTER(NF4Weight),
                                      c_void_p, c_int64, c_void_p, c_int64, c_int, c_void_p]),
    "nf4_linear_swiglu_tiled": (c_int, [c_void_p, c_int64, c_int64, ctypes.POINTER(NF4Weight),
                                        c_void_p, c_int64, c_void_p, c_int64, c_int, c_void_p,
                                        c_int, c_int]),
    "nf4_lora_xa": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int, c_void_p, c_int,
                            c_void_p]),
    "nf4_lora_da": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int, c_float,
                            c_void_p, c_int, c_void_p]),
    "nf4_lora_wgrad": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int, c_float,
                               c_void_p, c_int, c_int, c_void_p, c_size_t, c_void_p]),
    "nf4_lora_wgrad_workspace": (c_size_t, [c_int64, c_int64, c_int]),
    "nf4_lora_xa_multi": (c_int, [ctypes.POINTER(NF4LoraJob), c_int, c_int64, c_int, c_int,
                                  c_void_p]),
    "nf4_lora_da_multi": (c_int, [ctypes.POINTER(NF4LoraJob), c_int, c_int64, c_int, c_int,
                                  c_void_p]),
    "nf4_lora_ax_multi": (c_int, [ctypes.POINTER(NF4LoraJob), c_int, c_int64, c_int, c_int,
                                  c_void_p]),
    "nf4_lora_wgrad_multi": (c_int, [ctypes.POINTER(NF4LoraJob), c_int, c_int64, c_int, c_int,
                                     c_void_p, c_size_t, c_void_p]),
    "nf4_lora_wgrad_multi_workspace": (c_size_t, [ctypes.POINTER(NF4LoraJob), c_int, c_int64,
                                                  c_int]),
    "nf4_swiglu_fwd": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64,
                               c_int, c_void_p]),
    "nf4_swiglu_bwd": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p,
                               c_void_p, c_int64, c_int64, c_int, c_void_p]),
    "nf4_bias_grad": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int, c_void_p]),
    "nf4_int8_colscale_workspace": (c_size_t, [ctypes.POINTER(NF4Weight), c_int]),
    "nf4_int8_colscale": (c_int, [ctypes.POINTER(NF4Weight), c_int, c_void_p, c_int, c_void_p,
                                  c_size_t, c_void_p]),
    "nf4_int8_weight_t": (c_int, [ctypes.POINTER(NF4Weight), c_int, c_void_p, c_void_p, c_int64,
                                  c_void_p]),
    "nf4_int8_weight_rows": (c_int, [ctypes.POINTER(NF4Weight), c_int, c_void_p, c_int64,
                                     c_void_p, c_void_p]),
    "nf4_int8_rows": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p,
                              c_int, c_void_p]),
    "nf4_int8_gemm_workspace": (c_size_t, [c_int64, c_int64, c_int64]),
    "nf4_int8_gemm": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_int64,
                              c_void_p, c_void_p, c_void_p, c_int64, c_int, c_void_p, c_size_t,
                              c_void_p]),
    "nf4_int8_swiglu_bwd": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p,
                                    c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int,
                                    c_void_p]),
    "nf4_add_rmsnorm": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int, c_float,
                                c_float, c_void_p, c_void_p, c_int64, c_int64, c_float, c_int,
                                c_void_p]),
    "nf4_rmsnorm_bwd": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_float,
                                c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                c_void_p, c_int64, c_int64, c_int, c_void_p]),
    "nf4_qkv_rope": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                             c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_int, c_void_p]),
    "nf4_qkv_rope_bwd": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                 c_int64, c_int64, c_int, c_int, c_int, c_int, c_void_p]),
}

EXPORTS = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib = None


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """The loaded library (once per process).  Raises NF4LibraryError when it cannot load."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise NF4LibraryError(
                f"{p} is missing: build it with `python kaggle-mltest_amd/build.py` "
                "(the NF4 path has no fallback)")
        try:
            lib = ctypes.CDLL(str(p))
        except OSError as exc:
            raise NF4LibraryError(f"cannot load {p}: {exc}") from exc
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


def check(status: int, what: str) -> None:
    if status == NF4_OK:
        return
    text = load().nf4_status_string(status).decode()
    cls = NF4Unsupported if status == NF4_ERR_UNSUPPORTED else NF4LibraryError
    raise cls(f"{what}: {text} (status {status})")


def stream_of(t: torch.Tensor) -> int:
    """The handle of torch's current stream on `t`'s device (what every launch goes to)."""
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
