"""NF4 weights on disk: bitsandbytes' serialized QuantState layout, so that a pre-quantized
checkpoint loads straight into this package's kernel input format (packed bytes + uint8 absmax +
fp32 absmax2 + code maps + offset) and a weight quantized here saves in the same layout.

The format is bitsandbytes 0.50.2's (`QuantState.as_dict(packed=True)` /
`QuantState.from_dict`, and `Linear4bit._save_to_state_dict`, which stores every item under
`<module>.weight.<key>`); bitsandbytes is not installed here, so this is a restatement of its
published layout, not checked against a file bitsandbytes wrote:

  <prefix>weight                                    uint8 [ceil(N*K/2), 1]   packed codes
  <prefix>weight.absmax                             uint8 [blocks] (nested) or fp32 [blocks]
  <prefix>weight.quant_map                          fp32 [16]                NF4 code
  <prefix>weight.nested_absmax                      fp32 [ceil(blocks/256)]  (nested only)
  <prefix>weight.nested_quant_map                   fp32 [256]               (nested only)
  <prefix>weight.quant_state.bitsandbytes__nf4      uint8 [n]: UTF-8 JSON of quant_type,
      blocksize, dtype, shape, and when nested: nested_blocksize, nested_dtype, nested_offset

The reference never serializes weights itself: it quantizes at load time through
bitsandbytes and keeps host copies for streaming (/root/reference/solution/offload.py:93-136).
"""

from __future__ import annotations

import json

import torch

from .quant_state import QuantState

_PACKED_PREFIX = "quant_state.bitsandbytes__"
_KEYS = {"absmax", "quant_map", "nested_absmax", "nested_quant_map", "quant_type", "blocksize",
         "dtype", "shape", "nested_blocksize", "nested_dtype", "nested_offset"}


def _dtype_name(dtype) -> str:
    return str(dtype).split(".")[-1]


def _dtype(name: str):
    dt = getattr(torch, name, None)
    if not isinstance(dt, torch.dtype):
        raise ValueError(f"unknown dtype {name!r} in a serialized QuantState")
    return dt


def as_dict(qs: QuantState, packed: bool = False) -> dict:
    """The items bitsandbytes' QuantState.as_dict gives: tensors and plain values, or with
    `packed` the tensors plus one uint8 tensor holding the plain values as JSON."""
    d = {"quant_type": qs.quant_type, "absmax": qs.absmax, "blocksize": int(qs.blocksize),
         "quant_map": qs.code, "dtype": _dtype_name(qs.dtype),
         "shape": [int(v) for v in qs.shape] if qs.shape is not None else None}
    if qs.nested:
        d.update({"nested_absmax": qs.state2.absmax, "nested_blocksize": int(qs.state2.blocksize),
                  "nested_quant_map": qs.state2.code, "nested_dtype": _dtype_name(qs.state2.dtype),
                  "nested_offset": float(qs.offset)})
    if not packed:
        return d
    tensors = {k: v for k, v in d.items() if isinstance(v, torch.Tensor)}
    plain = {k: v for k, v in d.items() if not isinstance(v, torch.Tensor)}
    blob = json.dumps(plain).encode("utf-8")
    tensors[_PACKED_PREFIX + str(qs.quant_type)] = torch.tensor(list(blob), dtype=torch.uint8)
    return tensors


def from_dict(items: dict, device="cpu") -> QuantState:
    """A QuantState from as_dict items, packed or not, keys with or without a module prefix
    (bitsandbytes' QuantState.from_dict)."""
    items = dict(items)
    blobs = [k for k, v in items.items() if _PACKED_PREFIX in k and isinstance(v, torch.Tensor)]
    if len(blobs) > 1:
        raise ValueError(f"more than one packed quant-state entry: {blobs}")
    if blobs:
        key = blobs[0]
        if key.rsplit("__", 1)[-1] != "nf4":
            raise ValueError(f"only NF4 quant states are supported, found {key!r}")
        items.update(json.loads(bytes(items.pop(key).cpu().tolist()).decode("utf-8")))
    elif "quant_type" not in items:
        raise ValueError("no quant-state items: expected the packed JSON entry or quant_type")
    items = {k.split(".")[-1]: v for k, v in items.items()}
    unknown = set(items) - _KEYS
    if unknown:
        raise ValueError(f"unexpected quant-state items {sorted(unknown)}")
    if items["quant_type"] != "nf4":
        raise ValueError(f"only NF4 quant states are supported, found {items['quant_type']!r}")
    offset = state2 = None
    if "nested_absmax" in items:
        offset = torch.tensor(float(items["nested_offset"]), dtype=torch.float32, device=device)
        state2 = QuantState(absmax=items["nested_absmax"].to(device),
                            code=items["nested_quant_map"].to(device),
                            blocksize=int(items["nested_blocksize"]),
                            dtype=_dtype(items["nested_dtype"]))
    shape = torch.Size(items["shape"]) if items.get("shape") is not None else None
    return QuantState(absmax=items["absmax"].to(device), shape=shape,
                      code=items["quant_map"].to(device), blocksize=int(items["blocksize"]),
                      quant_type="nf4", dtype=_dtype(items["dtype"]), offset=offset,
                      state2=state2)


def state_dict_items(prefix: str, packed: torch.Tensor, qs: QuantState) -> dict:
    """The tensors Linear4bit stores for one weight under module prefix `prefix` (with its
    trailing dot): `<prefix>weight` and `<prefix>weight.<item>`."""
    out = {prefix + "weight": packed.reshape(-1, 1)}
    for k, v in as_dict(qs, packed=True).items():
        out[prefix + "weight." + k] = v
    return out


def load_weight(tensors: dict, prefix: str, device="cpu") -> tuple[torch.Tensor, QuantState]:
    """(packed flat uint8 on `device`, QuantState) of the weight stored under `prefix`."""
    base = prefix + "weight"
    if base not in tensors:
        raise KeyError(base)
    items = {k[len(base) + 1:]: v for k, v in tensors.items() if k.startswith(base + ".")}
    qs = from_dict(items, device)
    packed = tensors[base].to(device).reshape(-1).contiguous()
    n = int(qs.shape[0]) * int(qs.shape[1])
    if packed.dtype != torch.uint8 or packed.numel() != (n + 1) // 2:
        raise ValueError(f"{base}: {packed.numel()} packed bytes for a {tuple(qs.shape)} weight")
    return packed, qs


def save_safetensors(path, weights: dict) -> None:
    """Write {module prefix: (packed, QuantState)} as a safetensors file in the layout above."""
    from safetensors.torch import save_file

    tensors = {}
    for prefix, (packed, qs) in weights.items():
        for k, v in state_dict_items(prefix, packed, qs).items():
            tensors[k] = v.detach().to("cpu").contiguous()
    save_file(tensors, str(path))


def load_safetensors(path, device="cpu") -> dict:
    """{module prefix: (packed, QuantState)} of every NF4 weight in a safetensors file."""
    from safetensors.torch import load_file

    tensors = load_file(str(path))
    prefixes = sorted(k[:-len("weight")] for k in tensors
                      if k.endswith("weight") and k + "." + _PACKED_PREFIX + "nf4" in tensors)
    return {p: load_weight(tensors, p, device) for p in prefixes}


__all__ = ["as_dict", "from_dict", "state_dict_items", "load_weight", "save_safetensors",
           "load_safetensors"]
