"""Shared helpers of the GPU parity tests: move oracle states to the device and back."""

import numpy as np
import torch

from oracle import nf4_oracle as o


def to_device_state(packed: np.ndarray, st: "o.OracleQuantState", dev):
    """(packed uint8 tensor, solution QuantState) on `dev` from an oracle state."""
    from solution.quant_state import QuantState

    p = torch.from_numpy(np.ascontiguousarray(packed)).to(dev)
    code = torch.from_numpy(st.code).to(dev)
    if st.nested:
        s2 = QuantState(absmax=torch.from_numpy(st.state2.absmax).to(dev),
                        code=torch.from_numpy(st.state2.code).to(dev), blocksize=256,
                        dtype=torch.float32)
        qs = QuantState(absmax=torch.from_numpy(st.absmax).to(dev), shape=torch.Size(st.shape),
                        code=code, blocksize=st.blocksize, quant_type="nf4",
                        dtype=torch.float16, offset=torch.tensor(st.offset, dtype=torch.float32),
                        state2=s2)
    else:
        qs = QuantState(absmax=torch.from_numpy(st.absmax).to(dev), shape=torch.Size(st.shape),
                        code=code, blocksize=st.blocksize, quant_type="nf4", dtype=torch.float16)
    return p, qs


def to_oracle_state(packed: torch.Tensor, qs) -> tuple:
    """(packed numpy, OracleQuantState) from a device state."""
    if qs.nested:
        st = o.OracleQuantState(
            absmax=qs.absmax.cpu().numpy(), shape=tuple(qs.shape), code=qs.code.cpu().numpy(),
            blocksize=int(qs.blocksize), offset=float(qs.offset), nested=True,
            state2=o.OracleState2(absmax=qs.state2.absmax.cpu().numpy(),
                                  code=qs.state2.code.cpu().numpy()))
    else:
        st = o.OracleQuantState(absmax=qs.absmax.cpu().numpy(), shape=tuple(qs.shape),
                                code=qs.code.cpu().numpy(), blocksize=int(qs.blocksize))
    return packed.reshape(-1).cpu().numpy(), st


def random_weight(n, k, seed, dev, std=0.02, blocksize=64, nested=True):
    """A seeded N(0, std) [n, k] weight quantized to NF4 on `dev` (product quantizer)."""
    from solution.quant_state import quantize_4bit

    g = torch.Generator().manual_seed(seed)
    w = torch.randn(n, k, generator=g) * std
    packed, qs = quantize_4bit(w.to(dev), blocksize=blocksize, compress_statistics=nested)
    return packed.view(-1), qs


def oracle_w16(packed, qs, dtype="f16"):
    p, st = to_oracle_state(packed, qs)
    w = o.dequantize(p, st, dtype)
    if dtype == "bf16":
        return torch.from_numpy(w.view(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(w)


def assert_rel(out, ref, max_rel=1e-2, mean_rel=1e-3, what=""):
    """The path's tolerance.  fp16 (the contract): max rel <= 1e-2, mean rel <= 1e-3.  A bf16
    output's own rounding (8 significant bits) already gives mean rel ~1.4e-3, so bf16 results
    are held to mean rel <= 3e-3 (max rel unchanged)."""
    if getattr(out, "dtype", None) == torch.bfloat16:
        mean_rel = max(mean_rel, 3e-3)
    mx, mean = o.rel_errors(out, ref)
    assert mx <= max_rel and mean <= mean_rel, f"{what}: max rel {mx:.3e}, mean rel {mean:.3e}"
    return mx, mean


def banner(*parts):
    print("[case]", *parts, flush=True)
