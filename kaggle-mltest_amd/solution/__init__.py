"""MI355X-native NF4 quantized-linear path, behind the reference's plugin surface.

`apply()` installs the same patches as the NF4 part of /root/reference/solution/__init__.py:56-112
(lines 94-99 there): `patch_qwen2_mlp_recompute`, `patch_bnb_matmul_4bit`, `patch_linear4bit`.
Each runs under `_try`, which logs a failure and never raises (__init__.py:49-53): without
bitsandbytes - absent on this machine - the patches report that and the process goes on.

The compute path is libnf4_mi355x.so (hand-written HIP for gfx950) through ctypes; see
`kernels` for the tensor-level calls and `nf4`, `layer`, `mlp` for the reference's operators.
"""

from __future__ import annotations

import sys
import time

_T0 = time.perf_counter()


def since_start():
    """Seconds since this package was imported."""
    return time.perf_counter() - _T0


def mark(what):
    print(f"[solution] t+{since_start():6.2f} s since import  {what}", file=sys.stderr, flush=True)


def _try(name, patch):
    """Run one patch; a failure is logged, never raised."""
    try:
        patch()
        return True
    except Exception as exc:  # noqa: BLE001 - a missing piece must not stop the run
        print(f"[solution] {name} not applied: {exc.__class__.__name__}: {exc}", file=sys.stderr)
        return False


def apply():
    """Install the NF4 patches.  Returns {patch name: applied?}."""
    mark("apply() starts")
    from .mlp import patch_qwen2_mlp_recompute
    from .nf4 import patch_bnb_matmul_4bit, patch_linear4bit

    done = {
        "MLP recomputing its activations": _try("MLP recomputing its activations",
                                                patch_qwen2_mlp_recompute),
        "NF4 dequantization": _try("NF4 dequantization", patch_bnb_matmul_4bit),
        "4-bit linear layers in fp16": _try("4-bit linear layers in fp16", patch_linear4bit),
    }
    mark("apply() done")
    return done
