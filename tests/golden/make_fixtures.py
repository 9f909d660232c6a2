"""Writes tests/golden/nf4_fixtures.npz: small seeded NF4 QuantStates in bitsandbytes layout
with their expected dequantized weights and GEMM results, all from the CPU oracle.

The reference holds no golden vectors of its own for this path (its tests generate inputs from
seeds and compare against bitsandbytes at run time, solution/test_kernels.py:41-75), so these
fixtures freeze the oracle's outputs: a later change to the oracle or to a kernel that moves a
single bit shows against them.  Run: `python tests/golden/make_fixtures.py`.
"""

from pathlib import Path
import sys

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import nf4_oracle as o  # noqa: E402

OUT = Path(__file__).with_name("nf4_fixtures.npz")

CASES = [
    # name, shape, seed, blocksize, nested
    ("w128x256", (128, 256), 11, 64, True),
    ("w64x1536", (64, 1536), 12, 64, True),
    ("w48x320_plain", (48, 320), 13, 64, False),
    ("w40x512_bs128", (40, 512), 14, 128, True),
]


def main():
    data = {}
    rng = np.random.default_rng(2024)
    for name, shape, seed, bs, nested in CASES:
        w = np.random.default_rng(seed).standard_normal(shape).astype(np.float32) * 0.02
        packed, st = o.quantize_nf4(w, blocksize=bs, compress_statistics=nested)
        data[f"{name}/packed"] = packed
        data[f"{name}/absmax"] = st.absmax
        data[f"{name}/code"] = st.code
        data[f"{name}/shape"] = np.array(shape, np.int64)
        data[f"{name}/blocksize"] = np.array(bs, np.int64)
        data[f"{name}/nested"] = np.array(int(nested), np.int64)
        if nested:
            data[f"{name}/absmax2"] = st.state2.absmax
            data[f"{name}/code2"] = st.state2.code
            data[f"{name}/offset"] = np.array(st.offset, np.float32)
        data[f"{name}/w_f16"] = o.dequantize(packed, st, "f16")
        data[f"{name}/w_bf16"] = o.dequantize(packed, st, "bf16")
        w16 = data[f"{name}/w_f16"]
        m = 37
        x = rng.standard_normal((m, shape[1])).astype(np.float16)
        bias = (rng.standard_normal(shape[0]) * 0.1).astype(np.float16)
        dy = (rng.standard_normal((m, shape[0])) * 1e-3).astype(np.float16)
        data[f"{name}/x"] = x
        data[f"{name}/bias"] = bias
        data[f"{name}/dy"] = dy
        data[f"{name}/y_ref"] = o.linear_fwd(x, w16, bias).numpy()
        data[f"{name}/dx_ref"] = o.linear_dx(dy, w16).numpy()
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(data)} arrays)")


def load_state(z, name):
    """(packed, OracleQuantState) of fixture `name` from the loaded npz `z`."""
    nested = bool(z[f"{name}/nested"])
    st = o.OracleQuantState(
        absmax=z[f"{name}/absmax"], shape=tuple(int(v) for v in z[f"{name}/shape"]),
        code=z[f"{name}/code"], blocksize=int(z[f"{name}/blocksize"]), nested=nested,
        offset=float(z[f"{name}/offset"]) if nested else 0.0,
        state2=o.OracleState2(absmax=z[f"{name}/absmax2"], code=z[f"{name}/code2"])
        if nested else None)
    return z[f"{name}/packed"], st


if __name__ == "__main__":
    main()
