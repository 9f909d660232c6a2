"""The C-ABI library loads and exports every entry point the header declares (no GPU needed);
argument validation answers before any launch."""

import ctypes
import re

import numpy as np
import pytest

from tests.conftest import ROOT
from tests.golden.make_fixtures import OUT as FIXTURES, load_state
from oracle import nf4_oracle as o

HEADER = ROOT / "include" / "nf4_mi355x.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nf4_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from solution import _lib

    return _lib.load()


def test_header_declares_the_binding(lib):
    from solution import _lib

    declared = _declared()
    assert declared == sorted(_lib.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name


def test_exports_in_shared_object():
    import subprocess

    from solution import _lib

    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (nf4_[a-z0-9_]+)", out))
    assert set(_declared()) <= exported


def test_struct_layouts_match_header():
    from solution._lib import NF4Lora, NF4LoraJob, NF4Weight

    assert ctypes.sizeof(NF4Weight) == 72
    assert NF4Weight.rows.offset == 48 and NF4Weight.blocksize2.offset == 68
    assert ctypes.sizeof(NF4Lora) == 48 and NF4Lora.t.offset == 16
    assert ctypes.sizeof(NF4LoraJob) == 48 and NF4LoraJob.scale.offset == 40
    assert NF4LoraJob.transpose_out.offset == 44


def test_version_and_status_strings(lib):
    assert lib.nf4_abi_version() == 1
    assert lib.nf4_status_string(0) == b"ok"
    assert b"unsupported" in lib.nf4_status_string(2)


def test_argument_validation_without_launch(lib):
    from solution._lib import NF4_ERR_ARG, NF4Weight

    empty = NF4Weight(blocksize=64)
    assert lib.nf4_dequant(ctypes.byref(empty), None, 0, None) == 0  # nothing to do
    w = NF4Weight(rows=4, cols=64, blocksize=64)  # non-empty with null pointers
    assert lib.nf4_dequant(None, None, 0, None) == NF4_ERR_ARG
    assert lib.nf4_dequant(ctypes.byref(w), None, 0, None) == NF4_ERR_ARG
    assert lib.nf4_dequant(ctypes.byref(w), ctypes.c_void_p(16), 0, None) == NF4_ERR_ARG
    assert lib.nf4_dequant_multi(ctypes.byref(w), 0, ctypes.c_void_p(16), 0, None) == NF4_ERR_ARG
    assert lib.nf4_linear_fwd(None, 4, 64, ctypes.byref(w), 1, None, None, 0, None, 64, 0, None,
                              0, None) == NF4_ERR_ARG
    assert lib.nf4_linear_fwd(None, 4, 64, ctypes.byref(w), 1, None, None, 0,
                              ctypes.c_void_p(16), 64, 7, None, 0, None) == NF4_ERR_ARG
    assert lib.nf4_lora_xa(None, 4, 64, 64, None, 0, None, 0, None) == NF4_ERR_ARG
    assert lib.nf4_swiglu_fwd(None, None, 8, None, 8, 1, 8, 5, None) == NF4_ERR_ARG


def test_unsupported_layout_reported(lib):
    """blocksize 32 (not a multiple of the 64-wide GEMM step) is refused by the fused GEMM
    before anything is launched."""
    from solution._lib import NF4_ERR_UNSUPPORTED, NF4Weight

    buf = (ctypes.c_uint8 * 64)()
    code = (ctypes.c_float * 16)()
    w = NF4Weight(packed=ctypes.addressof(buf), absmax=ctypes.addressof(buf),
                  code=ctypes.addressof(code), rows=4, cols=32, blocksize=32)
    x = (ctypes.c_uint16 * 256)()
    y = (ctypes.c_uint16 * 256)()
    st = lib.nf4_linear_fwd(ctypes.addressof(x), 4, 32, ctypes.byref(w), 1, None, None, 0,
                            ctypes.addressof(y), 4, 0, None, 0, None)
    assert st == NF4_ERR_UNSUPPORTED


def test_fixtures_reproduce_with_oracle():
    z = np.load(FIXTURES)
    names = sorted({k.split("/")[0] for k in z.files})
    assert len(names) == 4
    for name in names:
        packed, st = load_state(z, name)
        np.testing.assert_array_equal(o.dequantize(packed, st, "f16"), z[f"{name}/w_f16"])
        np.testing.assert_array_equal(o.dequantize(packed, st, "bf16"), z[f"{name}/w_bf16"])
        y = o.linear_fwd(z[f"{name}/x"], z[f"{name}/w_f16"], z[f"{name}/bias"]).numpy()
        np.testing.assert_allclose(y, z[f"{name}/y_ref"], rtol=1e-5, atol=1e-6)
