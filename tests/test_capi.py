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
    assert lib.nf4_abi_version() == 4
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


def test_dequant_table_pack_on_the_host(lib):
    """nf4_dequant_table_pack is host code: it validates the weights (unsupported layouts,
    a short buffer) and lays out header, entries and the per-workgroup weight index, whose
    workgroup counts follow the 8-elements-per-thread, 256-thread, 8-unit layout."""
    from solution._lib import NF4_ERR_UNSUPPORTED, NF4_ERR_WORKSPACE, NF4_OK, NF4Weight

    buf = (ctypes.c_uint8 * 4096)()
    code = (ctypes.c_float * 272)()
    a = ctypes.addressof(buf)

    def w(rows, cols, bs=64, nested=1):
        return NF4Weight(packed=a, absmax=a, absmax2=ctypes.addressof(code),
                         code2=ctypes.addressof(code), code=ctypes.addressof(code), nested=nested,
                         rows=rows, cols=cols, blocksize=bs, blocksize2=256)

    shapes = [(1536, 1536), (256, 1536), (8960, 1536), (3, 100)]
    ws = (NF4Weight * 4)(*[w(r, c) for r, c in shapes])
    outs = (ctypes.c_void_p * 4)(*[a + 64 * i for i in range(4)])
    nbytes = lib.nf4_dequant_table_bytes(ws, 4)
    per_wg = 256 * 8 * 8
    blocks_each = [-(-(-(-r * c // 8)) // (256 * 8)) for r, c in shapes]
    assert blocks_each[:3] == [r * c // per_wg for r, c in shapes[:3]]
    host = (ctypes.c_uint8 * nbytes)()
    blocks = ctypes.c_int64(0)
    assert lib.nf4_dequant_table_pack(ws, 4, outs, 0, host, nbytes - 1,
                                      ctypes.byref(blocks)) == NF4_ERR_WORKSPACE
    assert lib.nf4_dequant_table_pack(ws, 4, outs, 0, host, nbytes, ctypes.byref(blocks)) == NF4_OK
    assert blocks.value == sum(blocks_each)
    raw = bytes(host)
    tag, nw, dt = np.frombuffer(raw[:12], np.uint32)
    assert (tag, nw, dt) == (0x4E463454, 4, 0)
    hdr = np.frombuffer(raw[16:40], np.int64)
    assert hdr[0] == blocks.value
    index = np.frombuffer(raw[hdr[2]:hdr[2] + 4 * blocks.value], np.uint32)
    np.testing.assert_array_equal(index, np.repeat(np.arange(4), blocks_each))
    assert nbytes == hdr[2] + 4 * blocks.value
    odd = (NF4Weight * 1)(w(4, 96, bs=96))  # not a power of two: the batch entry points' job
    n1 = lib.nf4_dequant_table_bytes(odd, 1)
    h1 = (ctypes.c_uint8 * n1)()
    assert lib.nf4_dequant_table_pack(odd, 1, outs, 0, h1, n1,
                                      ctypes.byref(blocks)) == NF4_ERR_UNSUPPORTED
    misaligned = (ctypes.c_void_p * 1)(a + 8)
    one = (NF4Weight * 1)(w(4, 64))
    assert lib.nf4_dequant_table_pack(one, 1, misaligned, 0, h1, n1,
                                      ctypes.byref(blocks)) == NF4_ERR_UNSUPPORTED
