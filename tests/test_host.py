"""Host-side logic of the package on the CPU: patches, routing, quantizer, descriptors,
loud failure without a GPU."""

import numpy as np
import pytest
import torch

from oracle import nf4_oracle as o


def test_apply_without_bitsandbytes_logs_and_continues(capsys):
    import solution

    done = solution.apply()
    err = capsys.readouterr().err
    assert set(done) == {"MLP recomputing its activations", "NF4 dequantization",
                         "4-bit linear layers in fp16"}
    try:
        import bitsandbytes  # noqa: F401
        has_bnb = True
    except ImportError:
        has_bnb = False
    if not has_bnb:
        assert not any(done.values())
        assert "not applied: ModuleNotFoundError" in err


def test_try_never_raises(capsys):
    import solution

    def boom():
        raise RuntimeError("x")

    assert solution._try("boom", boom) is False
    assert "boom not applied: RuntimeError: x" in capsys.readouterr().err


@pytest.mark.parametrize("nested", [True, False])
@pytest.mark.parametrize("shape", [(256, 1536), (7, 9), (64, 64)])
def test_product_quantizer_matches_oracle_on_cpu(shape, nested):
    from solution.quant_state import quantize_4bit

    g = torch.Generator().manual_seed(5)
    w = torch.randn(shape, generator=g) * 0.02
    packed, qs = quantize_4bit(w, compress_statistics=nested)
    pn, sn = o.quantize_nf4(w.numpy(), compress_statistics=nested)
    assert packed.shape == (pn.size, 1) and packed.dtype == torch.uint8
    np.testing.assert_array_equal(packed.view(-1).numpy(), pn)
    np.testing.assert_array_equal(qs.absmax.numpy(), sn.absmax)
    assert qs.nested == nested and qs.blocksize == 64 and qs.quant_type == "nf4"
    if nested:
        assert float(qs.offset) == np.float32(sn.offset)
        np.testing.assert_array_equal(qs.state2.absmax.numpy(), sn.state2.absmax)
        np.testing.assert_array_equal(qs.state2.code.numpy(), o.DYNAMIC_CODE)
        assert qs.state2.blocksize == 256
    np.testing.assert_array_equal(qs.code.numpy(), o.NF4_CODE)


def test_state_checks_mirror_reference():
    from solution.nf4 import _fused_ok, _nf4_state_ok
    from solution.quant_state import quantize_4bit

    packed, qs = quantize_4bit(torch.randn(8, 128))
    assert _nf4_state_ok(packed, qs, 128)
    assert not _nf4_state_ok(packed, qs, 64)
    assert not _nf4_state_ok(packed.float(), qs, 128)
    assert _fused_ok(qs)
    _, qs32 = quantize_4bit(torch.randn(8, 128), blocksize=32)
    assert not _fused_ok(qs32)
    qs.state2.blocksize = 128
    assert not _nf4_state_ok(packed, qs, 128)


def test_weight_descriptor_fields():
    from solution.quant_state import quantize_4bit, weight_desc

    packed, qs = quantize_4bit(torch.randn(16, 256))
    d = weight_desc(packed, qs)
    assert d.packed == packed.data_ptr() and d.rows == 16 and d.cols == 256
    assert d.blocksize == 64 and d.blocksize2 == 256 and d.nested == 1
    assert abs(d.offset - float(qs.offset)) == 0.0
    assert d.absmax == qs._nf4_refs[2].data_ptr()


def test_kernels_refuse_cpu_tensors_loudly():
    """No CPU fallback: the product path raises instead of computing on the host."""
    from solution.nf4 import NF4Linear, dequantize_nf4
    from solution.quant_state import quantize_4bit

    packed, qs = quantize_4bit(torch.randn(16, 128))
    with pytest.raises(ValueError, match="GPU"):
        dequantize_nf4(packed, qs)
    x = torch.randn(3, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="GPU"):
        NF4Linear.apply(x, packed.view(-1), qs, None)


def test_lora_struct_keeps_its_tensors_alive(monkeypatch):
    """make_lora stores raw pointers; a temporary passed to it (t=lora_xa(...)) must not return
    to torch's cache while the struct is in use, or the call's own output may be allocated over
    it.  The struct holds references: the tensor outlives the caller's last name for it."""
    import gc
    import weakref

    from solution import kernels

    t = torch.empty(4, 16, dtype=torch.float16)
    ref = weakref.ref(t)
    lo = kernels.make_lora(0, 16, 2.0, t=t, b=torch.empty(8, 16, dtype=torch.float16))
    del t
    gc.collect()
    assert ref() is not None and lo.t == ref().data_ptr()
    del lo
    gc.collect()
    assert ref() is None
    # the multi-launch LoRA jobs too (their device check switched off for CPU tensors)
    monkeypatch.setattr(kernels, "_check_device", lambda *t: None)
    out = torch.empty(4, 16, dtype=torch.float16)
    ref = weakref.ref(out)
    job = kernels.lora_job(torch.empty(4, 32, dtype=torch.float16),
                           torch.empty(16, 32, dtype=torch.float16), out)
    del out
    gc.collect()
    assert ref() is not None and job.out == ref().data_ptr()
    del job
    gc.collect()
    assert ref() is None


def test_missing_library_raises(tmp_path):
    from solution import _lib

    with pytest.raises(_lib.NF4LibraryError, match="missing"):
        _lib.load(tmp_path / "nope.so")


def test_supported_requires_cuda_and_layout():
    from solution.nf4 import _supported
    from solution.quant_state import quantize_4bit

    packed, qs = quantize_4bit(torch.randn(8, 128))
    x = torch.randn(2, 128, dtype=torch.float16)
    assert not _supported(x, packed, qs)  # CPU tensor: the original function would run


def test_layers_to_dequant_signature():
    from solution.layer import _dequant

    with pytest.raises(ValueError):
        _dequant([], torch.float16, streamed=[(None, None)])


def test_cu_seqlens_validation():
    from solution.stack import tokens_from_cu_seqlens

    assert tokens_from_cu_seqlens([0, 64, 200, 201]) == 201
    assert tokens_from_cu_seqlens(torch.tensor([0], dtype=torch.int32)) == 0
    for bad in ([1, 5], [0, 5, 3], [[0, 1]]):
        with pytest.raises(ValueError):
            tokens_from_cu_seqlens(bad)


@pytest.mark.parametrize("junk", [False, True])
def test_apply_with_unloadable_library_keeps_bitsandbytes(monkeypatch, capsys, tmp_path, junk):
    """A library that is missing or does not load: every patch is skipped and logged, and
    bitsandbytes' functions (here the stand-in's) stay in place (__init__.py:49-53)."""
    from transformers.models.qwen2 import modeling_qwen2

    import solution
    from solution import _lib
    from tests import bnb_standin

    bnb, _ = bnb_standin.install(monkeypatch)
    path = tmp_path / "libnf4_mi355x.so"
    if junk:
        path.write_bytes(b"not an ELF file")
    monkeypatch.setattr(_lib, "LIB_PATH", path)
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(modeling_qwen2.Qwen2MLP, "forward", modeling_qwen2.Qwen2MLP.forward)
    before = (bnb.nn.modules.Linear4bit.forward, bnb.matmul_4bit,
              bnb.autograd._functions.matmul_4bit, modeling_qwen2.Qwen2MLP.forward)
    done = solution.apply()
    assert not any(done.values())
    after = (bnb.nn.modules.Linear4bit.forward, bnb.matmul_4bit,
             bnb.autograd._functions.matmul_4bit, modeling_qwen2.Qwen2MLP.forward)
    assert after == before
    err = capsys.readouterr().err
    assert err.count("not applied: NF4LibraryError") == 3, err
