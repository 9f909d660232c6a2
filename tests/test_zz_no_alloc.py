"""nf4_linear_dx_noalloc - the input-gradient GEMM that allocates nothing (split-K partials in a
static device array) - against nf4_linear_dx through the C ABI, on two calls in a row, the
second with a smaller input: bit for bit where nf4_linear_dx's own plan fits the array (the
same tiling and split order), and within the path's tolerance (max rel 1e-2, mean rel 1e-3)
where the array forces a smaller split."""

import pytest
import torch

from tests.gpu_util import assert_rel, banner, random_weight

pytestmark = pytest.mark.gpu

CAP = 64 << 20  # NF4_STATIC_SCRATCH_BYTES


def _noalloc(dy, weights, out, accumulate=False, loras=()):
    from solution import _lib, kernels

    arr = kernels._descs(weights)
    larr, nl = kernels._lora_array(list(loras))
    st = _lib.load().nf4_linear_dx_noalloc(dy.data_ptr(), dy.shape[0], dy.stride(0), arr,
                                           len(weights), larr, nl, out.data_ptr(), out.stride(0),
                                           int(accumulate), _lib.DTYPE_CODE[dy.dtype],
                                           _lib.stream_of(dy))
    _lib.check(st, "nf4_linear_dx_noalloc")
    return out


def _need(m, weights):
    from solution import _lib, kernels

    return _lib.load().nf4_linear_dx_workspace(m, kernels._descs(weights), len(weights), 0)


def test_noalloc_dx_matches_linear_dx(cuda):
    from solution import kernels

    gate = random_weight(8960, 1536, seed=104, dev=cuda)
    up = random_weight(8960, 1536, seed=105, dev=cuda)
    q = random_weight(1536, 1536, seed=100, dev=cuda)
    g = torch.Generator().manual_seed(9)
    # 1: the benchmark's gate|up input gradient (256x256 tiles split 5: 60 MiB of partials)
    banner("noalloc dx gate|up M=2048")
    dy = (torch.randn(2048, 17920, generator=g) * 1e-3).half().to(cuda)
    need = _need(2048, [gate, up])
    assert 0 < need <= CAP
    ref = kernels.linear_dx(dy, [gate, up])
    out = torch.full_like(ref, float("nan"))
    _noalloc(dy, [gate, up], out)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    # 2: a smaller call right after, accumulating, with a LoRA slab; the array still holds the
    # first call's partials
    banner("noalloc dx q + LoRA M=300 accumulate")
    r, s = 16, 2.0
    dy2 = (torch.randn(300, 1536, generator=g) * 1e-3).half().to(cuda)
    a = (torch.randn(r, 1536, generator=g) * 0.02).half().to(cuda)
    da = (torch.randn(300, r, generator=g) * 1e-3).half().to(cuda)
    lora = [kernels.make_lora(0, r, s, a=a, da=da)]
    base = (torch.randn(300, 1536, generator=g) * 1e-2).half().to(cuda)
    ref2 = kernels.linear_dx(dy2, [q], lora, out=base.clone(), accumulate=True)
    out2 = _noalloc(dy2, [q], base.clone(), accumulate=True, loras=lora)
    torch.cuda.synchronize()
    assert torch.equal(out2, ref2)
    # 3: a plan whose partials would not fit: a smaller split, within tolerance
    banner("noalloc dx gate|up M=8192 (plan restricted to the array)")
    dy3 = (torch.randn(8192, 17920, generator=g) * 1e-3).half().to(cuda)
    assert _need(8192, [gate, up]) > CAP
    ref3 = kernels.linear_dx(dy3, [gate, up])
    out3 = _noalloc(dy3, [gate, up], torch.empty_like(ref3))
    torch.cuda.synchronize()
    assert_rel(out3, ref3.float().cpu(), what="restricted plan")
