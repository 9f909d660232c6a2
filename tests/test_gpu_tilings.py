"""Every tiling of the tiled dequant-GEMMs, pinned through the *_tiled entry points: 256x256
tiles, 128x128 tiles, and 128x128 tiles whose reduction is split between two wave groups of
one workgroup, each with and without a reduction split across workgroups.  Odd step counts
(a wave group with one step fewer runs it on zero activations), stacked segments whose rows
end inside a 64-row step (the dX kernel zeroes the dY columns past a segment), bias, LoRA and
accumulation are covered; the dequantized weight must stay bit-exact through each tiling
(X = I, dY = I), and the products hold the path's tolerance against the fp32 oracle."""

import numpy as np
import pytest
import torch

from oracle import nf4_oracle as o
from tests.gpu_util import assert_rel, banner, oracle_w16, random_weight

pytestmark = pytest.mark.gpu

TILES = [0, 1, 3]  # kernels.TILE_256, TILE_128, TILE_128_KSPLIT2


def _x(m, k, seed, dev, dtype=torch.float16, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(m, k, generator=g) * std).to(dtype).to(dev)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("splits", [1, 2])
@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("shape,bs,nested", [((136, 320), 64, True), ((200, 512), 128, False)])
def test_tiling_dequant_is_bit_exact(cuda, tile, splits, shape, bs, nested, dtype):
    from solution import kernels

    n, k = shape
    banner("tiling dequant exact", tile, splits, shape, bs, nested, dtype)
    p, qs = random_weight(n, k, seed=n + k + 7, dev=cuda, blocksize=bs, nested=nested)
    ref = oracle_w16(p, qs, "bf16" if dtype == torch.bfloat16 else "f16").view(torch.int16)
    y = kernels.linear_fwd(torch.eye(k, dtype=dtype, device=cuda), [(p, qs)], tile=tile,
                           splits=splits)
    assert torch.equal(y.t().contiguous().cpu().view(torch.int16), ref)
    dx = kernels.linear_dx(torch.eye(n, dtype=dtype, device=cuda), [(p, qs)], tile=tile,
                           splits=splits)
    assert torch.equal(dx.cpu().view(torch.int16), ref)


def _lora(k, rows, r, seed, dev, dtype):
    g = torch.Generator().manual_seed(seed)
    bound = 1 / np.sqrt(k)
    a = ((torch.rand(r, k, generator=g) * 2 - 1) * bound).to(dtype).to(dev)
    b = (torch.randn(rows, r, generator=g) * 0.05).to(dtype).to(dev)
    return a, b


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [37, 300])
@pytest.mark.parametrize("splits", [1, 2, 3])
@pytest.mark.parametrize("tile", TILES)
def test_tiling_stacked_segments(cuda, tile, splits, m, dtype):
    """Segments of 96, 40 and 200 rows over K = 320 (5 forward steps; 2 + 1 + 4 dX steps, the
    last of each segment partial), bias, LoRA on segments 0 and 2, dX accumulated."""
    from solution import kernels

    banner("tiling stacked", tile, splits, m, dtype)
    dt = "bf16" if dtype == torch.bfloat16 else "f16"
    k, r, s = 320, 16, 2.0
    rows = (96, 40, 200)
    segs = [random_weight(n, k, seed=300 + i, dev=cuda) for i, n in enumerate(rows)]
    w = torch.cat([oracle_w16(p, q, dt) for p, q in segs])
    x = _x(m, k, 11, cuda, dtype)
    bias = _x(1, sum(rows), 12, cuda, dtype, std=0.5).view(-1)
    a0, b0 = _lora(k, rows[0], r, 13, cuda, dtype)
    a2, b2 = _lora(k, rows[2], r, 14, cuda, dtype)
    t0, t2 = kernels.lora_xa(x, a0), kernels.lora_xa(x, a2)
    loras = [kernels.make_lora(0, r, s, t=t0, b=b0), kernels.make_lora(2, r, s, t=t2, b=b2)]
    spec = [(0, rows[0], x, a0, b0, s), (rows[0] + rows[1], rows[2], x, a2, b2, s)]
    y = kernels.linear_fwd(x, segs, bias, loras, tile=tile, splits=splits)
    assert_rel(y, o.linear_fwd(x, w, bias, spec), what="fwd")

    dy = _x(m, sum(rows), 15, cuda, dtype, std=1e-2)
    c2 = rows[0] + rows[1]
    da0 = kernels.lora_da(dy[:, :rows[0]], b0, s)
    da2 = kernels.lora_da(dy[:, c2:], b2, s)
    dl = [kernels.make_lora(0, r, s, a=a0, da=da0), kernels.make_lora(2, r, s, a=a2, da=da2)]
    base = _x(m, k, 16, cuda, dtype, std=1e-2)
    out = base.clone()
    kernels.linear_dx(dy, segs, dl, out=out, accumulate=True, tile=tile, splits=splits)
    assert_rel(out, base.float().cpu() + o.linear_dx(dy, w, spec), what="dx accumulate")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("tile", TILES)
def test_tiling_swiglu_epilogue(cuda, tile, dtype):
    """The paired gate | up tiles with the SwiGLU epilogue under each tiling (I = 200 is not a
    multiple of any tile; K = 320 gives an odd step count)."""
    from solution import kernels

    banner("tiling swiglu", tile, dtype)
    dt = "bf16" if dtype == torch.bfloat16 else "f16"
    m, inter, k = 300, 200, 320
    gate = random_weight(inter, k, seed=401, dev=cuda)
    up = random_weight(inter, k, seed=402, dev=cuda)
    wg, wu = oracle_w16(*gate, dt), oracle_w16(*up, dt)
    x = _x(m, k, 41, cuda, dtype)
    dh = _x(m, inter, 42, cuda, dtype, std=1e-2)
    g, u = o.linear_fwd(x, wg), o.linear_fwd(x, wu)
    sig = 1.0 / (1.0 + torch.exp(-g))
    h = kernels.linear_swiglu_fwd(x, gate, up, tile=tile)
    assert_rel(h, g * sig * u, what="H")
    dgu = kernels.linear_swiglu_bwd(x, gate, up, dh, tile=tile)
    d = dh.float().cpu()
    assert_rel(dgu[:, :inter], d * u * sig * (1.0 + g * (1.0 - sig)), what="dG")
    assert_rel(dgu[:, inter:], d * g * sig, what="dU")


def test_tiling_arguments(cuda):
    """Unknown tilings and empty splits are refused before any launch."""
    from solution import kernels
    from solution._lib import NF4LibraryError

    p, qs = random_weight(64, 128, seed=5, dev=cuda)  # 2 forward steps, 1 dX step
    x = _x(8, 128, 1, cuda)
    for tile, splits in ((2, 1), (4, 1), (1, 3), (1, 0), (0, 17)):
        with pytest.raises(NF4LibraryError):
            kernels.linear_fwd(x, [(p, qs)], tile=tile, splits=splits)
    with pytest.raises(NF4LibraryError):
        kernels.linear_dx(_x(8, 64, 2, cuda), [(p, qs)], tile=1, splits=2)


def test_head_tail_plans_bit_exact(cuda):
    """At M = 2048 the cost model runs the stacked gate | up forward and the down projection's
    input gradient as two launches (whole rounds of 256x256 tiles, then the remaining rows or
    columns in 128x128 tiles; the gate | up split falls inside the up weight).  One-hot
    activation rows (row r selects k = r mod K) return weight columns exactly, so every output
    of both launches is checked bit for bit.  (The SwiGLU pair at this shape takes the same
    plan; test_swiglu_epilogue holds it to the path's tolerance.)"""
    from solution import kernels

    banner("head + tail plans", 2048)
    m, k, inter = 2048, 1536, 8960
    gate = random_weight(inter, k, seed=501, dev=cuda)
    up = random_weight(inter, k, seed=502, dev=cuda)
    w = torch.cat([oracle_w16(*gate), oracle_w16(*up)]).view(torch.int16)
    onehot = torch.zeros(m, k, dtype=torch.float16, device=cuda)
    onehot[torch.arange(m), torch.arange(m) % k] = 1.0
    y = kernels.linear_fwd(onehot, [gate, up]).cpu().view(torch.int16)
    assert torch.equal(y, w[:, torch.arange(m) % k].t().contiguous())

    down = random_weight(k, inter, seed=503, dev=cuda)
    wd = oracle_w16(*down).view(torch.int16)
    dy = torch.zeros(m, k, dtype=torch.float16, device=cuda)
    dy[torch.arange(m), torch.arange(m) % k] = 1.0
    dx = kernels.linear_dx(dy, [down]).cpu().view(torch.int16)
    assert torch.equal(dx, wd[torch.arange(m) % k])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("tile", TILES)
def test_lds_epilogue_matches_register_epilogue(cuda, tile, dtype):
    """The epilogues that stage a finished tile through LDS (16-byte row stores; in fp32 when a
    bias is added or the output accumulates, so the result is rounded once) against the
    register epilogue that writes from the MFMA layout, which runs when the output rows are
    not 16-byte aligned.  Same plan, same accumulators: outputs bit-equal, forward with a bias
    and input gradient with accumulation, a partial last 8-column chunk included (N = 1000)."""
    from solution import kernels

    banner(f"LDS epilogue vs register epilogue tile={tile} {dtype}")
    m, k = 300, 320
    segs = [random_weight(n, k, seed=500 + n, dev=cuda) for n in (1000, 256)]
    n = 1256
    x = _x(m, k, 51, cuda, dtype)
    bias = _x(1, n, 52, cuda, dtype).view(-1)
    y_al = torch.empty(m, n, dtype=dtype, device=cuda)
    y_mis = torch.empty(m * n + 8, dtype=dtype, device=cuda)[1:1 + m * n].view(m, n)
    kernels.linear_fwd(x, segs, bias, out=y_al, tile=tile)
    kernels.linear_fwd(x, segs, bias, out=y_mis, tile=tile)
    assert torch.equal(y_al, y_mis)
    dy = _x(m, n, 53, cuda, dtype, std=1e-2)
    base = _x(m, k, 54, cuda, dtype)
    d_al = base.clone()
    d_mis = torch.empty(m * k + 8, dtype=dtype, device=cuda)[1:1 + m * k].view(m, k)
    d_mis.copy_(base)
    kernels.linear_dx(dy, segs, out=d_al, accumulate=True, tile=tile)
    kernels.linear_dx(dy, segs, out=d_mis, accumulate=True, tile=tile)
    assert torch.equal(d_al, d_mis)
