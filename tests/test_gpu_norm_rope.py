"""The q|k|v projection's neighbours on the GPU (RMSNorm with LoRA's dropout inputs, the rotary
embedding, both backward) against the fp32 oracle.  RoPE is one fp32 product pair per output in
both (no fused multiply-add in either), so its outputs must equal the oracle rounded once, bit
for bit; the norm sums a row in a different order, so it is held to the path's tolerance."""

import pytest
import torch

from oracle import nf4_oracle as o
from tests.gpu_util import assert_rel, banner

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]


def _r(shape, seed, dev, dtype, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype).to(dev)


def _keep(shape, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return (torch.rand(*shape, generator=g) > 0.1).to(dev)


def _packed(kq, kv):
    return torch.from_numpy(o.pack_keep_bits(kq.cpu().numpy(), kv.cpu().numpy()))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,cols", [(1, 1536), (37, 3584), (300, 1536), (5, 24)])
@pytest.mark.parametrize("res32", [False, True])
@pytest.mark.parametrize("residual,dropout", [(False, False), (True, True)])
def test_add_rmsnorm(cuda, dtype, rows, cols, res32, residual, dropout):
    """y, rstd and the dropout inputs against the oracle; with dropout, masks drawn over a
    padded batch of rows + 3 rows and gathered through a token -> row map (mode 1): the packed
    bits must equal the oracle's packing bit for bit, and feeding them back (mode 2) must give
    the same outputs bit for bit.  res32: the residual stream x in fp32."""
    from solution import kernels

    banner("rmsnorm fwd", dtype, rows, cols, res32, residual, dropout)
    x = _r((rows, cols), 1, cuda, torch.float32 if res32 else dtype)
    d = _r((rows, cols), 2, cuda, dtype, 0.5) if residual else None
    w = (torch.rand(cols, generator=torch.Generator().manual_seed(3)) + 0.5).to(cuda)
    if not dropout:
        y, rstd = kernels.add_rmsnorm(x, w, 1e-6, d=d, dtype=dtype)
        ry, rr, _, _ = o.add_rmsnorm(x, w, 1e-6, d=d)
        assert y.dtype == dtype
        assert_rel(y, ry, what="y")
        torch.testing.assert_close(rstd.cpu(), rr, rtol=1e-5, atol=0)
        return
    kq_pad, kv_pad = _keep((rows + 3, cols), 4, cuda), _keep((rows + 3, cols), 5, cuda)
    src = torch.randperm(rows + 3, generator=torch.Generator().manual_seed(6))[:rows].to(cuda)
    y, rstd, oq, ov, packed = kernels.add_rmsnorm(x, w, 1e-6, d=d, dtype=dtype, keep_q=kq_pad,
                                                  keep_v=kv_pad, rows=src, scale_q=1.0 / 0.9,
                                                  scale_v=1.0 / 0.8)
    kq, kv = kq_pad[src], kv_pad[src]
    assert torch.equal(packed.cpu(), _packed(kq, kv))
    ry, rr, rq, rv = o.add_rmsnorm(x, w, 1e-6, d=d, keep_q=kq, keep_v=kv, scale_q=1.0 / 0.9,
                                   scale_v=1.0 / 0.8)
    assert_rel(y, ry, what="y")
    torch.testing.assert_close(rstd.cpu(), rr, rtol=1e-5, atol=0)
    assert_rel(oq, rq, what="oq")
    assert_rel(ov, rv, what="ov")
    y2, rstd2, oq2, ov2 = kernels.add_rmsnorm(x, w, 1e-6, d=d, dtype=dtype, packed=packed,
                                              scale_q=1.0 / 0.9, scale_v=1.0 / 0.8)
    for a, b in ((y, y2), (rstd, rstd2), (oq, oq2), (ov, ov2)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,cols", [(37, 3584), (300, 1536)])
@pytest.mark.parametrize("res32", [False, True])
def test_rmsnorm_bwd(cuda, dtype, rows, cols, res32):
    """dX with every branch (output gradient, LoRA's two masked dropout branches from packed
    bits, the recomputed residual sum, the residual gradient) against the oracle; res32: x,
    dres and dX in fp32."""
    from solution import kernels

    banner("rmsnorm bwd", dtype, rows, cols, res32)
    rt = torch.float32 if res32 else dtype
    x, d = _r((rows, cols), 11, cuda, rt), _r((rows, cols), 12, cuda, dtype, 0.5)
    w = (torch.rand(cols, generator=torch.Generator().manual_seed(13)) + 0.5).to(cuda)
    y, rstd = kernels.add_rmsnorm(x, w, 1e-6, d=d, dtype=dtype)
    dy, dq, dv = (_r((rows, cols), s, cuda, dtype, 1e-2) for s in (14, 15, 16))
    dres = _r((rows, cols), 17, cuda, rt, 1e-2)
    kq, kv = _keep((rows, cols), 18, cuda), _keep((rows, cols), 19, cuda)
    packed = _packed(kq, kv).to(cuda)
    dx = kernels.rmsnorm_bwd(x, w, rstd, dy=dy, d=d, dres=dres, dq=dq, dv=dv, packed=packed,
                             scale_q=1.25, scale_v=0.75)
    assert dx.dtype == rt
    ref = o.rmsnorm_bwd(x, w, rstd, dy=dy, d=d, dres=dres, dq=dq, dv=dv, keep_q=kq, keep_v=kv,
                        scale_q=1.25, scale_v=0.75)
    assert_rel(dx, ref, what="dx")
    # only the output's gradient, no residual input
    dx1 = kernels.rmsnorm_bwd(x, w, rstd, dy=dy)
    assert_rel(dx1, o.rmsnorm_bwd(x, w, rstd, dy=dy), what="dx (dy only)")


def _rope_tables(tokens, head_dim, dev):
    pos = torch.arange(tokens, dtype=torch.float32)[:, None]
    inv = 1.0 / (1e6 ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    ang = pos * inv[None, :]
    cos = torch.cat([ang.cos(), ang.cos()], 1).to(dev)
    sin = torch.cat([ang.sin(), ang.sin()], 1).to(dev)
    return cos, sin


def _bits(t):
    return t.cpu().contiguous().view(torch.int16)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("tokens,n_heads,n_kv,head_dim", [(300, 12, 2, 128), (37, 28, 4, 128),
                                                          (5, 8, 8, 64), (1, 4, 1, 256),
                                                          (3, 4, 2, 6), (2, 2, 1, 1024)])
def test_qkv_rope_bit_exact(cuda, dtype, tokens, n_heads, n_kv, head_dim):
    """Vector kernels (head_dim a multiple of 8 up to 512) and the scalar ones (6, 1024)."""
    from solution import kernels

    banner("qkv rope", dtype, tokens, n_heads, n_kv, head_dim)
    width = (n_heads + 2 * n_kv) * head_dim
    qkv = _r((tokens, width + 8), 21, cuda, dtype)[:, :width]  # row stride != width
    cos, sin = _rope_tables(tokens, head_dim, cuda)
    q, k, v, kc, vc = kernels.qkv_rope(qkv, cos, sin, n_heads, n_kv, head_dim)
    rq, rk, rv, rkc, rvc = o.qkv_rope(qkv, cos, sin, n_heads, n_kv, head_dim)
    for got, ref, name in ((q, rq, "q"), (k, rk, "k"), (v, rv, "v"), (kc, rkc, "k cache"),
                           (vc, rvc, "v cache")):
        assert torch.equal(_bits(got), _bits(ref.to(dtype))), name


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("tokens,n_heads,n_kv,head_dim", [(300, 12, 2, 128), (37, 28, 4, 128),
                                                          (3, 4, 2, 6)])
def test_qkv_rope_bwd(cuda, dtype, tokens, n_heads, n_kv, head_dim):
    from solution import kernels

    banner("qkv rope bwd", dtype, tokens, n_heads, n_kv, head_dim)
    dq, dk, dv = (_r((tokens, n_heads, head_dim), s, cuda, dtype, 1e-2) for s in (31, 32, 33))
    cos, sin = _rope_tables(tokens, head_dim, cuda)
    d = kernels.qkv_rope_bwd(dq, dk, dv, cos, sin, n_kv)
    ref = o.qkv_rope_bwd(dq, dk, dv, cos, sin, n_kv)
    assert_rel(d, ref, what="dqkv")
    # the q block is one product pair per output: exact
    nq = n_heads * head_dim
    assert torch.equal(_bits(d[:, :nq]), _bits(ref[:, :nq].to(dtype)))


def test_norm_rope_arguments(cuda):
    from solution import kernels
    from solution._lib import NF4Unsupported

    x = torch.zeros(4, 20, dtype=torch.float16, device=cuda)  # 20 % 8 != 0
    with pytest.raises(NF4Unsupported):
        kernels.add_rmsnorm(x, torch.ones(20, device=cuda), 1e-6)
    qkv = torch.zeros(2, 5 * 64, dtype=torch.float16, device=cuda)
    cos = torch.ones(2, 64, device=cuda)
    with pytest.raises(Exception):
        kernels.qkv_rope(qkv, cos, cos, 3, 2, 64)  # 3 heads do not group over 2 kv heads


def test_add_rmsnorm_row_map_out_of_range(cuda):
    """A token -> mask-row map entry outside the masks' rows (negative or past the last) reads
    nothing: that token's masks count as all dropped (zero bits, zero dropout inputs) while the
    others match the in-range gather bit for bit."""
    from solution import kernels

    banner("rmsnorm fwd, row map out of range")
    rows, cols, dtype = 6, 256, torch.float16
    x = _r((rows, cols), 21, cuda, torch.float32)
    w = (torch.rand(cols, generator=torch.Generator().manual_seed(22)) + 0.5).to(cuda)
    kq, kv = _keep((4, cols), 23, cuda), _keep((4, cols), 24, cuda)
    src = torch.tensor([3, 0, 4, 1, -1, 1000], dtype=torch.int64, device=cuda)
    y, _, oq, ov, packed = kernels.add_rmsnorm(x, w, 1e-6, dtype=dtype, keep_q=kq, keep_v=kv,
                                               rows=src, scale_q=2.0, scale_v=2.0)
    ok = torch.tensor([3, 0, 1, 1])
    y2, _, oq2, ov2, packed2 = kernels.add_rmsnorm(x[[0, 1, 3, 3]].contiguous(), w, 1e-6,
                                                   dtype=dtype, keep_q=kq, keep_v=kv,
                                                   rows=ok.to(cuda), scale_q=2.0, scale_v=2.0)
    for mine, other in ((0, 0), (1, 1), (3, 2)):
        assert torch.equal(packed[mine], packed2[other])
        assert torch.equal(oq[mine], oq2[other]) and torch.equal(ov[mine], ov2[other])
    for bad in (2, 4, 5):
        assert not packed[bad].any() and not oq[bad].any() and not ov[bad].any()
        assert torch.equal(y[bad], kernels.add_rmsnorm(x[bad:bad + 1].contiguous(), w, 1e-6,
                                                       dtype=dtype)[0][0])
