"""The reference's operators on the HIP path: NF4Linear (solution/test_kernels.py:62-75),
the q|k|v projection with LoRA on q and v (layer.py:871-878, 1072-1090) and RecomputedMLP
(test_kernels.py:200-221), against fp32 autograd of the oracle formulas."""

import numpy as np
import pytest
import torch

from oracle import nf4_oracle as o
from tests.gpu_util import assert_rel, banner, oracle_w16, random_weight

pytestmark = pytest.mark.gpu


def test_nf4_linear_forward_backward(cuda):
    """The reference's own test case: x [3, 100, 1536], W [256, 1536] with bias."""
    from solution.nf4 import NF4Linear

    banner("NF4Linear 3x100x1536 -> 256")
    p, qs = random_weight(256, 1536, seed=0, dev=cuda, std=0.05)
    w = oracle_w16(p, qs).float()
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 100, 1536, generator=g).half().to(cuda).requires_grad_()
    bias = torch.randn(256, generator=g).half().to(cuda).requires_grad_()
    grad = torch.randn(3, 100, 256, generator=g).half().to(cuda)
    out = NF4Linear.apply(x, p, qs, bias)
    out.backward(grad)
    xr = x.detach().float().cpu().requires_grad_()
    br = bias.detach().float().cpu().requires_grad_()
    ref = torch.nn.functional.linear(xr, w, br)
    ref.backward(grad.float().cpu())
    assert out.shape == (3, 100, 256) and out.dtype == torch.float16
    assert_rel(out, ref.detach(), what="out")
    assert_rel(x.grad, xr.grad, what="dx")
    assert_rel(bias.grad, br.grad, max_rel=1e-3, mean_rel=1e-3, what="dbias")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_qkv_projection_with_lora_grads(cuda, dtype):
    from solution.layer import LoraAdapter, ProjectionSpec, project

    banner("NF4Projection qkv + LoRA", dtype)
    m, k, r, alpha = 2048, 1536, 16, 32
    s = alpha / r
    segs = [random_weight(n, k, seed=100 + i, dev=cuda) for i, n in enumerate((1536, 256, 256))]
    wname = "bf16" if dtype == torch.bfloat16 else "f16"
    w = torch.cat([oracle_w16(pp, q, wname) for pp, q in segs]).float()
    g = torch.Generator().manual_seed(1)
    x = torch.randn(4, 512, k, generator=g).to(dtype).to(cuda).requires_grad_()
    bias = (torch.randn(2048, generator=g) * 0.5).to(dtype).to(cuda)
    g3 = torch.Generator().manual_seed(3)
    bound = 1 / np.sqrt(k)
    a_q = ((torch.rand(r, k, generator=g3) * 2 - 1) * bound).to(cuda).requires_grad_()
    a_v = ((torch.rand(r, k, generator=g3) * 2 - 1) * bound).to(cuda).requires_grad_()
    g4 = torch.Generator().manual_seed(4)
    b_q = (torch.randn(1536, r, generator=g4) * 0.01).to(cuda).requires_grad_()
    b_v = (torch.randn(256, r, generator=g4) * 0.01).to(cuda).requires_grad_()
    spec = ProjectionSpec(weights=segs, loras=[LoraAdapter(0, s), LoraAdapter(2, s)])
    y = project(x, spec, bias, (a_q, b_q, a_v, b_v))
    g2 = torch.Generator().manual_seed(2)
    dy = (torch.randn(4, 512, 2048, generator=g2) * 1e-3).to(dtype).to(cuda)
    y.backward(dy)

    # fp32 autograd of the same formula on the CPU
    xr = x.detach().float().cpu().requires_grad_()
    leaves = [t.detach().float().cpu().requires_grad_() for t in (a_q, b_q, a_v, b_v)]
    aq, bq, av, bv = leaves
    yr = xr @ w.t() + bias.float().cpu()
    yr = torch.cat([yr[..., :1536] + s * (xr @ aq.t()) @ bq.t(), yr[..., 1536:1792],
                    yr[..., 1792:] + s * (xr @ av.t()) @ bv.t()], -1)
    yr.backward(dy.float().cpu())
    assert_rel(y, yr.detach(), what="y")
    assert_rel(x.grad, xr.grad, what="dx")
    for name, got, ref in zip(("dA_q", "dB_q", "dA_v", "dB_v"), (a_q.grad, b_q.grad, a_v.grad,
                                                                 b_v.grad), leaves):
        assert got.dtype == torch.float32
        # fp32 gradients from half-precision operands (da is rounded to the GEMM dtype, as the
        # reference's fp16 da is): bf16 operands carry the bf16 mean tolerance
        assert_rel(got, ref.grad, mean_rel=3e-3 if dtype == torch.bfloat16 else 1e-3, what=name)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_qkv_projection_lora_dropout_chain(cuda, dtype):
    """LoRA dropout p = 0.1 on q and v through the reference's chain (layer.py:859-878,
    1072-1090, 135-164): RMSNorm of the fp32 residual stream with keep masks drawn over a padded
    batch (mode 1, packed bits out), the q|k|v projection whose adapters read the dropout
    outputs, then the backward: the projection's d(drop_q), d(drop_v) masked in the norm
    backward with the packed bits, plus a residual gradient.  Against fp32 autograd of the same
    formulas on the CPU with the same masks."""
    from solution import layer
    from solution.layer import LoraAdapter, NF4Projection, ProjectionSpec

    banner("LoRA dropout chain p=0.1", dtype)
    m, k, r, alpha, p = 384, 1536, 16, 32, 0.1
    s, keep_scale = alpha / r, 1.0 / (1.0 - p)
    segs = [random_weight(n, k, seed=300 + i, dev=cuda) for i, n in enumerate((1536, 256, 256))]
    wname = "bf16" if dtype == torch.bfloat16 else "f16"
    w = torch.cat([oracle_w16(pp, q, wname) for pp, q in segs]).float()
    g = torch.Generator().manual_seed(11)
    x = torch.randn(m, k, generator=g).to(cuda)                       # fp32 residual stream
    nw = (torch.rand(k, generator=g) + 0.5).to(cuda)                  # norm weight
    bias = (torch.randn(2048, generator=g) * 0.5).to(dtype).to(cuda)
    kq_pad = torch.rand(m + 5, k, generator=g) > p                    # masks over a padded batch
    kv_pad = torch.rand(m + 5, k, generator=g) > p
    src = torch.randperm(m + 5, generator=g)[:m]
    bound = 1 / np.sqrt(k)
    a_q = ((torch.rand(r, k, generator=g) * 2 - 1) * bound).to(cuda).requires_grad_()
    a_v = ((torch.rand(r, k, generator=g) * 2 - 1) * bound).to(cuda).requires_grad_()
    b_q = (torch.randn(1536, r, generator=g) * 0.01).to(cuda).requires_grad_()
    b_v = (torch.randn(256, r, generator=g) * 0.01).to(cuda).requires_grad_()
    dy = (torch.randn(m, 2048, generator=g) * 1e-3).to(dtype).to(cuda)
    dres = (torch.randn(m, k, generator=g) * 1e-3).to(cuda)

    y16, rstd, drop_q, drop_v, packed = layer._norm(
        x, None, nw, 1e-6, dtype, (kq_pad.to(cuda), kv_pad.to(cuda), src.to(cuda), keep_scale,
                                   keep_scale))
    y16, drop_q, drop_v = (t.requires_grad_() for t in (y16, drop_q, drop_v))
    spec = ProjectionSpec(weights=segs, loras=[LoraAdapter(0, s, own_input=True),
                                               LoraAdapter(2, s, own_input=True)])
    y = NF4Projection.apply(y16, bias, spec, a_q, b_q, drop_q, a_v, b_v, drop_v)
    y.backward(dy)
    dx = layer._norm_bwd(y16.grad, drop_q.grad, drop_v.grad, packed, x, None, nw, rstd, dres,
                         keep_scale, keep_scale)
    assert dx.dtype == torch.float32

    xr = x.cpu().requires_grad_()
    leaves = [t.detach().float().cpu().requires_grad_() for t in (a_q, b_q, a_v, b_v)]
    aq, bq, av, bv = leaves
    kq, kv = kq_pad[src].float(), kv_pad[src].float()
    rs = 1.0 / (xr.pow(2).mean(-1, keepdim=True) + 1e-6).sqrt()
    yn = nw.cpu() * (xr * rs)
    dq_in, dv_in = yn * kq * keep_scale, yn * kv * keep_scale
    yr = yn @ w.t() + bias.float().cpu()
    yr = torch.cat([yr[:, :1536] + s * (dq_in @ aq.t()) @ bq.t(), yr[:, 1536:1792],
                    yr[:, 1792:] + s * (dv_in @ av.t()) @ bv.t()], -1)
    (yr * dy.float().cpu()).sum().add_((xr * dres.cpu()).sum()).backward()
    assert_rel(y, yr.detach(), what="y")
    assert_rel(dx, xr.grad, what="dx")
    for name, got, ref in zip(("dA_q", "dB_q", "dA_v", "dB_v"), (a_q.grad, b_q.grad, a_v.grad,
                                                                 b_v.grad), leaves):
        assert_rel(got, ref.grad, mean_rel=3e-3 if dtype == torch.bfloat16 else 1e-3, what=name)
    # dropped elements are zero in the dropout inputs
    assert torch.all(drop_q.detach().cpu()[kq == 0] == 0)
    assert torch.all(drop_v.detach().cpu()[kv == 0] == 0)


@pytest.mark.parametrize("tokens", [200, 8])
def test_recomputed_mlp_matches_fp32(cuda, tokens):
    """The reference's MLP test shapes (gate/up 1024x512, down 512x1024, x [1, 200, 512]): the
    fused SwiGLU-epilogue path; and 8 tokens, below FUSED_MIN_TOKENS (separate SwiGLU step)."""
    from solution.mlp import RecomputedMLP

    banner("RecomputedMLP", tokens)
    gate = random_weight(1024, 512, seed=1, dev=cuda, std=0.05)
    up = random_weight(1024, 512, seed=2, dev=cuda, std=0.05)
    down = random_weight(512, 1024, seed=3, dev=cuda, std=0.05)
    wg, wu, wd = (oracle_w16(p, q).float() for p, q in (gate, up, down))
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, tokens, 512, generator=g).half().to(cuda).requires_grad_()
    grad = torch.randn(1, tokens, 512, generator=g).half().to(cuda)
    out = RecomputedMLP.apply(x, gate[0], gate[1], up[0], up[1], down[0], down[1])
    out.backward(grad)
    xr = x.detach().float().cpu().requires_grad_()
    ref = o.mlp_fwd(xr, wg, wu, wd)
    ref.backward(grad.float().cpu())
    assert_rel(out, ref.detach(), what="mlp out")
    assert_rel(x.grad, xr.grad, what="mlp dx")


def test_projection_backward_with_dirty_allocator_cache(cuda):
    """The backward's LoRA side buffers (da) are reached by the kernels only through raw
    pointers: they must stay allocated until the last launch is queued.  torch's cache is first
    filled with NaN so that a buffer freed too early and handed to another allocation shows as
    NaN in dX (it once did, on the second of two runs)."""
    from solution.layer import LoraAdapter, ProjectionSpec, project

    banner("NF4Projection backward, NaN-filled allocator cache")
    m, k, r, s = 512, 1536, 16, 2.0
    segs = [random_weight(n, k, seed=100 + i, dev=cuda) for i, n in enumerate((1536, 256, 256))]
    w = torch.cat([oracle_w16(pp, q) for pp, q in segs]).float()
    g = torch.Generator().manual_seed(7)
    x0 = torch.randn(m, k, generator=g).half()
    dy = (torch.randn(m, 2048, generator=g) * 1e-3).half()
    params0 = [(torch.rand(r, k, generator=g) - 0.5) * 0.05, torch.randn(1536, r, generator=g) * 0.01,
               (torch.rand(r, k, generator=g) - 0.5) * 0.05, torch.randn(256, r, generator=g) * 0.01]
    spec = ProjectionSpec(weights=segs, loras=[LoraAdapter(0, s), LoraAdapter(2, s)])
    xr = x0.float().requires_grad_()
    leaves = [p.clone().requires_grad_() for p in params0]
    aq, bq, av, bv = leaves
    yr = xr @ w.t()
    yr = torch.cat([yr[:, :1536] + s * (xr @ aq.t()) @ bq.t(), yr[:, 1536:1792],
                    yr[:, 1792:] + s * (xr @ av.t()) @ bv.t()], -1)
    yr.backward(dy.float())
    for _ in range(3):
        torch.full((1 << 28,), float("nan"), dtype=torch.float16, device=cuda)  # freed at once
        x = x0.to(cuda).requires_grad_()
        params = [p.to(cuda).requires_grad_() for p in params0]
        y = project(x, spec, None, params)
        torch.full((1 << 28,), float("nan"), dtype=torch.float16, device=cuda)
        y.backward(dy.to(cuda))
        torch.cuda.synchronize()
        assert_rel(x.grad, xr.grad, what="dx")
        for name, p, ref in zip(("dA_q", "dB_q", "dA_v", "dB_v"), params, leaves):
            assert_rel(p.grad, ref.grad, what=name)


def test_projection_backward_misaligned_lora_segments(cuda):
    """Two adapters on segments whose dY columns start off a 16-byte boundary (segment rows
    4, 98, 42: offsets 4 and 102): the backward copies each adapter's dY slice, and those copies
    are reached only through the job structs, so they must outlive the loop that makes them.
    The allocator cache is filled with NaN first, so a copy freed early and handed to the next
    allocation shows in dA / dB."""
    from solution.layer import LoraAdapter, ProjectionSpec, project

    banner("NF4Projection backward, adapters on misaligned dY segments")
    m, k, r, s = 384, 512, 16, 2.0
    rows = (4, 98, 42)
    segs = [random_weight(n, k, seed=300 + i, dev=cuda) for i, n in enumerate(rows)]
    w = torch.cat([oracle_w16(pp, q) for pp, q in segs]).float()
    g = torch.Generator().manual_seed(11)
    x0 = torch.randn(m, k, generator=g).half()
    dy = (torch.randn(m, sum(rows), generator=g) * 1e-3).half()
    params0 = [(torch.rand(r, k, generator=g) - 0.5) * 0.05, torch.randn(rows[1], r, generator=g) * 0.01,
               (torch.rand(r, k, generator=g) - 0.5) * 0.05, torch.randn(rows[2], r, generator=g) * 0.01]
    spec = ProjectionSpec(weights=segs, loras=[LoraAdapter(1, s), LoraAdapter(2, s)])
    xr = x0.float().requires_grad_()
    leaves = [p.clone().requires_grad_() for p in params0]
    a1, b1, a2, b2 = leaves
    yr = xr @ w.t()
    o1, o2 = rows[0], rows[0] + rows[1]
    yr = torch.cat([yr[:, :o1], yr[:, o1:o2] + s * (xr @ a1.t()) @ b1.t(),
                    yr[:, o2:] + s * (xr @ a2.t()) @ b2.t()], -1)
    yr.backward(dy.float())
    for _ in range(3):
        torch.full((1 << 26,), float("nan"), dtype=torch.float16, device=cuda)  # freed at once
        x = x0.to(cuda).requires_grad_()
        params = [p.to(cuda).requires_grad_() for p in params0]
        y = project(x, spec, None, params)
        assert_rel(y, yr.detach(), what="y")
        torch.full((1 << 26,), float("nan"), dtype=torch.float16, device=cuda)
        y.backward(dy.to(cuda))
        torch.cuda.synchronize()
        assert_rel(x.grad, xr.grad, what="dx")
        for name, p, ref in zip(("dA_1", "dB_1", "dA_2", "dB_2"), params, leaves):
            assert_rel(p.grad, ref.grad, what=name)
