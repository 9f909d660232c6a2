"""Fused NF4 dequant-GEMMs (forward and input gradient, with bias and LoRA) vs the fp32 oracle
on the bit-exact dequantized weight.  Tolerance from the path's contract (fp16 and bf16):
max |out - ref| / max |ref| <= 1e-2 and mean |out - ref| / mean |ref| <= 1e-3."""

import numpy as np
import pytest
import torch

from oracle import nf4_oracle as o
from tests.golden.make_fixtures import OUT as FIXTURES, load_state
from tests.gpu_util import assert_rel, banner, oracle_w16, random_weight, to_device_state

pytestmark = pytest.mark.gpu

QWEN_15B = {"q": (1536, 1536), "k": (256, 1536), "v": (256, 1536), "o": (1536, 1536),
            "gate": (8960, 1536), "up": (8960, 1536), "down": (1536, 8960)}


def _x(m, k, seed, dev, dtype=torch.float16, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(m, k, generator=g) * std).to(dtype).to(dev)


def test_fixture_forward_and_dx(cuda):
    from solution import kernels

    z = np.load(FIXTURES)
    for name in sorted({k.split("/")[0] for k in z.files}):
        banner("gemm fixture", name)
        packed, st = load_state(z, name)
        p, qs = to_device_state(packed, st, cuda)
        x = torch.from_numpy(z[f"{name}/x"]).to(cuda)
        bias = torch.from_numpy(z[f"{name}/bias"]).to(cuda)
        y = kernels.linear_fwd(x, [(p, qs)], bias)
        assert_rel(y, torch.from_numpy(z[f"{name}/y_ref"]), what=f"{name} fwd")
        dy = torch.from_numpy(z[f"{name}/dy"]).to(cuda)
        dx = kernels.linear_dx(dy, [(p, qs)])
        assert_rel(dx, torch.from_numpy(z[f"{name}/dx_ref"]), what=f"{name} dx")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape,bs,nested", [((384, 256), 64, True), ((256, 1536), 64, True),
                                             ((200, 512), 128, True), ((136, 320), 64, False)])
def test_fused_dequant_is_bit_exact(cuda, shape, bs, nested, dtype):
    """With X = I the forward GEMM returns W^T and with dY = I the input gradient returns W,
    each output one exact product: the weight dequantized inside the GEMM main loop must equal
    the oracle's bit for bit."""
    from solution import kernels

    n, k = shape
    banner("fused dequant exact", shape, bs, nested, dtype)
    p, qs = random_weight(n, k, seed=n + k, dev=cuda, blocksize=bs, nested=nested)
    ref = oracle_w16(p, qs, "bf16" if dtype == torch.bfloat16 else "f16").view(torch.int16)
    eye_k = torch.eye(k, dtype=dtype, device=cuda)
    y = kernels.linear_fwd(eye_k, [(p, qs)])
    assert torch.equal(y.t().contiguous().cpu().view(torch.int16), ref)
    eye_n = torch.eye(n, dtype=dtype, device=cuda)
    dx = kernels.linear_dx(eye_n, [(p, qs)])
    assert torch.equal(dx.cpu().view(torch.int16), ref)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape,bs,nested", [((136, 384), 64, True), ((40, 1024), 128, True),
                                             ((72, 256), 64, False), ((48, 1536), 64, True),
                                             ((32, 3072), 64, True)])
def test_decode_dequant_is_bit_exact(cuda, shape, bs, nested, dtype):
    """The decode path (M <= 16): 16 one-hot activation rows X = I[c0:c0+16] give the weight
    columns c0 .. c0+15 exactly, for every column block; rows past a 16-row weight tile, plain
    fp32 absmax and block 128 included.  The reductions of 3 to 24 super-steps give 1, 2, 4 and
    8 waves per tile (the cross-wave sum in LDS)."""
    from solution import kernels

    n, k = shape
    banner("decode dequant exact", shape, bs, nested, dtype)
    p, qs = random_weight(n, k, seed=n + 3 * k, dev=cuda, blocksize=bs, nested=nested)
    ref = oracle_w16(p, qs, "bf16" if dtype == torch.bfloat16 else "f16").view(torch.int16)
    eye = torch.eye(k, dtype=dtype, device=cuda)
    for c0 in range(0, k, 16):
        y = kernels.linear_fwd(eye[c0:c0 + 16], [(p, qs)])
        assert torch.equal(y.t().contiguous().cpu().view(torch.int16), ref[:, c0:c0 + 16]), c0


# (segment rows, K, M, blocksize, nested): each case lands on one skinny workgroup shape by the
# planner's cost model - token groups MT, row tiles RT, super-step DKS - noted per case
SKINNY_CASES = [
    ((1200,), 2048, 16, 64, True),        # MT 1, RT 1 (8 k-parts), DKS 128
    ((5000,), 1024, 13, 64, True),        # MT 1, RT 2, DKS 128
    ((5000,), 2048, 16, 128, False),      # MT 1, RT 2, DKS 128, block 128, fp32 absmax
    ((9000,), 768, 16, 64, True),         # MT 1, RT 4, DKS 128
    ((9000,), 1024, 16, 64, True),        # MT 1, RT 4, DKS 256
    ((8960, 8960), 1536, 16, 64, True),   # MT 1, RT 8, DKS 256: gate|up of Qwen2.5-1.5B
    ((8960, 8960), 1536, 3, 64, True),    # the same at 3 tokens
    ((1200,), 2048, 24, 64, True),        # MT 2, RT 1
    ((1200,), 1024, 17, 64, True),        # MT 2, RT 2
    ((700, 500), 512, 24, 64, True),      # MT 2, RT 4, two segments
    ((1200,), 256, 32, 64, True),         # MT 2, RT 8
    ((1200,), 1024, 40, 64, True),        # MT 4, RT 2
    ((1200,), 512, 64, 64, True),         # MT 4, RT 4
    ((1200,), 256, 33, 64, True),         # MT 4, RT 8
    ((1024,), 8192, 16, 64, True),        # MT 1, RT 2, 8 reduction splits (fp32 partials)
    ((1024,), 8960, 24, 64, True),        # MT 2, RT 2, 8 splits, the last one shorter
    ((1024,), 4096, 40, 64, True),        # MT 4, RT 2, 4 splits
    ((3584,), 18944, 8, 64, True),        # MT 1, RT 8, DKS 256, 8 splits, the last one shorter:
                                          # down of Qwen2.5-7B
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case", SKINNY_CASES, ids=lambda c: f"{'+'.join(map(str, c[0]))}x{c[1]}-m{c[2]}")
def test_skinny_dequant_is_bit_exact(cuda, case, dtype):
    """The skinny path (2 < M <= 64): m one-hot activation rows X = I[c0:c0+m] give the weight
    columns c0 .. c0+m-1 exactly (every stacked segment), over column blocks spread across K:
    one to four 16-token groups, a token group only partly used, k-parts with a shorter last
    part, rows past a row tile, and both super-step depths (their nibble-plane order of the
    weight and activation fragments included)."""
    from solution import kernels

    rows, k, m, bs, nested = case
    banner("skinny dequant exact", rows, k, m, bs, nested, dtype)
    ws, refs = [], []
    for i, n in enumerate(rows):
        p, qs = random_weight(n, k, seed=n + 7 * k + i, dev=cuda, blocksize=bs, nested=nested)
        ws.append((p, qs))
        refs.append(oracle_w16(p, qs, "bf16" if dtype == torch.bfloat16 else "f16").view(torch.int16))
    ref = torch.cat(refs, 0)
    eye = torch.eye(k, dtype=dtype, device=cuda)
    starts = sorted({min(c, k - m) for c in range(0, k, m)})
    if len(starts) > 24:  # 24 blocks spread over K, the first and the last included
        starts = [starts[round(i * (len(starts) - 1) / 23)] for i in range(24)]
    for c0 in starts:
        y = kernels.linear_fwd(eye[c0:c0 + m], ws)
        assert torch.equal(y.t().contiguous().cpu().view(torch.int16), ref[:, c0:c0 + m]), c0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("proj", list(QWEN_15B))
def test_qwen_projection_m2048(cuda, proj, dtype):
    from solution import kernels

    n, k = QWEN_15B[proj]
    banner("gemm qwen", proj, n, k, dtype)
    p, qs = random_weight(n, k, seed=100 + list(QWEN_15B).index(proj), dev=cuda)
    w = oracle_w16(p, qs, "bf16" if dtype == torch.bfloat16 else "f16")
    x = _x(2048, k, 1, cuda, dtype)
    y = kernels.linear_fwd(x, [(p, qs)])
    assert_rel(y, o.linear_fwd(x, w), what=f"{proj} fwd")
    dy = _x(2048, n, 2, cuda, dtype, std=1e-3)
    dx = kernels.linear_dx(dy, [(p, qs)])
    assert_rel(dx, o.linear_dx(dy, w), what=f"{proj} dx")


@pytest.mark.parametrize("m", [1, 37, 129, 300, 2049])
@pytest.mark.parametrize("n,k", [(100, 256), (1000, 320), (256, 64)])
def test_ragged_shapes(cuda, m, n, k):
    from solution import kernels

    banner("gemm ragged", m, n, k)
    p, qs = random_weight(n, k, seed=m + n + k, dev=cuda)
    w = oracle_w16(p, qs)
    x = _x(m, k, 3, cuda)
    bias = _x(1, n, 4, cuda, std=0.1).view(-1)
    y = kernels.linear_fwd(x, [(p, qs)], bias)
    assert_rel(y, o.linear_fwd(x, w, bias), what="fwd")
    if n % 8 == 0:
        dy = _x(m, n, 5, cuda, std=1e-3)
        assert_rel(kernels.linear_dx(dy, [(p, qs)]), o.linear_dx(dy, w), what="dx")


def test_stacked_qkv_with_bias_and_lora(cuda):
    from solution import kernels

    banner("gemm stacked qkv + lora")
    m, k, r, s = 2048, 1536, 16, 2.0
    segs = [random_weight(n, k, seed=100 + i, dev=cuda) for i, n in enumerate((1536, 256, 256))]
    w = torch.cat([oracle_w16(p, q) for p, q in segs])
    x = _x(m, k, 1, cuda)
    bias = _x(1, 2048, 6, cuda, std=0.5).view(-1)
    g = torch.Generator().manual_seed(3)
    bound = 1 / np.sqrt(k)
    a_q = ((torch.rand(r, k, generator=g) * 2 - 1) * bound).half().to(cuda)
    a_v = ((torch.rand(r, k, generator=g) * 2 - 1) * bound).half().to(cuda)
    g = torch.Generator().manual_seed(4)
    b_q = (torch.randn(1536, r, generator=g) * 0.01).half().to(cuda)
    b_v = (torch.randn(256, r, generator=g) * 0.01).half().to(cuda)
    t_q, t_v = kernels.lora_xa(x, a_q), kernels.lora_xa(x, a_v)
    assert_rel(t_q, x.float().cpu() @ a_q.float().cpu().t(), what="lora_xa")
    loras = [kernels.make_lora(0, r, s, t=t_q, b=b_q), kernels.make_lora(2, r, s, t=t_v, b=b_v)]
    y = kernels.linear_fwd(x, segs, bias, loras)
    ref = o.linear_fwd(x, w, bias, [(0, 1536, x, a_q, b_q, s), (1792, 256, x, a_v, b_v, s)])
    assert_rel(y, ref, what="qkv fwd")
    # the LoRA term alone is visible: compare the difference to the base
    base = o.linear_fwd(x, w, bias)
    lora_only = (y.float().cpu() - base)[:, :1536]
    assert_rel(lora_only, (ref - base)[:, :1536], max_rel=5e-2, mean_rel=5e-2, what="lora part")

    dy = _x(m, 2048, 2, cuda, std=1e-3)
    da_q = kernels.lora_da(dy[:, :1536], b_q, s)
    da_v = kernels.lora_da(dy[:, 1792:], b_v, s)
    assert_rel(da_q, s * dy[:, :1536].float().cpu() @ b_q.float().cpu(), what="lora_da")
    dl = [kernels.make_lora(0, r, s, a=a_q, da=da_q), kernels.make_lora(2, r, s, a=a_v, da=da_v)]
    dx = kernels.linear_dx(dy, segs, dl)
    ref_dx = o.linear_dx(dy, w, [(0, 1536, x, a_q, b_q, s), (1792, 256, x, a_v, b_v, s)])
    assert_rel(dx, ref_dx, what="qkv dx")
    ga, gb = o.lora_grads(dy[:, :1536], x, a_q, b_q, s)
    assert_rel(kernels.lora_wgrad(dy[:, :1536], t_q, s, False), gb, what="dB")
    assert_rel(kernels.lora_wgrad(x, da_q, 1.0, True), ga, what="dA")


def test_dx_accumulate_and_gate_up_stack(cuda):
    from solution import kernels

    banner("gemm dx accumulate, gate|up stack")
    m, k = 512, 1536
    segs = [random_weight(8960, k, seed=104 + i, dev=cuda) for i in range(2)]
    w = torch.cat([oracle_w16(p, q) for p, q in segs])
    dy = _x(m, 2 * 8960, 7, cuda, std=1e-3)
    base = _x(m, k, 8, cuda, std=1e-2)
    out = base.clone()
    kernels.linear_dx(dy, segs, out=out, accumulate=True)
    assert_rel(out, base.float().cpu() + o.linear_dx(dy, w), what="dx accumulate")
    x = _x(m, k, 9, cuda)
    assert_rel(kernels.linear_fwd(x, segs), o.linear_fwd(x, w), what="gate|up fwd")


def test_bias_grad_and_swiglu(cuda):
    from solution import kernels

    banner("bias grad, swiglu")
    dy = _x(300, 200, 10, cuda, std=1e-2)
    torch.testing.assert_close(kernels.bias_grad(dy).cpu(), dy.float().cpu().sum(0),
                               rtol=1e-5, atol=1e-5)
    gu = _x(64, 2 * 96, 11, cuda)
    h = kernels.swiglu_fwd(gu[:, :96], gu[:, 96:])
    g, u = gu[:, :96].float().cpu(), gu[:, 96:].float().cpu()
    torch.testing.assert_close(h.float().cpu(), o.silu(g) * u, rtol=2e-3, atol=2e-3)
    grad = _x(64, 96, 12, cuda)
    d = gu.clone()
    kernels.swiglu_bwd(grad, d[:, :96], d[:, 96:], d[:, :96], d[:, 96:])
    gg = g.clone().requires_grad_()
    uu = u.clone().requires_grad_()
    (o.silu(gg) * uu).backward(grad.float().cpu())
    torch.testing.assert_close(d[:, :96].float().cpu(), gg.grad, rtol=5e-3, atol=5e-3)
    torch.testing.assert_close(d[:, 96:].float().cpu(), uu.grad, rtol=5e-3, atol=5e-3)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,n,pad", [(0, 64, 0), (1, 8, 0), (37, 100, 0), (2048, 2048, 0),
                                     (5000, 264, 0), (300, 96, 3), (257, 2048, 8)])
def test_bias_grad_shapes(cuda, m, n, pad, dtype):
    """nf4_bias_grad (the column sum of nf4.py:100-101) on the 16-byte path (n and the row
    pitch multiples of 8) and the element path (n = 100, pitch n + 3), M = 0 and M beyond one
    row lane's stride; deterministic (two calls bit-equal).  fp32 sums in a fixed order: the
    error against the fp64 sum stays below 2e-5 of the column's absolute sum."""
    from solution import kernels

    banner(f"bias grad m={m} n={n} pad={pad} {dtype}")
    g = torch.Generator().manual_seed(m * 7 + n)
    full = (torch.randn(m, n + pad, generator=g) * 0.1).to(dtype)
    dy = full.to(cuda)[:, :n]
    got = kernels.bias_grad(dy)
    again = kernels.bias_grad(dy)
    assert torch.equal(got, again)
    ref = full[:, :n].double().sum(0)
    bound = 2e-5 * full[:, :n].double().abs().sum(0) + 1e-30
    err = (got.cpu().double() - ref).abs()
    assert bool((err <= bound).all()), float((err / bound).max())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [1, 3, 8, 16, 17, 33, 48, 64])
def test_small_m_stacked_bias_lora(cuda, m, dtype):
    """The small-M forward path (decode regime): stacked segments whose row counts are not
    multiples of its 32-row tiles, bias, LoRA on two segments; and a long reduction (split over
    workgroups, fp32 partials + fixed-order reduction)."""
    from solution import kernels

    banner("gemm small-M", m, dtype)
    dt = "bf16" if dtype == torch.bfloat16 else "f16"
    k, r, s = 640, 16, 2.0
    segs = [random_weight(n, k, seed=300 + n, dev=cuda) for n in (100, 36, 28)]
    w = torch.cat([oracle_w16(p, q, dt) for p, q in segs])
    x = _x(m, k, 31, cuda, dtype)
    bias = _x(1, 164, 32, cuda, dtype, std=0.5).view(-1)
    g = torch.Generator().manual_seed(33)
    a0 = ((torch.rand(r, k, generator=g) * 2 - 1) / k ** 0.5).to(dtype).to(cuda)
    a2 = ((torch.rand(r, k, generator=g) * 2 - 1) / k ** 0.5).to(dtype).to(cuda)
    b0 = (torch.randn(100, r, generator=g) * 0.05).to(dtype).to(cuda)
    b2 = (torch.randn(28, r, generator=g) * 0.05).to(dtype).to(cuda)
    t0, t2 = kernels.lora_xa(x, a0), kernels.lora_xa(x, a2)
    loras = [kernels.make_lora(0, r, s, t=t0, b=b0), kernels.make_lora(2, r, s, t=t2, b=b2)]
    y = kernels.linear_fwd(x, segs, bias, loras)
    ref = o.linear_fwd(x, w, bias, [(0, 100, x, a0, b0, s), (136, 28, x, a2, b2, s)])
    assert_rel(y, ref, what="small-M stacked fwd")
    # long K, two segments, bias, LoRA on the second: the reduction split over workgroups
    # (fp32 partials; the bias and the rounding in the fixed-order reduction kernel, the LoRA
    # term in the first split's partial)
    segs_d = [random_weight(n, 8960, seed=301 + n, dev=cuda) for n in (96, 40)]
    wd = torch.cat([oracle_w16(p, q, dt) for p, q in segs_d])
    xd = _x(m, 8960, 34, cuda, dtype)
    bd = _x(1, 136, 35, cuda, dtype, std=0.5).view(-1)
    ad = ((torch.rand(r, 8960, generator=g) * 2 - 1) / 8960 ** 0.5).to(dtype).to(cuda)
    bbd = (torch.randn(40, r, generator=g) * 0.05).to(dtype).to(cuda)
    td = kernels.lora_xa(xd, ad)
    yd = kernels.linear_fwd(xd, segs_d, bd, [kernels.make_lora(1, r, s, t=td, b=bbd)])
    assert_rel(yd, o.linear_fwd(xd, wd, bd, [(96, 40, xd, ad, bbd, s)]), what="small-M long K")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,r", [(1, 16), (3, 16), (8, 8), (8, 16), (16, 16), (17, 16), (32, 16),
                                 (8, 32), (33, 16), (64, 16), (100, 16)])
@pytest.mark.parametrize("shape", [((300, 64, 40), 640), ((1536, 256, 256), 1536)],
                         ids=["300+64+40x640", "qkv-1.5B"])
def test_forward_computes_lora_down_projection(cuda, shape, m, r, dtype):
    """An adapter with `a` set in the forward: the call computes t = x A^T itself (inside the
    skinny GEMM launch at 3 to 32 tokens with rank <= 16, ranks below 16 zero-padded; in a
    launch of its own at other token counts, rank 32, or on other paths), writes it to t and
    uses it.  t is nf4_lora_xa's up to a rounding step (the fp32 sums run in another order) and
    Y matches the call given the caller's t, and the fp32 oracle."""
    from solution import kernels

    rows, k = shape
    s = 2.0
    banner("forward with LoRA down-projection", rows, k, m, r, dtype)
    dt = "bf16" if dtype == torch.bfloat16 else "f16"
    segs = [random_weight(n, k, seed=400 + n, dev=cuda) for n in rows]
    w = torch.cat([oracle_w16(p, q, dt) for p, q in segs])
    x = _x(m, k, 41, cuda, dtype)
    bias = _x(1, sum(rows), 42, cuda, dtype, std=0.5).view(-1)
    g = torch.Generator().manual_seed(43)
    a0, a2 = [((torch.rand(r, k, generator=g) * 2 - 1) / k ** 0.5).to(dtype).to(cuda) for _ in range(2)]
    b0 = (torch.randn(rows[0], r, generator=g) * 0.05).to(dtype).to(cuda)
    b2 = (torch.randn(rows[2], r, generator=g) * 0.05).to(dtype).to(cuda)
    t_ref = [kernels.lora_xa(x, a0), kernels.lora_xa(x, a2)]
    y_given = kernels.linear_fwd(x, segs, bias, [kernels.make_lora(0, r, s, t=t_ref[0], b=b0),
                                                 kernels.make_lora(2, r, s, t=t_ref[1], b=b2)])
    t = [torch.full((m, r), float("nan"), dtype=dtype, device=cuda) for _ in range(2)]
    y = kernels.linear_fwd(x, segs, bias, [kernels.make_lora(0, r, s, t=t[0], b=b0, a=a0),
                                           kernels.make_lora(2, r, s, t=t[1], b=b2, a=a2)])
    eps = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
    for got, ref in zip(t, t_ref):
        scale = ref.float().abs().max().item()
        torch.testing.assert_close(got.float(), ref.float(), rtol=2 * eps, atol=eps * scale)
    assert_rel(y, y_given, what="forward with computed t vs given t")
    ref = o.linear_fwd(x, w, bias, [(0, rows[0], x, a0, b0, s), (sum(rows[:2]), rows[2], x, a2, b2, s)])
    assert_rel(y, ref, what="forward with computed t vs oracle")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,k,r", [(1, 3584, 16), (2, 1536, 16), (5, 2056, 8), (8, 4096, 16),
                                   (9, 1536, 16), (13, 3584, 12), (40, 2056, 16), (64, 3584, 16),
                                   (65, 1536, 16)])
def test_lora_xa_decode_sizes(cuda, dtype, m, k, r):
    """t = x A^T at decode token counts (up to 64 tokens: one workgroup per (adapter, A row,
    group of up to 8 tokens), the last group partly used; 65 tokens: the MFMA kernel), two
    adapters in one launch, against an fp32 product; K not a multiple of the 2048-wide step."""
    from solution import kernels

    banner("lora xa decode", dtype, m, k, r)
    x = _x(m, k, 51, cuda, dtype)
    g = torch.Generator().manual_seed(52)
    a = [((torch.rand(r, k, generator=g) * 2 - 1) / k ** 0.5).to(dtype).to(cuda) for _ in range(2)]
    t = [torch.empty(m, r, dtype=dtype, device=cuda) for _ in range(2)]
    kernels.lora_xa_multi([kernels.lora_job(x, a[i], t[i], 1.5) for i in range(2)], m, r, dtype, x)
    for i in range(2):
        ref = 1.5 * (x.float().cpu() @ a[i].float().cpu().t())
        assert_rel(t[i], ref, what=f"xa {i}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,k,r", [(1, 1536, 16), (37, 3584, 16), (300, 1536, 64), (19, 200, 5)])
def test_lora_ax(cuda, dtype, m, k, r):
    """d(xd) = scale * da A ([M, K]) for two jobs of different widths in one launch, against an
    fp32 product (rounded once, so within the path's tolerance)."""
    from solution import kernels

    banner("lora ax", dtype, m, k, r)
    da = [_x(m, r, 61 + i, cuda, dtype) for i in range(2)]
    g = torch.Generator().manual_seed(63)
    a = [(torch.randn(r, kk, generator=g) / r ** 0.5).to(dtype).to(cuda) for kk in (k, k // 2 + 8)]
    out = [torch.empty(m, aa.shape[1], dtype=dtype, device=cuda) for aa in a]
    kernels.lora_ax_multi([kernels.lora_ax_job(da[i], a[i], out[i], 0.5 + i) for i in range(2)],
                          m, r, dtype, da[0])
    for i in range(2):
        ref = (0.5 + i) * (da[i].float().cpu() @ a[i].float().cpu())
        assert_rel(out[i], ref, what=f"ax {i}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_lora_multi_matches_single(cuda, dtype):
    """The multi-job LoRA launches give the single-job results bit for bit (same kernels, same
    order of arithmetic), with jobs on column ranges of a stacked gradient."""
    from solution import kernels

    banner("lora multi", dtype)
    m, k, r = 300, 512, 16
    x = _x(m, k, 41, cuda, dtype)
    dy = _x(m, 768, 42, cuda, dtype, std=1e-3)
    g = torch.Generator().manual_seed(43)
    a = [((torch.rand(r, k, generator=g) * 2 - 1) / k ** 0.5).to(dtype).to(cuda) for _ in range(2)]
    b = [(torch.randn(n, r, generator=g) * 0.05).to(dtype).to(cuda) for n in (512, 128)]
    cols = [dy[:, :512], dy[:, 640:]]
    t = [torch.empty(m, r, dtype=dtype, device=cuda) for _ in range(2)]
    kernels.lora_xa_multi([kernels.lora_job(x, a[i], t[i]) for i in range(2)], m, r, dtype, x)
    for i in range(2):
        assert torch.equal(t[i], kernels.lora_xa(x, a[i]))
    da = [torch.empty(m, r, dtype=dtype, device=cuda) for _ in range(2)]
    kernels.lora_da_multi([kernels.lora_job(cols[i], b[i], da[i], 2.0) for i in range(2)], m, r,
                          dtype, x)
    for i in range(2):
        assert torch.equal(da[i], kernels.lora_da(cols[i].contiguous(), b[i], 2.0))
    gb = [torch.empty(n, r, dtype=torch.float32, device=cuda) for n in (512, 128)]
    ga = [torch.empty(r, k, dtype=torch.float32, device=cuda) for _ in range(2)]
    jobs = [kernels.lora_job(cols[i], t[i], gb[i], 2.0) for i in range(2)] + \
        [kernels.lora_job(x, da[i], ga[i], 1.0, transpose_out=True) for i in range(2)]
    kernels.lora_wgrad_multi(jobs, m, r, dtype, x)
    for i in range(2):
        ref_b = kernels.lora_wgrad(cols[i].contiguous(), t[i], 2.0, False)
        ref_a = kernels.lora_wgrad(x, da[i], 1.0, True)
        ga_o, gb_o = o.lora_grads(cols[i], x, a[i], b[i], 2.0)
        assert_rel(gb[i], gb_o, mean_rel=3e-3 if dtype == torch.bfloat16 else 1e-3, what="dB")
        assert_rel(ga[i], ga_o, mean_rel=3e-3 if dtype == torch.bfloat16 else 1e-3, what="dA")
        # the multi launch reduces over the widest job's chunking: equal within fp32 rounding
        torch.testing.assert_close(gb[i], ref_b, rtol=1e-5, atol=1e-7)
        torch.testing.assert_close(ga[i], ref_a, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,n,rank,offset", [(300, 1000, 8, 0), (2048, 1536, 16, 0),
                                             (77, 256, 24, 0), (129, 640, 64, 0),
                                             (300, 1000, 12, 0), (200, 512, 16, 1)])
def test_lora_da_xa_ranks(cuda, m, n, rank, offset, dtype):
    """da = s dY B and t = X A^T at ranks 8..64 (B rows 16-byte loadable through the LDS
    transpose, or strided gathers: rank 12, or B starting one element in) against fp64 sums of
    the same 16-bit inputs."""
    from solution import kernels

    banner("lora da/xa ranks", m, n, rank, offset, dtype)
    dy = _x(m, n, 71, cuda, dtype, std=0.1)
    bbuf = _x(n * rank + offset, 1, 72, cuda, dtype, std=0.1).view(-1)
    b = bbuf[offset:].view(n, rank)
    da = kernels.lora_da(dy, b, 1.5)
    ref = 1.5 * (dy.double().cpu() @ b.double().cpu())
    assert_rel(da, ref.float(), what="da")
    a = _x(rank, n, 73, cuda, dtype, std=0.1)
    t = kernels.lora_xa(dy, a)
    assert_rel(t, (dy.double().cpu() @ a.double().cpu().t()).float(), what="xa")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,p,ld,rank,transpose", [
    (2048, 1536, 2048, 16, False),  # one pass over M (aligned rows, ld % 8 == 0, rank % 8 == 0)
    (300, 100, 104, 8, True),       # ... p not a multiple of the 32-column tile
    (1, 256, 256, 32, False),
    (1243, 1000, 1000, 64, True),
    (37, 72, 72, 24, False),
    (300, 100, 101, 16, False),     # row chunks + final pass: rows not 16-byte loadable
    (5000, 64, 64, 16, True),       # ... long M over few workgroups
    (200, 96, 96, 12, False),       # ... rank not a multiple of 8
])
def test_lora_wgrad_paths(cuda, m, p, ld, rank, transpose, dtype):
    """LoRA weight gradients scale * U^T V (fp32 out, [P, r] or [r, P]) on both kernels (one
    pass over M, or row chunks with a final fixed-order pass) against fp64 sums of the same
    16-bit inputs; a second call gives the same bits."""
    from solution import kernels

    banner("lora wgrad", m, p, ld, rank, transpose, dtype)
    base = _x(m, ld, 61, cuda, dtype)
    u = base[:, ld - p:] if (ld - p) % 8 == 0 else base[:, :p]  # rows ld elements apart
    v = _x(m, rank, 62, cuda, dtype, std=0.1)
    out = kernels.lora_wgrad(u, v, 0.5, transpose)
    ref = 0.5 * (u.double().cpu().t() @ v.double().cpu())
    if transpose:
        ref = ref.t()
    assert tuple(out.shape) == tuple(ref.shape)
    assert_rel(out, ref.float(), max_rel=1e-4, mean_rel=1e-5, what="wgrad")
    assert torch.equal(out, kernels.lora_wgrad(u, v, 0.5, transpose))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,inter,k", [(2048, 8960, 1536), (300, 200, 320), (129, 1000, 256)])
def test_swiglu_epilogue(cuda, m, inter, k, dtype):
    """gate | up with the SwiGLU step in the GEMM epilogue: H = silu(g) u and the gradients
    dG = dH u silu'(g), dU = dH silu(g) against the fp32 oracle (g, u = X W^T on the bit-exact
    weights), at the Qwen2.5-1.5B MLP shape and ragged ones (I not a multiple of the tile)."""
    from solution import kernels

    banner("swiglu epilogue", m, inter, k, dtype)
    dt = "bf16" if dtype == torch.bfloat16 else "f16"
    gate = random_weight(inter, k, seed=inter + 1, dev=cuda)
    up = random_weight(inter, k, seed=inter + 2, dev=cuda)
    wg, wu = oracle_w16(*gate, dt), oracle_w16(*up, dt)
    x = _x(m, k, 61, cuda, dtype)
    dh = _x(m, inter, 62, cuda, dtype, std=1e-2)
    g, u = o.linear_fwd(x, wg), o.linear_fwd(x, wu)
    sig = 1.0 / (1.0 + torch.exp(-g))
    h = kernels.linear_swiglu_fwd(x, gate, up)
    assert_rel(h, g * sig * u, what="H")
    dgu = kernels.linear_swiglu_bwd(x, gate, up, dh)
    d = dh.float().cpu()
    assert_rel(dgu[:, :inter], d * u * sig * (1.0 + g * (1.0 - sig)), what="dG")
    assert_rel(dgu[:, inter:], d * g * sig, what="dU")


def _scaled_codes(p, qs, dtype):
    from tests.gpu_util import to_oracle_state

    pn, st = to_oracle_state(p, qs)
    w = o.dequantize_scaled_codes(pn, st, "bf16" if dtype == torch.bfloat16 else "f16")
    return torch.from_numpy(w.view(np.int16))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [1, 2])
@pytest.mark.parametrize("shapes,bs,nested", [([(384, 256)], 64, True), ([(200, 512)], 128, True),
                                              ([(136, 320)], 64, False),
                                              ([(256, 512), (64, 512), (64, 512)], 64, True),
                                              ([(200, 3584)], 64, True),
                                              ([(96, 2560), (40, 2560)], 128, False),
                                              ([(72, 9472)], 64, True)])
def test_rows_decode_one_hot_is_exact(cuda, m, shapes, bs, nested, dtype):
    """The row-streaming decode path (M <= 2): token t one-hot at column c_t returns the weight
    column c_t as the GEMV multiplies it - round(fp32(round(code)) * absmax) - bit for bit, over
    every row of every stacked segment, for columns spread over the reduction.  K <= 2048 runs
    the one-copy pair table, longer rows the 64-copy table (two slots per part; K = 9472 in
    three parts)."""
    from solution import kernels

    banner("rows decode one-hot", m, shapes, bs, nested, dtype)
    ws = [random_weight(n, k, seed=7 * n + k + i, dev=cuda, blocksize=bs, nested=nested)
          for i, (n, k) in enumerate(shapes)]
    k = shapes[0][1]
    ref = torch.cat([_scaled_codes(p, q, dtype) for p, q in ws])  # [sum rows, K] bits
    for c0 in range(0, k, max(1, k // 6)):
        cols = [(c0 + 37 * t) % k for t in range(m)]
        x = torch.zeros(m, k, dtype=dtype)
        x[torch.arange(m), cols] = 1.0
        y = kernels.linear_fwd(x.to(cuda), ws)
        assert torch.equal(y.cpu().view(torch.int16), ref[:, cols].t()), (c0, cols)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [1, 2])
@pytest.mark.parametrize("shape", [(1536, 1536), (512, 3584), (256, 8960)])
def test_rows_decode_against_fp32_code_product(cuda, m, shape, dtype):
    """The row-streaming path (M <= 2) against the product bitsandbytes' decode GEMV forms, fp32
    code x fp32 absmax x activation (the reference's small-M numerics, nf4.py:15-16, 105-118),
    with the bound that follows from its one deviation: the 16 codes enter the GEMM rounded to
    its dtype, a relative error of at most u = 2^-9 (bf16) or 2^-12 (fp16) per code, so for
    every output n
        |y - sum_k W32[n,k] x[k]| <= u sum_k |W32[n,k] x[k]| + 2u |y_ref| + 2^-20 sum_k |W32 x|
    (code rounding, the final rounding to the dtype, fp32 accumulation).  Activations of mixed
    sign and magnitude, K of one, two and five 1 KB slots."""
    from solution import kernels
    from tests.gpu_util import to_oracle_state

    n, k = shape
    banner("rows decode vs fp32-code product", m, shape, dtype)
    p, qs = random_weight(n, k, seed=n + 5 * k, dev=cuda)
    pn, st = to_oracle_state(p, qs)
    w32 = torch.from_numpy(o.dequantize(pn, st, "f32")).double()  # fp32(code * absmax)
    x = _x(m, k, 61, cuda, dtype)
    y = kernels.linear_fwd(x, [(p, qs)]).double().cpu()
    xd = x.double().cpu()
    ref = xd @ w32.t()
    mag = xd.abs() @ w32.abs().t()
    u = 2.0 ** -9 if dtype == torch.bfloat16 else 2.0 ** -12
    bound = u * mag + 2 * u * ref.abs() + 2.0 ** -20 * mag
    err = (y - ref).abs()
    assert bool((err <= bound).all()), f"max excess {(err - bound).max().item():.3e}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_rows_decode_qkv_bias_lora(cuda, m, dtype):
    """Stacked q|k|v with bias and LoRA on q and v at M <= 4 tokens (the row-streaming path up to
    2 tokens, the decode kernel above) against fp32 on the oracle's weight (the row-streaming
    path's rounding of the code table is inside the tolerance)."""
    from solution import kernels

    banner("rows decode q|k|v + bias + LoRA", m, dtype)
    k, r, s = 1536, 16, 2.0
    segs = [random_weight(n, k, seed=300 + i, dev=cuda) for i, n in enumerate((1536, 256, 256))]
    wname = "bf16" if dtype == torch.bfloat16 else "f16"
    w = torch.cat([oracle_w16(p, q, wname) for p, q in segs])
    x = _x(m, k, 11, cuda, dtype)
    bias = _x(1, 2048, 12, cuda, dtype, std=0.5).view(-1)
    g = torch.Generator().manual_seed(13)
    a_q = ((torch.rand(r, k, generator=g) * 2 - 1) / np.sqrt(k)).to(dtype).to(cuda)
    a_v = ((torch.rand(r, k, generator=g) * 2 - 1) / np.sqrt(k)).to(dtype).to(cuda)
    b_q = (torch.randn(1536, r, generator=g) * 0.05).to(dtype).to(cuda)
    b_v = (torch.randn(256, r, generator=g) * 0.05).to(dtype).to(cuda)
    t_q, t_v = kernels.lora_xa(x, a_q), kernels.lora_xa(x, a_v)
    loras = [kernels.make_lora(0, r, s, t=t_q, b=b_q), kernels.make_lora(2, r, s, t=t_v, b=b_v)]
    y = kernels.linear_fwd(x, segs, bias, loras)
    ref = o.linear_fwd(x, w, bias, [(0, 1536, x, a_q, b_q, s), (1792, 256, x, a_v, b_v, s)])
    assert_rel(y, ref, what=f"q|k|v M={m}")


@pytest.mark.parametrize("m,n,k", [(1, 512, 18944), (2, 384, 8960), (1, 100, 64), (2, 72, 1024)])
def test_rows_decode_long_and_odd_rows(cuda, m, n, k):
    """Long rows (the 7B down projection's K = 18944: 37 units per lane), rows whose K / 8 units
    leave lanes idle (K = 64, 1024), an output width not a multiple of 8."""
    from solution import kernels

    banner("rows decode shapes", m, n, k)
    p, qs = random_weight(n, k, seed=n + k, dev=cuda)
    x = _x(m, k, 14, cuda)
    bias = _x(1, n, 15, cuda, std=0.1).view(-1)
    y = kernels.linear_fwd(x, [(p, qs)], bias)
    assert_rel(y, o.linear_fwd(x, oracle_w16(p, qs), bias), what=f"M={m} {n}x{k}")


@pytest.mark.parametrize("r", [1, 8, 17, 32, 48, 64])
@pytest.mark.parametrize("tile", [None, 0, 1, 3])
def test_lora_slab_ranks(cuda, r, tile):
    """The LoRA slabs of the fused forward and input-gradient GEMMs at ranks 1..64 (the ABI's
    range): the slab runs the rank in 16-deep MFMA chunks with the ranks past r masked, so
    ranks that are not a multiple of 16 and several chunks are the cases; every tiling.  The
    LoRA term is made large (B ~ N(0, 0.2)) so that it is checked on its own as well."""
    from solution import kernels

    banner("lora slab rank", r, "tile", tile)
    m, k, s = 300, 512, 0.5
    rows = (320, 64, 64)
    segs = [random_weight(n, k, seed=500 + i, dev=cuda) for i, n in enumerate(rows)]
    w = torch.cat([oracle_w16(p, q) for p, q in segs])
    x = _x(m, k, 11, cuda)
    g = torch.Generator().manual_seed(12)
    a0 = ((torch.rand(r, k, generator=g) * 2 - 1) / np.sqrt(k)).half().to(cuda)
    a2 = ((torch.rand(r, k, generator=g) * 2 - 1) / np.sqrt(k)).half().to(cuda)
    b0 = (torch.randn(rows[0], r, generator=g) * 0.2).half().to(cuda)
    b2 = (torch.randn(rows[2], r, generator=g) * 0.2).half().to(cuda)
    t0, t2 = kernels.lora_xa(x, a0), kernels.lora_xa(x, a2)
    loras = [kernels.make_lora(0, r, s, t=t0, b=b0), kernels.make_lora(2, r, s, t=t2, b=b2)]
    y = kernels.linear_fwd(x, segs, None, loras, tile=tile)
    spec = [(0, rows[0], x, a0, b0, s), (rows[0] + rows[1], rows[2], x, a2, b2, s)]
    ref = o.linear_fwd(x, w, None, spec)
    assert_rel(y, ref, what=f"fwd r={r}")
    base = o.linear_fwd(x, w)
    assert_rel((y.float().cpu() - base)[:, :rows[0]], (ref - base)[:, :rows[0]], max_rel=5e-2,
               mean_rel=5e-2, what=f"lora part r={r}")

    dy = _x(m, sum(rows), 13, cuda, std=1e-2)
    da0 = kernels.lora_da(dy[:, :rows[0]], b0, s)
    da2 = kernels.lora_da(dy[:, rows[0] + rows[1]:], b2, s)
    dl = [kernels.make_lora(0, r, s, a=a0, da=da0), kernels.make_lora(2, r, s, a=a2, da=da2)]
    dx = kernels.linear_dx(dy, segs, dl, tile=tile)
    ref_dx = o.linear_dx(dy, w, spec)
    assert_rel(dx, ref_dx, what=f"dx r={r}")
    base_dx = o.linear_dx(dy, w)
    assert_rel(dx.float().cpu() - base_dx, ref_dx - base_dx, max_rel=5e-2, mean_rel=5e-2,
               what=f"dx lora part r={r}")
