"""The bitsandbytes patch surface driven end to end on the GPU through a stand-in bitsandbytes
(tests/bnb_standin.py): `patch_linear4bit` and `patch_bnb_matmul_4bit` (reference
solution/nf4.py:148-216) and `patch_qwen2_mlp_recompute` (mlp.py:123-157, transformers' own
Qwen2MLP).  Each case asserts which path ran - the HIP kernels or bitsandbytes' original
function - and checks the HIP results against fp32 on the oracle's dequantized weight (max rel
1e-2, mean rel 1e-3; the fp32 GEMM path to 1e-5).  Routing rules: fp16 / bf16 GEMMs with a
fused layout and fp32 GEMMs go to the HIP path; `out=`, a layout outside the fused kernels
(blocksize 32) and CPU inputs go to the original."""

import pytest
import torch

from oracle import nf4_oracle as o
from tests import bnb_standin
from tests.gpu_util import assert_rel, banner, oracle_w16, random_weight

pytestmark = pytest.mark.gpu


@pytest.fixture
def bnb(monkeypatch, cuda):
    from solution import nf4

    mod, calls = bnb_standin.install(monkeypatch)
    nf4.patch_linear4bit()
    nf4.patch_bnb_matmul_4bit()
    return mod, calls


def _ref(x, w, bias=None):
    xr = x.detach().float().cpu().requires_grad_()
    br = None if bias is None else bias.detach().float().cpu().requires_grad_()
    y = torch.nn.functional.linear(xr, w.float(), br)
    return xr, br, y


def test_linear4bit_fp16_autocast_runs_the_fused_kernels(bnb, cuda):
    """The reference's training setting: fp32 residual input, compute dtype fp32 (after
    prepare_model_for_kbit_training), fp16 autocast -> the fp16 fused GEMM (nf4.py:140-145,
    174-191), bias cast to the compute dtype."""
    mod, calls = bnb
    banner("patch Linear4bit fp16 autocast")
    p, qs = random_weight(256, 1536, seed=0, dev=cuda, std=0.05)
    bias = torch.nn.Parameter((torch.randn(256) * 0.1).to(cuda))
    layer = mod.nn.Linear4bit(p, qs, bias=bias, compute_dtype=torch.float32)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 100, 1536, generator=g).to(cuda).requires_grad_()
    with torch.autocast("cuda", dtype=torch.float16):
        y = layer(x)
    assert calls.forward == 0 and calls.fix_state == 1
    assert y.dtype == torch.float16 and y.shape == (3, 100, 256)
    dy = (torch.randn(3, 100, 256, generator=g) * 1e-2).half().to(cuda)
    y.backward(dy)
    # the reference's numerics: x rounded to fp16, the bit-exact fp16 weight, fp32 accumulation
    xr, br, yr = _ref(x.detach().half(), oracle_w16(p, qs), bias)
    yr.backward(dy.float().cpu())
    assert_rel(y, yr.detach(), what="y")
    assert x.grad.dtype == torch.float32
    assert_rel(x.grad, xr.grad, what="dx")
    assert_rel(bias.grad, br.grad, max_rel=1e-3, mean_rel=1e-3, what="dbias")


def test_linear4bit_fp32_runs_dequant_and_fp32_gemm(bnb, cuda):
    """No autocast and no half compute dtype: an fp32 GEMM on the weight the HIP kernel
    dequantized to fp32 (the reference's NF4Linear in fp32, nf4.py:84-102)."""
    mod, calls = bnb
    banner("patch Linear4bit fp32")
    p, qs = random_weight(192, 512, seed=1, dev=cuda, std=0.05)
    layer = mod.nn.Linear4bit(p, qs)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(37, 512, generator=g).to(cuda).requires_grad_()
    y = layer(x)
    assert calls.forward == 0 and y.dtype == torch.float32
    dy = torch.randn(37, 192, generator=g).to(cuda)
    y.backward(dy)
    w32 = torch.from_numpy(o.dequantize_f32(*_oracle(p, qs)))
    xr, _, yr = _ref(x, w32)
    yr.backward(dy.cpu())
    assert_rel(y, yr.detach(), max_rel=1e-5, mean_rel=1e-5, what="y fp32")
    assert_rel(x.grad, xr.grad, max_rel=1e-5, mean_rel=1e-5, what="dx fp32")


def test_linear4bit_bf16_and_out_width_not_multiple_of_8(bnb, cuda):
    """bf16 autocast through the fused kernels, at an output width of 100 (the input gradient
    reads dY through a padded copy)."""
    mod, calls = bnb
    banner("patch Linear4bit bf16 N=100")
    p, qs = random_weight(100, 256, seed=2, dev=cuda, std=0.05)
    layer = mod.nn.Linear4bit(p, qs, compute_dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 129, 256, generator=g).to(torch.bfloat16).to(cuda).requires_grad_()
    y = layer(x)
    assert calls.forward == 0 and y.dtype == torch.bfloat16
    dy = (torch.randn(2, 129, 100, generator=g) * 1e-2).to(torch.bfloat16).to(cuda)
    y.backward(dy)
    xr, _, yr = _ref(x, oracle_w16(p, qs, "bf16"))
    yr.backward(dy.float().cpu())
    assert_rel(y, yr.detach(), what="y bf16")
    assert_rel(x.grad, xr.grad, what="dx bf16")


def test_nf4_linear_output_width_100(cuda):
    """NF4Linear forward and backward at N = 100 (not a multiple of 8), fp16, with bias."""
    from solution.nf4 import NF4Linear

    banner("NF4Linear N=100")
    p, qs = random_weight(100, 320, seed=3, dev=cuda, std=0.05)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(57, 320, generator=g).half().to(cuda).requires_grad_()
    bias = (torch.randn(100, generator=g) * 0.1).half().to(cuda).requires_grad_()
    y = NF4Linear.apply(x, p, qs, bias)
    dy = (torch.randn(57, 100, generator=g) * 1e-2).half().to(cuda)
    y.backward(dy)
    xr, br, yr = _ref(x, oracle_w16(p, qs), bias)
    yr.backward(dy.float().cpu())
    assert_rel(y, yr.detach(), what="y")
    assert_rel(x.grad, xr.grad, what="dx")
    assert_rel(bias.grad, br.grad, max_rel=1e-3, mean_rel=1e-3, what="dbias")


def test_linear4bit_unfused_layout_goes_to_original(bnb, cuda):
    mod, calls = bnb
    banner("patch Linear4bit blocksize 32")
    p, qs = random_weight(64, 256, seed=4, dev=cuda, blocksize=32)
    layer = mod.nn.Linear4bit(p, qs, compute_dtype=torch.float16)
    x = torch.randn(8, 256).half().to(cuda)
    layer(x)
    assert calls.forward == 1
    layer(x.cpu())  # CPU input: the original as well
    assert calls.forward == 2


def test_matmul_4bit_routing(bnb, cuda):
    mod, calls = bnb
    banner("patch matmul_4bit")
    p, qs = random_weight(256, 512, seed=5, dev=cuda, std=0.05)
    w = oracle_w16(p, qs)
    g = torch.Generator().manual_seed(5)
    a = torch.randn(33, 512, generator=g).half().to(cuda)
    bias = (torch.randn(256, generator=g) * 0.1).half().to(cuda)
    y = mod.matmul_4bit(a, p.view(-1, 1), qs, bias=bias)
    assert calls.matmul == 0
    assert_rel(y, _ref(a, w, bias)[2].detach(), what="matmul_4bit fp16")
    assert mod.autograd._functions.matmul_4bit is mod.matmul_4bit
    out = torch.empty(33, 256, dtype=torch.float16, device=cuda)
    mod.matmul_4bit(a, p.view(-1, 1), qs, out=out, bias=bias)
    assert calls.matmul == 1  # out= is the original's
    a32 = a.float()
    y32 = mod.matmul_4bit(a32, p.view(-1, 1), qs)
    assert calls.matmul == 1 and y32.dtype == torch.float32
    w32 = torch.from_numpy(o.dequantize_f32(*_oracle(p, qs)))
    assert_rel(y32, _ref(a32, w32)[2].detach(), max_rel=1e-5, mean_rel=1e-5, what="fp32")


def test_patches_are_idempotent(bnb):
    from solution import nf4

    mod, _ = bnb
    fwd, mm = mod.nn.modules.Linear4bit.forward, mod.matmul_4bit
    nf4.patch_linear4bit()
    nf4.patch_bnb_matmul_4bit()
    assert mod.nn.modules.Linear4bit.forward is fwd and mod.matmul_4bit is mm


def test_qwen2_mlp_patch_runs_recomputed_mlp(monkeypatch, cuda):
    """transformers' Qwen2MLP with stand-in Linear4bit projections under fp16 autocast: the
    patched forward runs RecomputedMLP (no Linear4bit.forward call), forward and input gradient
    within tolerance of fp32; without grad it keeps the previous forward (mlp.py:131-143)."""
    from transformers import Qwen2Config
    from transformers.models.qwen2 import modeling_qwen2

    from solution.mlp import patch_qwen2_mlp_recompute

    mod, calls = bnb_standin.install(monkeypatch)
    monkeypatch.setattr(modeling_qwen2.Qwen2MLP, "forward", modeling_qwen2.Qwen2MLP.forward)
    banner("patch Qwen2MLP")
    h, inter = 512, 1024
    mlp = modeling_qwen2.Qwen2MLP(Qwen2Config(hidden_size=h, intermediate_size=inter,
                                              hidden_act="silu"))
    ws = {"gate": random_weight(inter, h, seed=11, dev=cuda, std=0.05),
          "up": random_weight(inter, h, seed=12, dev=cuda, std=0.05),
          "down": random_weight(h, inter, seed=13, dev=cuda, std=0.05)}
    for name, (p, qs) in ws.items():
        setattr(mlp, name + "_proj", mod.nn.Linear4bit(p, qs, compute_dtype=torch.float32))
    patch_qwen2_mlp_recompute()
    g = torch.Generator().manual_seed(6)
    x = torch.randn(1, 200, h, generator=g).to(cuda).requires_grad_()
    with torch.autocast("cuda", dtype=torch.float16):
        y = mlp(x)
    assert calls.forward == 0 and y.dtype == torch.float16
    dy = torch.randn(1, 200, h, generator=g).half().to(cuda)
    y.backward(dy)
    wg, wu, wd = (oracle_w16(*ws[n]).float() for n in ("gate", "up", "down"))
    xr = x.detach().half().float().cpu().requires_grad_()
    yr = o.mlp_fwd(xr, wg, wu, wd)
    yr.backward(dy.float().cpu())
    assert_rel(y, yr.detach(), what="mlp y")
    assert_rel(x.grad, xr.grad, what="mlp dx")
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16):
        mlp(x)
    assert calls.forward == 3  # gate, up, down through the (stand-in) original


def _oracle(p, qs):
    from tests.gpu_util import to_oracle_state

    return to_oracle_state(p, qs)
