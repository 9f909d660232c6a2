"""The benchmark's own workloads checked against the oracle at their real shapes:

* config 3: the Qwen2.5-1.5B projection stack (layers 0 and 1 of the benchmark's 28, seeds
  1000 + 7 l + i) on the benchmark's varlen batch (4 lengths from U{64..512}, seed 5,
  concatenated through cu_seqlens; unpad.py:249-250, 283-292): every output, input gradient and
  LoRA gradient of both layers;
* config 4: one Qwen2.5-7B layer (seeds 2000 + i) in bf16 at M = 8192, forward, input gradients
  and LoRA gradients (outputs compared on a fixed sample of 256 rows: rows are independent, so
  the sample checks the same GEMM launches the benchmark times at a CPU cost of seconds; the
  LoRA gradients sum over all rows and are checked whole);
* the decode sweep: the forward of all seven projections at M in {1, 8, 64}, 1.5B (fp16) and
  7B (bf16);
* the M = 2048 plans the benchmark times for the stacked gate|up forward and input gradient and
  the down forward (split-K): one-hot activations pick single weight rows / columns, which the
  GEMM must return bit for bit, and seeded random inputs within tolerance.

Tolerance: fp16 max rel <= 1e-2 and mean rel <= 1e-3; bf16 mean rel <= 3e-3."""

import pytest
import torch

from oracle import nf4_oracle as o
from tests.gpu_util import assert_rel, banner, oracle_w16, random_weight

pytestmark = pytest.mark.gpu

RANK, ALPHA = 16, 32


def _bench_cu_seqlens():
    """The benchmark's varlen batch (bench.py varlen_stack_leg)."""
    g = torch.Generator().manual_seed(5)
    lens = torch.randint(64, 513, (4,), generator=g)
    cu = torch.zeros(5, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0)
    return cu


def _weights16(layer, dt):
    return {n: oracle_w16(*layer[n], dt) for n in layer}


def _check_layer(st, li, W, rows=None, what=""):
    """Forward, backward and LoRA gradients of layer li of a ProjectionStack vs the oracle on
    the rows `rows` (None: all of the current M)."""
    m, s, L = st.m, st.scale, st.per_layer[li]
    h, kv = st.shape.hidden, st.shape.kv
    sel = (lambda t: t[:m]) if rows is None else (lambda t: t[:m][rows])
    wqkv = torch.cat([W["q"], W["k"], W["v"]])
    wgu = torch.cat([W["gate"], W["up"]])
    x, attn, x2, act = (t[:m] for t in (st.x, st.attn, st.x2, st.act))
    st.forward(layers=[li])
    torch.cuda.synchronize()
    lor = [(0, h, sel(x), L["a_q"], L["b_q"], s), (h + kv, kv, sel(x), L["a_v"], L["b_v"], s)]
    assert_rel(sel(st.y_qkv), o.linear_fwd(sel(x), wqkv, L["bias"], lor), what=f"{what} qkv")
    assert_rel(sel(st.y_o), o.linear_fwd(sel(attn), W["o"]), what=f"{what} o")
    assert_rel(sel(st.y_gu), o.linear_fwd(sel(x2), wgu), what=f"{what} gate|up")
    assert_rel(sel(st.y_d), o.linear_fwd(sel(act), W["down"]), what=f"{what} down")
    if rows is not None or m > 64:  # the decode sweep checks the forward only
        dy_qkv, dy_o, dy_gu, dy_d = (t[:m] for t in (st.dy_qkv, st.dy_o, st.dy_gu, st.dy_d))
        st.backward(layers=[li])
        torch.cuda.synchronize()
        assert_rel(sel(st.dx_d), o.linear_dx(sel(dy_d), W["down"]), what=f"{what} dx down")
        assert_rel(sel(st.dx_gu), o.linear_dx(sel(dy_gu), wgu), what=f"{what} dx gate|up")
        assert_rel(sel(st.dx_o), o.linear_dx(sel(dy_o), W["o"]), what=f"{what} dx o")
        assert_rel(sel(st.dx_qkv), o.linear_dx(sel(dy_qkv), wqkv, lor), what=f"{what} dx qkv")
        ga_q, gb_q = o.lora_grads(dy_qkv[:, :h], x, L["a_q"], L["b_q"], s)
        ga_v, gb_v = o.lora_grads(dy_qkv[:, h + kv:], x, L["a_v"], L["b_v"], s)
        # fp32 gradients from operands stored in the GEMM dtype between kernels (t, da)
        mean = 3e-3 if st.dtype == torch.bfloat16 else 1e-3
        for name, got, ref in (("dB_q", L["gb_q"], gb_q), ("dA_q", L["ga_q"], ga_q),
                               ("dB_v", L["gb_v"], gb_v), ("dA_v", L["ga_v"], ga_v)):
            assert_rel(got, ref, mean_rel=mean, what=f"{what} {name}")


@pytest.fixture(scope="module")
def stack_15b(cuda):
    from solution.stack import QWEN2_15B, ProjectionStack

    cu = _bench_cu_seqlens()
    st = ProjectionStack.synthetic(QWEN2_15B, 2, int(cu[-1]), torch.float16, cuda,
                                   seed_base=1000, seed_stride=7, rank=RANK, alpha=ALPHA)
    W = [_weights16(w, "f16") for w in st.layers]
    yield st, cu, W
    del st
    torch.cuda.empty_cache()


@pytest.fixture(scope="module")
def stack_7b(cuda):
    from solution.stack import QWEN2_7B, ProjectionStack

    st = ProjectionStack.synthetic(QWEN2_7B, 1, 8192, torch.bfloat16, cuda, seed_base=2000,
                                   seed_stride=7, rank=RANK, alpha=ALPHA)
    W = _weights16(st.layers[0], "bf16")
    yield st, W
    del st
    torch.cuda.empty_cache()


@pytest.mark.parametrize("li", [0, 1])
def test_config3_varlen_stack_15b(stack_15b, li):
    st, cu, W = stack_15b
    banner("config 3 stack layer", li, cu.tolist())
    m = st.set_tokens(cu)
    assert m == int(cu[-1]) and 256 <= m <= 2048
    _check_layer(st, li, W[li], what=f"L{li}")


def test_config4_qwen7b_bf16_m8192(stack_7b):
    st, W = stack_7b
    banner("config 4 Qwen2.5-7B bf16 M=8192")
    st.set_tokens([0, 8192])
    rows = torch.randperm(8192, generator=torch.Generator().manual_seed(8192))[:256].sort().values
    _check_layer(st, 0, W, rows=rows.to(st.dev), what="7B")


@pytest.mark.parametrize("m", [1, 8, 64])
def test_decode_sweep_15b(stack_15b, m):
    st, _, W = stack_15b
    banner("decode 1.5B M =", m)
    st.set_tokens([0, m])
    _check_layer(st, 0, W[0], what=f"1.5B M={m}")


@pytest.mark.parametrize("m", [1, 8, 64])
def test_decode_sweep_7b(stack_7b, m):
    st, W = stack_7b
    banner("decode 7B M =", m)
    st.set_tokens([0, m])
    _check_layer(st, 0, W, what=f"7B M={m}")


# --------------------------------------------- the M = 2048 plans of the benchmark, one-hot

@pytest.fixture(scope="module")
def mlp_15b(cuda):
    # the benchmark's layer: seeds 100 + i for q, k, v, o, gate, up, down
    gate = random_weight(8960, 1536, seed=104, dev=cuda)
    up = random_weight(8960, 1536, seed=105, dev=cuda)
    down = random_weight(1536, 8960, seed=106, dev=cuda)
    w16 = [oracle_w16(*w) for w in (gate, up, down)]
    return (gate, up, down), w16


def _one_hot(m, n, cols, dev):
    x = torch.zeros(m, n, dtype=torch.float16)
    x[torch.arange(m), cols] = 1.0
    return x.to(dev)


def test_gate_up_stacked_m2048_one_hot(mlp_15b, cuda):
    """Forward Y = X W_gu^T with X one-hot picks weight columns; input gradient dX = dY W_gu
    with dY one-hot picks weight rows of both segments: each output is a single product."""
    from solution import kernels

    (gate, up, _), (wg, wu, _) = mlp_15b
    banner("gate|up stacked M=2048 one-hot")
    wgu = torch.cat([wg, wu]).view(torch.int16)
    cols = (torch.arange(2048) * 3) % 1536
    y = kernels.linear_fwd(_one_hot(2048, 1536, cols, cuda), [gate, up])
    assert torch.equal(y.cpu().view(torch.int16), wgu[:, cols].t())
    rows = (torch.arange(2048) * 35 + 3) % 17920  # both segments, every tile position
    dx = kernels.linear_dx(_one_hot(2048, 17920, rows, cuda), [gate, up])
    assert torch.equal(dx.cpu().view(torch.int16), wgu[rows])


def test_down_m2048_one_hot(mlp_15b, cuda):
    from solution import kernels

    (_, _, down), (_, _, wd) = mlp_15b
    banner("down M=2048 one-hot (split-K forward)")
    cols = (torch.arange(2048) * 37 + 5) % 8960
    y = kernels.linear_fwd(_one_hot(2048, 8960, cols, cuda), [down])
    assert torch.equal(y.cpu().view(torch.int16), wd.view(torch.int16)[:, cols].t())


def test_gate_up_stacked_m2048_values(mlp_15b, cuda):
    from solution import kernels

    (gate, up, _), (wg, wu, _) = mlp_15b
    banner("gate|up stacked M=2048 values")
    wgu = torch.cat([wg, wu])
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2048, 1536, generator=g).half().to(cuda)
    assert_rel(kernels.linear_fwd(x, [gate, up]), o.linear_fwd(x, wgu), what="fwd gate|up")
    dy = (torch.randn(2048, 17920, generator=g) * 1e-3).half().to(cuda)
    assert_rel(kernels.linear_dx(dy, [gate, up]), o.linear_dx(dy, wgu), what="dx gate|up")
