"""The projection-stack driver (varlen token batches through n layers of NF4 projections) vs
the fp32 oracle, layer by layer, on the bit-exact dequantized weights."""

import pytest
import torch

from oracle import nf4_oracle as o
from tests.gpu_util import assert_rel, banner, oracle_w16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_stack_layers_match_oracle(cuda, dtype):
    from solution.stack import ProjectionStack, Qwen2Shape

    shape = Qwen2Shape(hidden=256, inter=640, kv=64)
    cu = torch.tensor([0, 37, 100, 163, 300], dtype=torch.int32)  # 4 sequences, M = 300
    banner("stack", dtype, shape, cu.tolist())
    st = ProjectionStack.synthetic(shape, 2, 512, dtype, cuda, seed_base=7, rank=16, alpha=32)
    m = st.set_tokens(cu)
    assert m == 300
    dt = "bf16" if dtype == torch.bfloat16 else "f16"
    s = st.scale
    for li in range(2):
        L, w = st.per_layer[li], st.layers[li]
        W = {n: oracle_w16(*w[n], dt) for n in w}
        wqkv = torch.cat([W["q"], W["k"], W["v"]])
        x, attn, x2, act = (t[:m] for t in (st.x, st.attn, st.x2, st.act))
        lor = [(0, 256, x, L["a_q"], L["b_q"], s), (320, 64, x, L["a_v"], L["b_v"], s)]
        st.forward(layers=[li])
        torch.cuda.synchronize()
        assert_rel(st.y_qkv[:m], o.linear_fwd(x, wqkv, L["bias"], lor), what=f"L{li} qkv")
        assert_rel(st.y_o[:m], o.linear_fwd(attn, W["o"]), what=f"L{li} o")
        assert_rel(st.y_gu[:m], o.linear_fwd(x2, torch.cat([W["gate"], W["up"]])), what="gu")
        assert_rel(st.y_d[:m], o.linear_fwd(act, W["down"]), what=f"L{li} down")

        dy_qkv, dy_o, dy_gu, dy_d = (t[:m] for t in (st.dy_qkv, st.dy_o, st.dy_gu, st.dy_d))
        st.backward(layers=[li])
        torch.cuda.synchronize()
        assert_rel(st.dx_d[:m], o.linear_dx(dy_d, W["down"]), what=f"L{li} dx down")
        assert_rel(st.dx_gu[:m], o.linear_dx(dy_gu, torch.cat([W["gate"], W["up"]])), what="dgu")
        assert_rel(st.dx_o[:m], o.linear_dx(dy_o, W["o"]), what=f"L{li} dx o")
        assert_rel(st.dx_qkv[:m], o.linear_dx(dy_qkv, wqkv, lor), what=f"L{li} dx qkv")
        ga_q, gb_q = o.lora_grads(dy_qkv[:, :256], x, L["a_q"], L["b_q"], s)
        ga_v, gb_v = o.lora_grads(dy_qkv[:, 320:], x, L["a_v"], L["b_v"], s)
        # dA / dB are fp32, but their inputs t = X A^T and da = s dY B are stored in the GEMM
        # dtype between kernels (as the reference stores them): in bf16 that rounding alone
        # gives mean rel ~1.5e-3, so bf16 uses the bf16 mean bound
        mean = 3e-3 if dtype == torch.bfloat16 else 1e-3
        assert_rel(L["gb_q"], gb_q, mean_rel=mean, what=f"L{li} dB_q")
        assert_rel(L["ga_q"], ga_q, mean_rel=mean, what=f"L{li} dA_q")
        assert_rel(L["gb_v"], gb_v, mean_rel=mean, what=f"L{li} dB_v")
        assert_rel(L["ga_v"], ga_v, mean_rel=mean, what=f"L{li} dA_v")


def test_stack_token_count_changes(cuda):
    """set_tokens with a smaller and then a larger batch: outputs follow the current M."""
    from solution.stack import ProjectionStack, Qwen2Shape

    shape = Qwen2Shape(hidden=128, inter=256, kv=64)
    banner("stack varlen resize")
    st = ProjectionStack.synthetic(shape, 1, 256, torch.float16, cuda, seed_base=11)
    W = {n: oracle_w16(*st.layers[0][n]) for n in st.layers[0]}
    for cu in ([0, 5], [0, 64, 65, 200], [0, 1]):
        m = st.set_tokens(cu)
        st.forward()
        torch.cuda.synchronize()
        assert_rel(st.y_o[:m], o.linear_fwd(st.attn[:m], W["o"]), what=f"o M={m}")
        assert_rel(st.y_d[:m], o.linear_fwd(st.act[:m], W["down"]), what=f"down M={m}")
    with pytest.raises(ValueError):
        st.set_tokens([0, 300])


def test_stack_full_step_lora_grads(cuda):
    """A whole step (every layer's forward, then every layer's backward): each layer's dA / dB
    against the oracle from that layer's own t (kept per layer), and the q|k|v input gradient
    of the last layer run (layer 0)."""
    from solution.stack import ProjectionStack, Qwen2Shape

    shape = Qwen2Shape(hidden=256, inter=640, kv=64)
    banner("stack full step, 3 layers")
    st = ProjectionStack.synthetic(shape, 3, 512, torch.float16, cuda, seed_base=29, rank=16,
                                   alpha=32)
    m = st.set_tokens([0, 100, 300])
    st.step()
    torch.cuda.synchronize()
    s = st.scale
    x, dy_qkv = st.x[:m], st.dy_qkv[:m]
    for li in range(3):
        L = st.per_layer[li]
        ga_q, gb_q = o.lora_grads(dy_qkv[:, :256], x, L["a_q"], L["b_q"], s)
        ga_v, gb_v = o.lora_grads(dy_qkv[:, 320:], x, L["a_v"], L["b_v"], s)
        assert_rel(L["gb_q"], gb_q, what=f"L{li} dB_q")
        assert_rel(L["ga_q"], ga_q, what=f"L{li} dA_q")
        assert_rel(L["gb_v"], gb_v, what=f"L{li} dB_v")
        assert_rel(L["ga_v"], ga_v, what=f"L{li} dA_v")
    W = {n: oracle_w16(*st.layers[0][n]) for n in st.layers[0]}
    wqkv = torch.cat([W["q"], W["k"], W["v"]])
    L0 = st.per_layer[0]
    lor = [(0, 256, x, L0["a_q"], L0["b_q"], s), (320, 64, x, L0["a_v"], L0["b_v"], s)]
    assert_rel(st.dx_qkv[:m], o.linear_dx(dy_qkv, wqkv, lor), what="L0 dx qkv")
