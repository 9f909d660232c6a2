"""The drop-in at model level: a whole tiny Qwen2 QLoRA model (transformers' own
Qwen2ForCausalLM) trained one step through `solution.apply()`, against an fp32 composition of
the same model on the oracle's dequantized weights.

Mirrors the reference's test_fused_layer_matches_stock_modules (solution/test_kernels.py:224-320):
vocab 512, hidden 256, intermediate 512, 3 layers, 4 / 2 heads, tied embeddings, every
projection an NF4 bitsandbytes Linear4bit (double quant, blocksize 64), LoRA on q_proj and v_proj
(r 8, alpha 16), batch 3 x 40 tokens with padding and ignored labels, fp16 autocast; the loss
within 2e-3 relative and every LoRA gradient within 3e-2 of its largest magnitude.  bitsandbytes
and peft are absent here and on the GPU box: the Linear4bit layers are the stand-in of
tests/bnb_standin.py (its own forward never runs on the patched path, which the test asserts)
and the LoRA wrapper is written out below with peft's arithmetic (LoraLayer.forward:
base(x) + lora_B(lora_A(dropout(x))) * alpha / r, dropout 0 here so both runs see the same
inputs).  The reference run differs from the reference's own in one respect: its yardstick is
an fp32 composition on the dequantized weights instead of the stock bitsandbytes run, which
cannot run here."""

import copy

import pytest
import torch

from oracle import nf4_oracle as o
from tests import bnb_standin
from tests.gpu_util import banner, to_oracle_state

pytestmark = pytest.mark.gpu

PROJ = (("self_attn", ("q_proj", "k_proj", "v_proj", "o_proj")),
        ("mlp", ("gate_proj", "up_proj", "down_proj")))


class LoraLinear(torch.nn.Module):
    """peft's LoRA wrapper of one linear layer: base(x) + lora_B(lora_A(x)) * alpha / r."""

    def __init__(self, base, in_features, out_features, r, alpha, a=None, b=None):
        super().__init__()
        self.base_layer = base
        self.lora_A = torch.nn.Linear(in_features, r, bias=False)
        self.lora_B = torch.nn.Linear(r, out_features, bias=False)
        if a is not None:
            self.lora_A.weight.data.copy_(a)
            self.lora_B.weight.data.copy_(b)
        self.scaling = alpha / r

    def forward(self, x):
        result = self.base_layer(x)
        x = x.to(self.lora_A.weight.dtype)
        return result + self.lora_B(self.lora_A(x)) * self.scaling


def _models(mod, dev):
    """(HIP model on dev, fp32 reference model on the CPU, LoRA parameter names)."""
    from transformers import Qwen2Config, Qwen2ForCausalLM

    from solution.quant_state import quantize_4bit

    torch.manual_seed(0)
    cfg = Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512,
                      num_hidden_layers=3, num_attention_heads=4, num_key_value_heads=2,
                      tie_word_embeddings=True, attn_implementation="sdpa")
    base = Qwen2ForCausalLM(cfg)  # fp32 weights: the values both models start from
    ref = copy.deepcopy(base)
    fused = base
    g = torch.Generator().manual_seed(1)
    r, alpha = 8, 16
    for layer_f, layer_r in zip(fused.model.layers, ref.model.layers):
        for part, names in PROJ:
            for name in names:
                lin_f, lin_r = getattr(getattr(layer_f, part), name), getattr(getattr(layer_r, part), name)
                packed, qs = quantize_4bit(lin_f.weight.data.to(dev), blocksize=64,
                                           compress_statistics=True)
                packed = packed.view(-1)
                bias = None
                if lin_f.bias is not None:
                    bias = torch.nn.Parameter(lin_f.bias.data.to(dev), requires_grad=False)
                q4 = mod.nn.Linear4bit(packed, qs, bias=bias, compute_dtype=torch.float32)
                # the reference: the bit-exact dequantized weight, in fp32
                p, st = to_oracle_state(packed, qs)
                w16 = torch.from_numpy(o.dequantize(p, st, "f16")).float()
                lin_r.weight.data.copy_(w16)
                new_f, new_r = q4, lin_r
                if name in ("q_proj", "v_proj"):
                    a = (torch.rand(r, lin_f.in_features, generator=g) * 2 - 1) / lin_f.in_features ** 0.5
                    b = torch.randn(lin_f.out_features, r, generator=g) * 0.02
                    new_f = LoraLinear(q4, lin_f.in_features, lin_f.out_features, r, alpha, a, b)
                    new_r = LoraLinear(lin_r, lin_r.in_features, lin_r.out_features, r, alpha, a, b)
                setattr(getattr(layer_f, part), name, new_f)
                setattr(getattr(layer_r, part), name, new_r)
    fused.to(dev)
    for m in (fused, ref):
        for n, prm in m.named_parameters():
            prm.requires_grad_("lora_" in n)
        m.train()
    names = [n for n, _ in ref.named_parameters() if "lora_" in n]
    return fused, ref, names


def test_tiny_qwen2_qlora_step_through_apply(monkeypatch, cuda):
    import solution
    from transformers.models.qwen2 import modeling_qwen2

    banner("tiny Qwen2 QLoRA step through solution.apply()")
    mod, calls = bnb_standin.install(monkeypatch)
    monkeypatch.setattr(modeling_qwen2.Qwen2MLP, "forward", modeling_qwen2.Qwen2MLP.forward)
    fused, ref, names = _models(mod, cuda)
    done = solution.apply()
    assert all(done.values()), done

    g = torch.Generator().manual_seed(2)
    batch, seq = 3, 40
    ids = torch.randint(0, 512, (batch, seq), generator=g)
    mask = torch.ones(batch, seq, dtype=torch.long)
    mask[0, 25:] = 0
    mask[2, 9:] = 0
    labels = ids.clone()
    labels[:, :5] = -100
    labels[mask == 0] = -100

    with torch.autocast("cuda", dtype=torch.float16):
        loss = fused(input_ids=ids.to(cuda), attention_mask=mask.to(cuda),
                     labels=labels.to(cuda)).loss
    loss.backward()
    torch.cuda.synchronize()
    assert calls.forward == 0 and calls.matmul == 0, "a projection ran bitsandbytes' own path"

    loss_r = ref(input_ids=ids, attention_mask=mask, labels=labels).loss
    loss_r.backward()
    assert abs(loss.item() - loss_r.item()) <= 2e-3 * abs(loss_r.item()), (loss.item(), loss_r.item())
    got = dict(fused.named_parameters())
    for n, p in ref.named_parameters():
        if n not in names:
            continue
        gr, gf = p.grad, got[n].grad
        assert gf is not None, n
        scale = gr.abs().max().item() + 1e-12
        err = (gf.float().cpu() - gr).abs().max().item()
        assert err <= 3e-2 * scale, f"{n}: max |dg| {err:.3e} vs 3e-2 * {scale:.3e}"
