"""Standalone NF4 dequant kernel vs the CPU oracle: bit-exact (reference test:
solution/test_kernels.py:51-59, same shapes)."""

import numpy as np
import pytest
import torch

from oracle import nf4_oracle as o
from tests.golden.make_fixtures import OUT as FIXTURES, load_state
from tests.gpu_util import banner, oracle_w16, random_weight, to_device_state

pytestmark = pytest.mark.gpu

DT = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def _bits(t):
    return t.cpu().view(torch.int16 if t.element_size() == 2 else torch.int32)


def _oracle(packed, qs, dt):
    from tests.gpu_util import to_oracle_state

    p, st = to_oracle_state(packed, qs)
    w = o.dequantize(p, st, dt)
    if dt == "bf16":
        return torch.from_numpy(w.view(np.int16))
    if dt == "f16":
        return torch.from_numpy(w).view(torch.int16)
    return torch.from_numpy(w).view(torch.int32)


def test_fixtures_bit_exact(cuda):
    from solution.nf4 import dequantize_nf4

    z = np.load(FIXTURES)
    for name in sorted({k.split("/")[0] for k in z.files}):
        banner("dequant fixture", name)
        packed, st = load_state(z, name)
        p, qs = to_device_state(packed, st, cuda)
        out = dequantize_nf4(p, qs, torch.float16)
        assert torch.equal(_bits(out), torch.from_numpy(z[f"{name}/w_f16"]).view(torch.int16))
        out = dequantize_nf4(p, qs, torch.bfloat16)
        assert torch.equal(_bits(out), torch.from_numpy(z[f"{name}/w_bf16"].view(np.int16)))


@pytest.mark.parametrize("shape", [(1536, 1536), (256, 1536), (8960, 1536), (1536, 8960)])
def test_reference_shapes_bit_exact(cuda, shape):
    from solution.nf4 import dequantize_nf4

    banner("dequant shape", shape)
    packed, qs = random_weight(*shape, seed=sum(shape), dev=cuda, std=0.05)
    out = dequantize_nf4(packed, qs, torch.float16)
    torch.cuda.synchronize()
    assert out.shape == shape
    assert torch.equal(_bits(out), _oracle(packed, qs, "f16"))


def _double_rounding_pairs(count, seed=0):
    """(code index, fp32 absmax) pairs whose fp32 product code * absmax is an exact fp16 tie
    while the exact product is not: rounding the fp32 product (the element formula's two
    roundings) and rounding the exact product once give neighbouring fp16 values."""
    code = o.NF4_CODE.astype(np.float32)
    rng = np.random.default_rng(seed)
    a = rng.uniform(1e-3, 1e-1, 2_000_000).astype(np.float32)
    i = rng.integers(0, 16, a.size)
    double = (code[i] * a).astype(np.float32).astype(np.float16)
    single = (code[i].astype(np.float64) * a.astype(np.float64)).astype(np.float16)
    hit = np.nonzero(double != single)[0]  # ~3.5e-5 of the draws
    assert hit.size >= 16
    hit = np.resize(hit, count)
    return i[hit], a[hit]


@pytest.mark.parametrize("shape,bs", [((4, 30), 2), ((3, 66), 64)])
def test_scalar_paths_round_the_fp32_product(cuda, shape, bs):
    """The scalar dequant paths (element kernel for blocksize 2; the ragged tail of the 8-element
    kernel) on products where one rounding of the exact product would differ from rounding the
    fp32 product: the output must be the latter, bit for bit."""
    banner("dequant scalar double rounding", shape, bs)
    n = shape[0] * shape[1]
    nb = -(-n // bs)
    idx, am = _double_rounding_pairs(nb)
    nib = np.repeat(idx, bs)[:n].astype(np.uint8)
    if n % 2:
        nib = np.append(nib, 0)
    packed = ((nib[0::2] << 4) | nib[1::2]).astype(np.uint8)
    st = o.OracleQuantState(absmax=am.astype(np.float32), shape=shape, code=o.NF4_CODE.copy(),
                            blocksize=bs)
    p, qs = to_device_state(packed, st, cuda)
    from solution import kernels

    out = kernels.dequant([(p, qs)], torch.float16)
    ref = o.dequantize(packed, st, "f16")
    assert np.array_equal(out.cpu().numpy().view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("nested", [True, False])
@pytest.mark.parametrize("shape,bs", [((7, 9), 64), ((33, 64), 32), ((100, 384), 128),
                                      ((3, 1000), 256), ((5, 6), 2), ((64, 192), 64),
                                      ((12, 40), 8), ((9, 30), 16)])
def test_layouts_bit_exact(cuda, dt, nested, shape, bs):
    from solution.nf4 import dequantize_nf4

    banner("dequant layout", dt, nested, shape, bs)
    packed, qs = random_weight(*shape, seed=7, dev=cuda, blocksize=bs, nested=nested)
    out = dequantize_nf4(packed, qs, DT[dt])
    assert torch.equal(_bits(out), _oracle(packed, qs, dt))


def test_stacked_segments_bit_exact(cuda):
    from solution.layer import _dequant

    banner("dequant stacked q|k|v and gate|up")
    qkv = [random_weight(n, 1536, seed=100 + i, dev=cuda) for i, n in enumerate((1536, 256, 256))]
    out = _dequant(qkv, torch.float16)
    ref = torch.cat([_oracle(p, q, "f16").view(int(q.shape[0]), -1) for p, q in qkv])
    assert torch.equal(_bits(out), ref)
    odd = [random_weight(n, 68, seed=200 + i, dev=cuda) for i, n in enumerate((3, 5, 1))]
    out = _dequant(odd, torch.bfloat16)  # unaligned segment starts: general path
    ref = torch.cat([_oracle(p, q, "bf16").view(int(q.shape[0]), -1) for p, q in odd])
    assert torch.equal(_bits(out), ref)


def test_unaligned_output_and_empty(cuda):
    from solution import kernels

    banner("dequant unaligned output / empty")
    p, qs = random_weight(16, 64, seed=9, dev=cuda)
    buf = torch.zeros(16 * 64 + 1, dtype=torch.float16, device=cuda)
    kernels.dequant([(p, qs)], torch.float16, out=buf[1:].view(16, 64))
    assert torch.equal(_bits(buf[1:]), _oracle(p, qs, "f16").reshape(-1))
    assert buf[0].item() == 0
    p0, q0 = random_weight(0, 64, seed=9, dev=cuda)
    assert kernels.dequant([(p0, q0)], torch.float16).shape == (0, 64)


def test_round_to_nearest_even_ties(cuda):
    """Products that fall exactly halfway between two fp16 / bf16 values (absmax 1, table-driven
    codes): the conversion must round to even, like the oracle's."""
    from solution.quant_state import QuantState
    from solution.nf4 import dequantize_nf4

    banner("dequant RNE ties")
    ties = [1 + 2 ** -11, 1 + 3 * 2 ** -11, 1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -11),
            2 ** -25, 3 * 2 ** -25, 65520.0, -(1 + 3 * 2 ** -8), 0.1, -0.3, 1.0, 0.0, 2.0,
            1 + 2 ** -9, 3.0]
    code = torch.tensor(ties, dtype=torch.float32)
    n = 128
    q = (torch.arange(n) % 16).to(torch.uint8)
    packed = ((q[0::2] << 4) | q[1::2]).contiguous()
    qs = QuantState(absmax=torch.ones(2, dtype=torch.float32).to(cuda), shape=torch.Size((2, 64)),
                    code=code.to(cuda), blocksize=64, quant_type="nf4", dtype=torch.float16)
    p = packed.to(cuda)
    for dt in ("f16", "bf16"):
        out = dequantize_nf4(p, qs, DT[dt])
        st = o.OracleQuantState(absmax=np.ones(2, np.float32), shape=(2, 64), code=code.numpy())
        ref = o.dequantize(packed.numpy(), st, dt)
        ref = torch.from_numpy(ref.view(np.int16) if dt == "bf16" else ref.view(np.int16))
        assert torch.equal(_bits(out), ref), dt


@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
def test_batch_bit_exact(cuda, dt):
    """One launch, seven weights of a layer (different shapes) into separate outputs; then a
    batch with an unaligned output (general path)."""
    from solution import kernels

    banner("dequant batch", dt)
    shapes = [(192, 128), (64, 128), (64, 128), (128, 128), (320, 128), (320, 128), (128, 320)]
    ws = [random_weight(n, k, seed=400 + i, dev=cuda) for i, (n, k) in enumerate(shapes)]
    outs = kernels.dequant_batch(ws, DT[dt])
    for (p, qs), out in zip(ws, outs):
        assert torch.equal(_bits(out).reshape(-1), _oracle(p, qs, dt).reshape(-1))
    odd = [random_weight(n, k, seed=500 + n, dev=cuda, blocksize=bs)
           for n, k, bs in ((5, 12, 4), (33, 64, 64), (3, 100, 128))]
    buf = torch.zeros(5 * 12 + 1 + 33 * 64 + 3 * 100, dtype=DT[dt], device=cuda)
    views = [buf[1:61].view(5, 12), buf[61:61 + 2112].view(33, 64), buf[2173:2473].view(3, 100)]
    kernels.dequant_batch(odd, DT[dt], outs=views)
    for (p, qs), out in zip(odd, views):
        assert torch.equal(_bits(out).reshape(-1), _oracle(p, qs, dt).reshape(-1))
    assert _bits(buf[:1]).item() == 0


@pytest.mark.parametrize("nested", [True, False])
def test_checkpoint_loads_into_kernels(cuda, tmp_path, nested):
    """A weight saved in bitsandbytes' serialized layout and loaded straight onto the GPU feeds
    the kernels unchanged: dequant bit-exact against the oracle on the loaded state, and the
    same bytes as the weight before saving."""
    from solution.checkpoint import load_safetensors, save_safetensors
    from solution.nf4 import dequantize_nf4

    banner("checkpoint -> kernels", nested)
    packed, qs = random_weight(200, 512, seed=77, dev=cuda, nested=nested)
    save_safetensors(tmp_path / "w.safetensors", {"layer.q_proj.": (packed, qs)})
    p2, q2 = load_safetensors(tmp_path / "w.safetensors", cuda)["layer.q_proj."]
    w = dequantize_nf4(p2, q2, torch.float16)
    assert torch.equal(w.cpu().view(torch.int16), oracle_w16(p2, q2).view(torch.int16))
    assert torch.equal(w, dequantize_nf4(packed, qs, torch.float16))


@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
def test_table_bit_exact(cuda, dt):
    """One table launch over 21 weights (three layers' worth of shapes, nested and plain,
    blocksizes 8 to 256, an element count that is not a multiple of 8): every output bit-exact,
    also on a second launch into cleared outputs; a launch whose dtype or workgroup count does
    not match the table writes nothing (a wrong weight count is refused before the launch)."""
    from solution import kernels

    banner("dequant table", dt)
    shapes = [(192, 128, 64, True), (64, 128, 64, True), (64, 128, 64, False),
              (128, 128, 128, True), (320, 128, 256, True), (320, 128, 8, True),
              (128, 320, 64, True)]
    ws = [random_weight(n, k, seed=600 + 10 * layer + i, dev=cuda, blocksize=bs, nested=nest)
          for layer in range(3) for i, (n, k, bs, nest) in enumerate(shapes)]
    ws.append(random_weight(3, 100, seed=699, dev=cuda))  # 300 elements: a partial unit
    table = kernels.DequantTable(ws, DT[dt])
    for rep in range(2):
        for out in table.outs:
            out.zero_()
        table.run()
        for (p, qs), out in zip(ws, table.outs):
            assert torch.equal(_bits(out).reshape(-1), _oracle(p, qs, dt).reshape(-1)), rep
    for out in table.outs:
        out.zero_()
    lib, s = kernels.load(), kernels.stream_of(table.table)
    other = 1 if dt == "f16" else 0
    nw = len(ws)
    assert lib.nf4_dequant_table(table.table.data_ptr(), nw, table.blocks, other, s) == 0
    assert lib.nf4_dequant_table(table.table.data_ptr(), nw, table.blocks - 1, table._code, s) == 0
    torch.cuda.synchronize()
    assert all(not out.any() for out in table.outs)
    assert lib.nf4_dequant_table(table.table.data_ptr(), 0, table.blocks, table._code, s) != 0


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_table_qwen15b_layer_bit_exact(cuda, dt):
    """The timed dequant at its workload: one nf4_dequant_table launch over a whole
    Qwen2.5-1.5B decoder layer (q, k, v, o, gate, up, down at their real shapes, 46.8 M
    elements, each weight quantized on its own: distinct packed bytes, absmax codes and absmax2
    scales, as in the bench's 28-layer stack), every output bit-exact against the oracle."""
    from solution import kernels

    banner("dequant table, Qwen2.5-1.5B layer", dt)
    layer = [(1536, 1536), (256, 1536), (256, 1536), (1536, 1536), (8960, 1536), (8960, 1536),
             (1536, 8960)]
    ws = [random_weight(n, k, seed=1000 + i, dev=cuda) for i, (n, k) in enumerate(layer)]
    table = kernels.DequantTable(ws, DT[dt])
    table.run()
    for (p, qs), out in zip(ws, table.outs):
        assert torch.equal(_bits(out).reshape(-1), _oracle(p, qs, dt).reshape(-1)), tuple(qs.shape)
