"""The on-disk NF4 layout (bitsandbytes' serialized QuantState, `solution/checkpoint.py`): round
trips keep every tensor and the dequantized weight bit for bit, the packed JSON entry and the
state-dict keys have bitsandbytes' names and contents, and malformed entries are refused.  CPU
only.  There is no file written by bitsandbytes in the reference or here to load, so the layout
itself is parity unpinned against bitsandbytes."""

import json

import numpy as np
import pytest
import torch

from oracle import nf4_oracle as o
from tests.gpu_util import to_oracle_state


def _weight(n, k, seed, nested=True, blocksize=64):
    from solution.quant_state import quantize_4bit

    g = torch.Generator().manual_seed(seed)
    packed, qs = quantize_4bit(torch.randn(n, k, generator=g) * 0.02, blocksize=blocksize,
                               compress_statistics=nested)
    return packed.view(-1), qs


def _same(qa, qb):
    assert qa.quant_type == qb.quant_type == "nf4"
    assert tuple(qa.shape) == tuple(qb.shape) and qa.blocksize == qb.blocksize
    assert qa.dtype == qb.dtype and qa.nested == qb.nested
    assert torch.equal(qa.absmax, qb.absmax) and torch.equal(qa.code, qb.code)
    if qa.nested:
        assert float(qa.offset) == float(qb.offset)
        assert torch.equal(qa.state2.absmax, qb.state2.absmax)
        assert torch.equal(qa.state2.code, qb.state2.code)
        assert qa.state2.blocksize == qb.state2.blocksize


def _dequant(packed, qs):
    return o.dequantize(*to_oracle_state(packed, qs), "f16")


@pytest.mark.parametrize("nested,blocksize", [(True, 64), (False, 64), (True, 128)])
@pytest.mark.parametrize("packed_items", [True, False])
def test_as_dict_round_trip(nested, blocksize, packed_items):
    from solution.checkpoint import as_dict, from_dict

    packed, qs = _weight(96, 320, seed=5, nested=nested, blocksize=blocksize)
    back = from_dict(as_dict(qs, packed=packed_items))
    _same(qs, back)
    assert np.array_equal(_dequant(packed, qs).view(np.uint16), _dequant(packed, back).view(np.uint16))


def test_packed_json_entry():
    """One uint8 tensor named quant_state.bitsandbytes__nf4 holding the plain items as UTF-8
    JSON; the tensors under bitsandbytes' item names."""
    from solution.checkpoint import as_dict

    _, qs = _weight(64, 256, seed=6)
    d = as_dict(qs, packed=True)
    assert set(d) == {"absmax", "quant_map", "nested_absmax", "nested_quant_map",
                      "quant_state.bitsandbytes__nf4"}
    blob = d["quant_state.bitsandbytes__nf4"]
    assert blob.dtype == torch.uint8 and blob.dim() == 1
    plain = json.loads(bytes(blob.tolist()).decode("utf-8"))
    assert plain == {"quant_type": "nf4", "blocksize": 64, "dtype": "float32", "shape": [64, 256],
                     "nested_blocksize": 256, "nested_dtype": "float32",
                     "nested_offset": float(qs.offset)}
    assert d["absmax"].dtype == torch.uint8 and d["nested_absmax"].dtype == torch.float32
    assert d["quant_map"].numel() == 16 and d["nested_quant_map"].numel() == 256


def test_state_dict_keys_and_safetensors_file(tmp_path):
    """Linear4bit's key layout under a module prefix, and a safetensors file with several
    weights that loads back into the same kernel inputs."""
    from solution.checkpoint import load_safetensors, save_safetensors, state_dict_items

    w = {"model.layers.0.mlp.gate_proj.": _weight(128, 256, seed=7),
         "model.layers.0.self_attn.q_proj.": _weight(64, 256, seed=8, nested=False)}
    keys = set(state_dict_items("model.layers.0.mlp.gate_proj.", *w["model.layers.0.mlp.gate_proj."]))
    base = "model.layers.0.mlp.gate_proj.weight"
    assert keys == {base, base + ".absmax", base + ".quant_map", base + ".nested_absmax",
                    base + ".nested_quant_map", base + ".quant_state.bitsandbytes__nf4"}
    path = tmp_path / "nf4.safetensors"
    save_safetensors(path, w)
    back = load_safetensors(path)
    assert set(back) == set(w)
    for prefix, (packed, qs) in w.items():
        p2, q2 = back[prefix]
        assert torch.equal(p2, packed)
        _same(qs, q2)


def test_malformed_entries_are_refused():
    from solution.checkpoint import as_dict, from_dict, load_weight, state_dict_items

    packed, qs = _weight(32, 128, seed=9)
    d = as_dict(qs, packed=True)
    bad = dict(d)
    bad["quant_state.bitsandbytes__fp4"] = bad.pop("quant_state.bitsandbytes__nf4")
    with pytest.raises(ValueError):
        from_dict(bad)
    with pytest.raises(ValueError):
        from_dict({"absmax": qs.absmax})  # neither the packed entry nor quant_type
    with pytest.raises(ValueError):
        from_dict(dict(d, surprise=torch.zeros(1)))
    items = state_dict_items("m.", packed, qs)
    items["m.weight"] = packed[:-1]
    with pytest.raises(ValueError):
        load_weight(items, "m.")
