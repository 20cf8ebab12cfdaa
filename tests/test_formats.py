"""On-disk quantized linear formats, CPU only: the comfy_quant metadata
repair (``formats.fix_quant_meta`` through ``patches.quant_meta_fix``, as one
table of descriptor / weight dtype / scale cases covering the behaviour of
reference _patches/quant_meta_fix.py:34-59),
format detection, and loading layers from a .safetensors file into
QuantLinear modules. The loaded layers' numerics run on the GPU in
tests/test_gpu_formats.py."""
import json
import sys
import types

import pytest
import torch
from safetensors.torch import save_file

from cdna4q import formats
from cdna4q._lib import C4QError
from cdna4q.patches import quant_meta_fix


def _json_u8(desc):
    return torch.tensor(list(json.dumps(desc).encode()), dtype=torch.uint8)


def _state(desc, weight_dtype, scale_shape, prefix="blk.0.mlp."):
    """One layer's checkpoint entries: the comfy_quant descriptor as JSON
    bytes, a 6x8 weight of `weight_dtype` and (unless `scale_shape` is None)
    an f32 weight_scale of that shape."""
    sd = {prefix + "comfy_quant": _json_u8(desc),
          prefix + "weight": torch.zeros(6, 8, dtype=weight_dtype)}
    if scale_shape is not None:
        sd[prefix + "weight_scale"] = torch.full(scale_shape, 0.5)
    return sd


def _desc(sd, prefix="blk.0.mlp."):
    return json.loads(sd[prefix + "comfy_quant"].numpy().tobytes().decode())


_ROT = {"convrot": True, "convrot_groupsize": 256, "per_row": True}

# (descriptor on disk, weight dtype, weight_scale shape or None) -> descriptor
# after the repair: only an int8 weight with a scale and no declared format
# gains "format": "int8_tensorwise"; every other key is kept as written.
META_CASES = [
    (_ROT, torch.int8, (6, 1), dict(_ROT, format="int8_tensorwise")),
    ({"per_row": False}, torch.int8, (1,), {"per_row": False, "format": "int8_tensorwise"}),
    ({}, torch.int8, (6,), {"format": "int8_tensorwise"}),
    (dict(_ROT, format="int8_tensorwise"), torch.int8, (6, 1), dict(_ROT, format="int8_tensorwise")),
    ({"format": "float8_e4m3fn"}, torch.int8, (6, 1), {"format": "float8_e4m3fn"}),
    (_ROT, torch.uint8, (6, 1), _ROT),                     # packed 4-bit payload
    (_ROT, torch.float8_e4m3fn, (6, 1), _ROT),
    (_ROT, torch.int8, None, _ROT),                        # no weight_scale
]


@pytest.mark.parametrize("desc,wdt,scale_shape,want", META_CASES)
def test_quant_meta_repair_table(desc, wdt, scale_shape, want):
    sd = _state(desc, wdt, scale_shape)
    raw = sd["blk.0.mlp.comfy_quant"]
    quant_meta_fix._maybe_fix(sd, "blk.0.mlp.")
    assert _desc(sd) == want
    if want == desc:                                       # untouched: same tensor object
        assert sd["blk.0.mlp.comfy_quant"] is raw
    assert {k for k in sd} >= {"blk.0.mlp.weight"}         # tensors themselves untouched


def test_quant_meta_repair_only_touches_its_prefix():
    sd = _state(_ROT, torch.int8, (6, 1), "a.")
    sd.update(_state(_ROT, torch.int8, (6, 1), "b."))
    quant_meta_fix._maybe_fix(sd, "b.")
    assert "format" not in _desc(sd, "a.") and _desc(sd, "b.")["format"] == "int8_tensorwise"


def test_unparseable_descriptor_left_alone():
    sd = {"layer.comfy_quant": torch.tensor([0xff, 0x00], dtype=torch.uint8),
          "layer.weight": torch.zeros(4, 4, dtype=torch.int8),
          "layer.weight_scale": torch.ones(4, 1)}
    assert not formats.fix_quant_meta(sd, "layer.")


def test_install_wraps_comfy_loader(monkeypatch):
    """With a stand-in comfy.ops, install() wraps _load_quantized_module so
    the loader sees the repaired descriptor; without ComfyUI it installs
    nothing."""
    monkeypatch.setattr(quant_meta_fix, "_installed", False)
    monkeypatch.setitem(sys.modules, "comfy", None)
    assert quant_meta_fix.install() is False
    seen = []
    comfy = types.ModuleType("comfy")
    comfy_ops = types.ModuleType("comfy.ops")
    comfy_ops._load_quantized_module = lambda module, load_fn, sd, prefix: seen.append(_desc(sd, prefix))
    comfy.ops = comfy_ops
    monkeypatch.setitem(sys.modules, "comfy", comfy)
    monkeypatch.setitem(sys.modules, "comfy.ops", comfy_ops)
    assert quant_meta_fix.install() is True
    sd = {"blk.comfy_quant": _json_u8({"convrot": True}), "blk.weight": torch.zeros(2, 2, dtype=torch.int8),
          "blk.weight_scale": torch.ones(2, 1)}
    comfy_ops._load_quantized_module(None, None, sd, "blk.")
    assert seen == [{"convrot": True, "format": "int8_tensorwise"}]
    monkeypatch.setattr(quant_meta_fix, "_installed", False)


# -- format detection and loading -------------------------------------------

def _checkpoint():
    g = torch.Generator().manual_seed(3)
    N, K = 16, 512
    i8 = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    f8 = (0.02 * torch.randn(N, K, generator=g) * 400).clamp(-448, 448).to(torch.float8_e4m3fn)
    return {
        "a.weight": i8, "a.weight_scale": torch.rand(N, 1, generator=g),
        "a.comfy_quant": _json_u8({"format": "int8_tensorwise"}),
        "a.bias": torch.randn(N, generator=g).to(torch.bfloat16),
        "b.weight": i8.clone(), "b.weight_scale": torch.rand(N, 1, generator=g),
        "b.comfy_quant": _json_u8({"convrot": True, "convrot_groupsize": 256, "per_row": True}),
        "c.weight": i8.clone(), "c.weight_scale": torch.tensor(0.01),
        "c.comfy_quant": _json_u8({"format": "int8_tensorwise"}),
        "d.weight": f8, "d.scale_weight": torch.tensor(0.002),              # scaled fp8
        "e.weight": f8.clone(), "e.weight_scale": torch.tensor(0.003),
        "e.comfy_quant": _json_u8({"format": "float8_e4m3fn"}),
        "norm.weight": torch.ones(K, dtype=torch.bfloat16),                 # not a quantized linear
        "f.weight": torch.zeros(N, K, dtype=torch.uint8),
        "f.comfy_quant": _json_u8({"format": "w4_packed"}),
        "scaled_fp8": torch.zeros(0, dtype=torch.float8_e4m3fn),
    }


def test_layer_formats():
    sd = _checkpoint()
    assert formats.quantized_prefixes(sd) == ["a.", "b.", "c.", "d.", "e."]
    assert _desc(sd, "b.")["format"] == "int8_tensorwise"                 # repaired in place
    assert formats.layer_format(sd, "norm.") is None
    assert formats.layer_format(sd, "f.") is None
    with pytest.raises(C4QError):
        formats.load_linear(sd, "norm.", "cpu")


def test_load_safetensors_round_trip(tmp_path):
    sd = _checkpoint()
    path = tmp_path / "ckpt.safetensors"
    save_file(sd, str(path))
    layers = formats.load_safetensors(path, device="cpu")
    assert sorted(layers) == ["a.", "b.", "c.", "d.", "e."]
    a, b, c, d, e = (layers[k] for k in sorted(layers))
    assert a.kind == "int8" and a.weight._params.scale.shape == (16, 1) and not a.weight._params.convrot
    assert torch.equal(a.weight._qdata, sd["a.weight"]) and torch.equal(a.bias, sd["a.bias"])
    assert b.weight._params.convrot and b.weight._params.convrot_groupsize == 256
    assert c.weight._params.scale.shape == (1,)
    assert d.kind == "fp8" and float(d.scale) == pytest.approx(0.002) and d.bias is None
    assert torch.equal(d.weight.view(torch.uint8), sd["d.weight"].view(torch.uint8))
    assert e.kind == "fp8" and float(e.scale) == pytest.approx(0.003)
    assert (a.in_features, a.out_features) == (512, 16)


def test_bad_scale_layouts_raise():
    sd = _checkpoint()
    sd["a.weight_scale"] = torch.ones(3)
    with pytest.raises(C4QError, match="weight_scale"):
        formats.load_linear(sd, "a.", "cpu")
    sd["d.scale_weight"] = torch.ones(16)
    with pytest.raises(C4QError, match="per tensor"):
        formats.load_linear(sd, "d.", "cpu")
