"""Checkpoint layers loaded from a .safetensors file run on the GPU: each
format's QuantLinear against the oracle chain (int8: rowwise quant -- with
ConvRot the fused rotation pass -- INT8 GEMM and fused epilogue, bit-exact;
fp8: W8A16 within the bf16 tolerance, W8A8 through the scaled_mm route)."""
import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from _util import assert_bits_equal, assert_close, bf16_to_f32, bits16, gen, u8
from oracle import convrot as ocr
from oracle import fp8 as of
from oracle import int8 as oi

from cdna4q import formats

pytestmark = pytest.mark.gpu


def _blob(conf):
    return torch.frombuffer(bytearray(json.dumps(conf).encode()), dtype=torch.uint8)


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    g = gen(61)
    N, K = 384, 1024
    i8 = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    wf = 0.02 * torch.randn(N, K, generator=g)
    ws = wf.abs().amax() / 448
    f8 = (wf / ws).clamp(-448, 448).to(torch.float8_e4m3fn)
    sd = {
        "row.weight": i8, "row.weight_scale": torch.rand(N, 1, generator=g) * 0.002,
        "row.comfy_quant": _blob({"format": "int8_tensorwise", "per_row": True}),
        "row.bias": (0.1 * torch.randn(N, generator=g)).to(torch.bfloat16),
        "rot.weight": i8.flip(0).contiguous(), "rot.weight_scale": torch.rand(N, 1, generator=g) * 0.002,
        "rot.comfy_quant": _blob({"convrot": True, "convrot_groupsize": 256, "per_row": True}),
        "ten.weight": i8.flip(1).contiguous(), "ten.weight_scale": torch.tensor(0.001),
        "ten.comfy_quant": _blob({"format": "int8_tensorwise"}),
        "fp8.weight": f8, "fp8.scale_weight": ws.reshape(()),
        "fp8.bias": (0.01 * torch.randn(N, generator=g)).to(torch.bfloat16),
    }
    path = tmp_path_factory.mktemp("ckpt") / "layers.safetensors"
    save_file(sd, str(path))
    return path, sd


def test_int8_layers_exact(dev, ckpt):
    path, sd = ckpt
    layers = formats.load_safetensors(path, device=dev)
    g = gen(62)
    x = (torch.randn(2, 75, 1024, generator=g) * 2).to(torch.bfloat16)
    xb = bits16(x.reshape(-1, 1024))
    out = layers["row."](x.to(dev))
    assert out.shape == (2, 75, 384) and out.dtype == torch.bfloat16
    ref = oi.int8_linear(xb, sd["row.weight"].numpy(), sd["row.weight_scale"].numpy(),
                         bits16(sd["row.bias"]))
    assert_bits_equal(bits16(out.reshape(-1, 384)), ref, "int8 per-row layer")
    out = layers["ten."](x.to(dev))
    ref = oi.int8_linear(xb, sd["ten.weight"].numpy(), sd["ten.weight_scale"].reshape(1).numpy())
    assert_bits_equal(bits16(out.reshape(-1, 384)), ref, "int8 per-tensor layer")
    # ConvRot: rotation of every 256-group, rowwise quant, per-channel epilogue
    out = layers["rot."](x.to(dev))
    rq, rs = ocr.merge_rot_quant(xb.reshape(150, 4, 1, 256))
    ref = oi.epilogue_rowcolscale(oi.i8_matmul2d_nt(rq, sd["rot.weight"].numpy()), rs.reshape(-1),
                                  sd["rot.weight_scale"].reshape(-1).numpy())
    assert_bits_equal(bits16(out.reshape(-1, 384)), ref, "int8 convrot layer")


def test_fp8_layer_w8a16_and_w8a8(dev, ckpt):
    path, sd = ckpt
    g = gen(63)
    x = torch.randn(150, 1024, generator=g).to(torch.bfloat16)
    lay = formats.load_safetensors(path, device=dev, prefixes=["fp8."])["fp8."]
    out = lay(x.to(dev))
    ref = of.w8a16_linear(bits16(x), u8(sd["fp8.weight"]), sd["fp8.scale_weight"].reshape(1).numpy(),
                          bits16(sd["fp8.bias"]))
    assert_close(bf16_to_f32(bits16(out)), bf16_to_f32(ref), "fp8 layer w8a16")
    lay8 = formats.load_safetensors(path, device=dev, prefixes=["fp8."], fp8_mode="w8a8")["fp8."]
    out8 = lay8(x.to(dev))
    xq, xs = of.quant_pertensor(bits16(x))
    ref8 = of.scaled_mm(xq, u8(sd["fp8.weight"]), xs, sd["fp8.scale_weight"].reshape(1).numpy(),
                        bits16(sd["fp8.bias"]), "bf16", None, "bf16")
    assert_close(bf16_to_f32(bits16(out8)), bf16_to_f32(ref8), "fp8 layer w8a8")
