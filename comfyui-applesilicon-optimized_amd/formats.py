"""On-disk quantized linear formats: reading checkpoint layers into weights the
kernels take.

ComfyUI checkpoints store a quantized linear under a module prefix P as

    P.weight        int8 [N, K]  or  float8_e4m3fn [N, K]
    P.weight_scale  fp32: [N, 1] / [N] (per output row) or [] / [1] (per tensor)
    P.scale_weight  fp32 [] (the older "scaled fp8" checkpoints; their file
                    also holds a top-level ``scaled_fp8`` marker tensor)
    P.input_scale   fp32 [] (optional; static activation scale of fp8 W8A8)
    P.bias          bf16 / f16 / f32 [N] (optional)
    P.comfy_quant   uint8 bytes of a JSON descriptor, e.g.
                    {"format": "int8_tensorwise", "convrot": true,
                     "convrot_groupsize": 256, "per_row": true}

as the reference's patches read them (``_patches/quant_meta_fix.py:1-60``,
the ``TensorWiseINT8Layout`` fields ``_qdata`` / ``_params.scale`` /
``convrot`` / ``transposed`` used at
``_patches/int8_linear_kernel_mps.py:797-815``, the scaled-fp8
``scale_weight`` of ``_patches/linear_fp8_w8a16.py``). A descriptor without
``format`` over an int8 weight with a ``weight_scale`` is an
``int8_tensorwise`` layer (``fix_quant_meta``, the reference's
``_maybe_fix``).

``load_linear`` turns one prefix into a ``QuantLinear`` on a device;
``load_safetensors`` does it for every quantized linear of a file. Files are
read with ``safetensors`` (no pickle). ``QuantLinear.forward`` runs the
kernels: int8 layers through the W8A8 path of ``patches.int8_linear``
(rowwise activation quant -- with ConvRot, the fused rotate + quant pass --
and the fused per-channel or per-tensor epilogue), fp8 layers through the
W8A16 kernel (weight-only, the reference's standard-fp8 Linear route) or,
with ``fp8_mode="w8a8"``, dynamic per-tensor activation quant and
``scaled_mm`` (the reference's ``torch._scaled_mm`` route).
"""
import json
import types

import torch

from . import ops
from ._lib import C4QError

INT8_TENSORWISE = "int8_tensorwise"
FLOAT8_E4M3FN = "float8_e4m3fn"


def read_comfy_quant(blob):
    """The JSON descriptor stored as uint8 bytes, or None if unparseable."""
    try:
        conf = json.loads(bytes(blob.cpu().numpy().tobytes()))
    except Exception:
        return None
    return conf if isinstance(conf, dict) else None


def comfy_quant_blob(conf):
    """The uint8 tensor a descriptor is stored as."""
    return torch.frombuffer(bytearray(json.dumps(conf).encode()), dtype=torch.uint8)


def fix_quant_meta(state_dict, prefix):
    """Give a ``format``-less descriptor ``"format": "int8_tensorwise"`` when
    the layer's weight is int8 and it has a ``weight_scale`` (reference
    ``_maybe_fix``, ``quant_meta_fix.py:34-59``); anything else is left as
    it is. Returns True when the descriptor was changed."""
    key = f"{prefix}comfy_quant"
    blob = state_dict.get(key)
    if blob is None:
        return False
    conf = read_comfy_quant(blob)
    if conf is None or "format" in conf:
        return False
    weight = state_dict.get(f"{prefix}weight")
    scale = state_dict.get(f"{prefix}weight_scale")
    if weight is None or scale is None or weight.dtype != torch.int8:
        return False
    conf["format"] = INT8_TENSORWISE
    state_dict[key] = comfy_quant_blob(conf)
    return True


class Int8TensorwiseWeight:
    """The fields of comfy_kitchen's ``QuantizedTensor`` in
    ``TensorWiseINT8Layout`` that the kernel routes read: ``_qdata`` int8
    [N, K], ``_params`` with ``scale`` (fp32, per row [N, 1] or per tensor),
    ``convrot``, ``convrot_groupsize``, ``transposed``."""
    _layout_cls = "TensorWiseINT8Layout"

    def __init__(self, qdata, scale, convrot=False, convrot_groupsize=256, transposed=False):
        self._qdata = qdata
        self._params = types.SimpleNamespace(scale=scale, convrot=bool(convrot),
                                             convrot_groupsize=int(convrot_groupsize),
                                             transposed=bool(transposed))

    @property
    def shape(self):
        return self._qdata.shape


class QuantLinear(torch.nn.Module):
    """A linear layer over a quantized checkpoint weight (``load_linear``).
    ``kind`` is "int8" (weight: Int8TensorwiseWeight) or "fp8" (weight:
    float8_e4m3fn [N, K], ``scale`` its per-tensor fp32 scale or None)."""

    def __init__(self, kind, weight, scale=None, bias=None, fp8_mode="w8a16"):
        super().__init__()
        if kind not in ("int8", "fp8") or fp8_mode not in ("w8a16", "w8a8"):
            raise C4QError(f"QuantLinear: kind {kind!r} / fp8_mode {fp8_mode!r}")
        self.kind, self.weight, self.scale, self.bias, self.fp8_mode = (kind, weight, scale, bias,
                                                                        fp8_mode)
        self.out_features, self.in_features = (weight.shape[0], weight.shape[1])

    def forward(self, x):
        from .patches import int8_linear
        if self.kind == "int8":
            p = self.weight._params
            if p.transposed:
                raise C4QError("QuantLinear: transposed int8 storage is not supported")
            return int8_linear._int8_linear_kernel(x, self.weight._qdata, p.scale, self.bias, x.dtype,
                                                   p.convrot, p.convrot_groupsize)
        if self.fp8_mode == "w8a16":
            bias = self.bias.float() if self.bias is not None else None
            return ops.w8a16_linear(x, self.weight, self.scale, bias, out_dtype=x.dtype)
        lead = x.shape[:-1]
        xq, xs = ops.fp8_quant_pertensor(x.reshape(-1, x.shape[-1]))
        ws = self.scale if self.scale is not None else torch.ones((), device=x.device)
        out = ops.scaled_mm(xq, self.weight.t(), out_dtype=x.dtype, scale_a=xs,
                            scale_b=ws.float().reshape(()), bias=self.bias)
        return out.reshape(*lead, self.out_features)


def layer_format(state_dict, prefix):
    """The quantization format of the linear at ``prefix``: "int8_tensorwise",
    "float8_e4m3fn", or None (not a quantized linear this build reads)."""
    w = state_dict.get(f"{prefix}weight")
    if w is None:
        return None
    blob = state_dict.get(f"{prefix}comfy_quant")
    conf = read_comfy_quant(blob) if blob is not None else {}
    fmt = (conf or {}).get("format")
    if fmt == INT8_TENSORWISE and w.dtype == torch.int8:
        return INT8_TENSORWISE
    if w.dtype == torch.float8_e4m3fn and fmt in (None, FLOAT8_E4M3FN):
        return FLOAT8_E4M3FN
    return None


def load_linear(state_dict, prefix, device="cuda", fp8_mode="w8a16"):
    """The quantized linear at ``prefix`` as a QuantLinear with its tensors on
    ``device``; raises C4QError for a layer this build does not read."""
    fix_quant_meta(state_dict, prefix)
    fmt = layer_format(state_dict, prefix)
    if fmt is None:
        raise C4QError(f"{prefix}: not an int8_tensorwise or float8_e4m3fn linear")
    w = state_dict[f"{prefix}weight"]
    bias = state_dict.get(f"{prefix}bias")
    bias = bias.to(device) if bias is not None else None
    if w.dim() != 2:
        raise C4QError(f"{prefix}: weight must be 2-D, got {tuple(w.shape)}")
    if fmt == INT8_TENSORWISE:
        conf = read_comfy_quant(state_dict[f"{prefix}comfy_quant"])
        s = state_dict.get(f"{prefix}weight_scale")
        if s is None:
            raise C4QError(f"{prefix}: int8_tensorwise layer without weight_scale")
        s = s.to(torch.float32)
        if s.numel() == w.shape[0]:
            s = s.reshape(-1, 1)
        elif s.numel() != 1:
            raise C4QError(f"{prefix}: weight_scale of {s.numel()} elements for {w.shape[0]} rows")
        else:
            s = s.reshape(1)
        qt = Int8TensorwiseWeight(w.to(device).contiguous(), s.to(device),
                                  conf.get("convrot", False), conf.get("convrot_groupsize", 256),
                                  conf.get("transposed", False))
        return QuantLinear("int8", qt, bias=bias)
    s = state_dict.get(f"{prefix}weight_scale", state_dict.get(f"{prefix}scale_weight"))
    if s is not None:
        if s.numel() != 1:
            raise C4QError(f"{prefix}: fp8 weight scale must be per tensor ({s.numel()} elements)")
        s = s.to(torch.float32).reshape(()).to(device)
    return QuantLinear("fp8", w.to(device).contiguous(), s, bias, fp8_mode=fp8_mode)


def quantized_prefixes(state_dict):
    """Prefixes of the quantized linears of a state dict, in key order (after
    ``fix_quant_meta`` of each, which it applies to the state dict)."""
    out = []
    for key in list(state_dict):
        if key.endswith("weight") and not key.endswith("_weight"):
            prefix = key[:-len("weight")]
            fix_quant_meta(state_dict, prefix)
            if layer_format(state_dict, prefix) is not None:
                out.append(prefix)
    return out


def load_safetensors(path, device="cuda", prefixes=None, fp8_mode="w8a16"):
    """{prefix: QuantLinear} for the quantized linears of a .safetensors file
    (all of them, or the given prefixes)."""
    from safetensors.torch import load_file
    sd = load_file(str(path), device="cpu")
    if prefixes is None:
        prefixes = quantized_prefixes(sd)
    return {p: load_linear(sd, p, device, fp8_mode) for p in prefixes}
