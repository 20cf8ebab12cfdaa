"""Fused INT8 gate/up FFN pair with the SiLU-gated epilogue (Krea2 SwiGLU).

Mirrors ``_patches/krea2_ffn_pair.py`` ``project`` (``:37-49``): the
activation is rowwise-quantized once, one pair kernel multiplies it with the
gate and up int8 weights (both [F, K], per-output-channel f32 scales) and
stores ``bf16(bf16(SiLU(g)) * u)`` with ``g = bf16(acc_g * (gs * rs))``,
``u = bf16(acc_u * (us * rs))`` -- the exact bf16 intermediates of the unfused
chain (``krea2_ffn_pair.metal:281-304``). ``candidate`` mirrors the SwiGLU
forward seam (``:66-81``): eligible bf16 activations go through ``project``
and then the down projection, anything else keeps the original forward.

Not supported here: the ConvRot pre-rotation the reference applies to the
activation (comfy_kitchen's Hadamard rounding is not pinned), so
``convrot=True`` weights keep the original forward.
"""
import torch

from .. import ops
from .._lib import C4QError
from . import _common
from .int8_linear import _quant_cached

TAG = "[cdna4q/krea2_pair]"
calls = 0


def _weight(w):
    """(int8 [F, K], f32 scale [F]) of a TensorWiseINT8Layout QuantizedTensor or
    an explicit (qdata, scale) pair."""
    if isinstance(w, tuple):
        return w
    return w._qdata, w._params.scale.reshape(-1)


def project_prequant(q, scales, g, u):
    """Pair kernel on an already quantized activation q [M, K] int8 with
    per-row scales [M]; g / u are (qdata [F, K], scale [F]) or QuantizedTensors."""
    gq, gs = _weight(g)
    uq, us = _weight(u)
    silu = ops.act_table("silu", q.device)
    return ops.ffn_pair(q, gq, uq, scales.reshape(-1).float().contiguous(),
                        gs.float().contiguous(), us.float().contiguous(), silu, None)


def project(x, g, u):
    """x [..., K] bf16 -> bf16 [..., F] = SiLU(gate(x)) * up(x) on the int8 route
    (reference ``project`` ``:37-49``)."""
    global calls
    if x.dtype != torch.bfloat16:
        raise C4QError(f"{TAG} x must be bf16")
    q, s = _quant_cached(x)
    out = project_prequant(q, s, g, u)
    calls += 1
    return out.reshape(*x.shape[:-1], out.shape[-1])


def _eligible_layer(layer):
    w = getattr(layer, "weight", None)
    if not _common.is_quantized_int8(w) or getattr(layer, "bias", None) is not None:
        return False
    p = w._params
    return (not getattr(p, "convrot", False) and not getattr(p, "transposed", False)
            and w._qdata.dtype == torch.int8 and w._qdata.is_contiguous()
            and p.scale.numel() == w._qdata.shape[0]
            and not len(getattr(layer, "weight_function", []))
            and not len(getattr(layer, "bias_function", [])))


def candidate(original, self, x):
    """SwiGLU forward seam (reference ``candidate`` ``:66-81``): ``self.gate``,
    ``self.up``, ``self.down`` linear layers."""
    if (torch.is_grad_enabled() or not _common.on_device(x) or x.dtype != torch.bfloat16
            or not x.is_contiguous() or not _eligible_layer(self.gate)
            or not _eligible_layer(self.up)
            or self.gate.weight._qdata.shape != self.up.weight._qdata.shape):
        return original(self, x)
    return self.down(project(x, self.gate.weight, self.up.weight))


def install():
    """Hook ``comfy.ldm.krea2.model.SwiGLU.forward`` when ComfyUI's Krea2 model is
    importable and a ROCm device is present; ``C4Q_KREA2_FFN_PAIR=0`` disables it."""
    if not _common.env_on("C4Q_KREA2_FFN_PAIR") or not _common.rocm_available():
        return False
    try:
        import comfy.ldm.krea2.model as krea
    except Exception:
        return False
    original = krea.SwiGLU.forward
    if getattr(original, "_c4q_pair", False):
        return True

    def forward(self, x):
        return candidate(original, self, x)

    forward._c4q_pair = True
    krea.SwiGLU.forward = forward
    return True
