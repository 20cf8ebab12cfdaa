"""Fused INT8 gate/up FFN pair with the SiLU-gated epilogue (Krea2 SwiGLU).

Mirrors ``_patches/krea2_ffn_pair.py`` ``project`` (``:37-49``): the
activation is ConvRot-rotated (256-wide normalized Hadamard per group) and
rowwise-quantized once, through the fused rotate + quant pass
(``int8_linear._quant_cached(x, True, 256)``, reference ``:41``); one pair
kernel multiplies it with the gate and up int8 weights (both [F, K],
per-output-channel f32 scales) and stores ``bf16(bf16(SiLU(g)) * u)`` with
``g = bf16(acc_g * (gs * rs))``, ``u = bf16(acc_u * (us * rs))`` -- the
exact bf16 intermediates of the unfused chain
(``krea2_ffn_pair.metal:281-304``). ``candidate`` mirrors the SwiGLU forward
seam (``:66-81``): eligible bf16 activations go through ``project`` and then
the down projection, anything else keeps the original forward.

Eligible layers are the reference's (``_patches/moss_ffn_mps.py:30-54``):
TensorWiseINT8Layout weights with ConvRot group size 256, contiguous int8
payload, one f32 scale per output row, no bias, no transposition, no LoRA /
low-VRAM functions, hooks, forced casts, full-precision flag or runtime
adapter. The reference's Krea2 shape gates (``x`` [1, 4096..14336, 6144],
weights [16384, 6144]) are M5 bench results and are not applied; the
rotation pass needs K % 256 == 0 and K <= 15360.
"""
import os

import torch

from .. import ops
from .._lib import C4QError
from . import _common
from .int8_linear import _RUNTIME_LORA_ATTR, _convrot_ok, _quant_cached

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
    """x [..., K] bf16 -> bf16 [..., F] = SiLU(gate(x)) * up(x) on the int8
    route, the activation rotated and quantized as the reference does
    (``project`` ``:37-49``)."""
    global calls
    if x.dtype != torch.bfloat16:
        raise C4QError(f"{TAG} x must be bf16")
    q, s = _quant_cached(x, True, 256)
    out = project_prequant(q, s, g, u)
    calls += 1
    return out.reshape(*x.shape[:-1], out.shape[-1])


_LAYER_FLAGS = ("weight_function", "bias_function", "weight_lowvram_function",
                "bias_lowvram_function", "_forward_hooks", "_forward_pre_hooks",
                "_full_precision_mm", "comfy_force_cast_weights", _RUNTIME_LORA_ATTR)


def _eligible_layer(layer, device):
    """The reference's layer gate (``moss_ffn_mps.py:30-54``) without its
    source-hash and shape checks."""
    if hasattr(layer, "_v") or getattr(layer, "bias", None) is not None:
        return False
    if any(getattr(layer, key, None) for key in _LAYER_FLAGS):
        return False
    w = getattr(layer, "weight", None)
    if not _common.is_quantized_int8(w):
        return False
    p = w._params
    q, scale = w._qdata, p.scale
    return (isinstance(q, torch.Tensor) and q.device == device and q.dtype == torch.int8
            and q.dim() == 2 and q.is_contiguous()
            and isinstance(scale, torch.Tensor) and scale.device == device
            and scale.dtype == torch.float32 and scale.numel() == q.shape[0]
            and scale.is_contiguous()
            and bool(getattr(p, "convrot", False))
            and getattr(p, "convrot_groupsize", None) == 256
            and not getattr(p, "transposed", False))


def candidate(original, self, x):
    """SwiGLU forward seam (reference ``candidate`` ``:66-81``): ``self.gate``,
    ``self.up``, ``self.down`` linear layers."""
    if (not _common.env_on("C4Q_KREA2_FFN_PAIR", os.environ.get("ASFP8_KREA2_FFN_PAIR", "1"))
            or torch.is_grad_enabled() or not _common.on_device(x)
            or x.dtype != torch.bfloat16 or not x.is_contiguous()
            or not _convrot_ok(x, 256)):
        return original(self, x)
    if _global_hooks():
        return original(self, x)
    for layer in (self.gate, self.up):
        if ("forward" in getattr(layer, "__dict__", {}) or getattr(layer, "comfy_force_forward", False)
                or not _eligible_layer(layer, x.device)):
            return original(self, x)
    gq, uq = self.gate.weight._qdata, self.up.weight._qdata
    if gq.shape != uq.shape or gq.shape[1] != x.shape[-1]:
        return original(self, x)
    try:
        h = project(x, self.gate.weight, self.up.weight)
    except C4QError as e:
        print(f"{TAG} pair fell back ({e})")
        return original(self, x)
    return self.down(h)


def _global_hooks():
    """A global module forward (pre-)hook is registered: the fused route would
    skip it, so the original forward runs (reference ``:70-72``)."""
    from torch.nn.modules import module as module_hooks
    return bool(module_hooks._global_forward_hooks or module_hooks._global_forward_pre_hooks)


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
