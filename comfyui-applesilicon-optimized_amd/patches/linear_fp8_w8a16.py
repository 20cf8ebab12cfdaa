"""Standard-fp8 Linear (e4m3fn weights) through the W8A16 MFMA kernel.

Mirrors ``_patches/linear_fp8_w8a16.py``: ComfyUI's fp8 Linear normally
decodes the whole [N, K] fp8 weight to bf16 on every forward
(``cast_bias_weight``) and then calls ``F.linear``; the replacement forward
consumes the fp8 bytes directly (dequantized in registers) and adds the bias
in f32 before the single output rounding (``:151-196``). ``_eligible`` is the
per-call gate (``:89-117``), ``_self_check`` the one-time parity check of the
first eligible layer against a decode + fp32 matmul (``:120-148``, the same
5e-2 relative bound).

Differences from the reference, by design:

* the activation stays bf16 (the reference converts it to fp16 for its half
  kernel); the MFMA takes bf16 directly, so nothing is rounded on the way in;
* a per-tensor ``scale_weight`` on the layer (comfy's scaled-fp8 Linear) is
  honoured with the comfy_kitchen dequant formula, bit-exact;
* no size gate: the reference's ``max(N, K) >= 3072`` / ``M <= 4096`` gates are
  M5 bench results; ``C4Q_W8A16_MIN_DIM`` / ``C4Q_W8A16_M_MAX`` restore them;
* a failed self-check or kernel error raises instead of latching back to the
  decode path.
"""
import os

import torch

from .. import ops
from .._lib import C4QError
from . import _common

TAG = "[cdna4q/w8a16]"

_installed = False
_orig_forward = None
_self_checked = False
_ELIGIBLE_INPUT_DTYPES = (torch.bfloat16, torch.float16)


def _int_env(name, default):
    try:
        return int(os.environ.get(name, default))
    except ValueError:
        return default


def _weight_scale(module):
    s = getattr(module, "scale_weight", None)
    if s is None:
        return None
    return s if isinstance(s, torch.Tensor) and s.numel() == 1 else False


def _eligible(module, input):
    """Per-call gate over attributes only, nothing enqueued (reference
    ``:89-117``). Served: a plain 2-D contiguous e4m3fn weight on the ROCm
    device (tensor subclasses such as QuantizedTensor hide their dtype or
    keep their own forward), a bf16 / f16 input of matching K, no weight or
    bias functions (a LoRA patch needs the decoded weight), no offload
    bookkeeping, at most a per-tensor weight scale, and the optional size
    gates."""
    w = getattr(module, "weight", None)
    if w is None or getattr(w, "dtype", None) != torch.float8_e4m3fn:
        return False
    if type(w) not in (torch.Tensor, torch.nn.Parameter):
        return False
    if w.dim() != 2 or not _common.on_device(w) or not w.is_contiguous():
        return False
    if input.dtype not in _ELIGIBLE_INPUT_DTYPES or not _common.on_device(input):
        return False
    if input.shape[-1] != w.shape[1]:
        return False
    if len(getattr(module, "weight_function", [])) > 0 or len(getattr(module, "bias_function", [])) > 0:
        return False
    if hasattr(module, "_v") or hasattr(module, "_prefetch"):
        return False
    if _weight_scale(module) is False:
        return False
    N, K = int(w.shape[0]), int(w.shape[1])
    M = input.numel() // input.shape[-1]
    if max(N, K) < _int_env("C4Q_W8A16_MIN_DIM", 0):
        return False
    m_max = _int_env("C4Q_W8A16_M_MAX", 0)
    return not (m_max and M > m_max)


def _self_check(module, x2d):
    """One-time parity check on the first eligible layer's real weight against
    a decode + fp32 matmul (reference ``:120-148``)."""
    rows = x2d[: min(int(x2d.shape[0]), 32)].contiguous()
    w = module.weight
    ws = _weight_scale(module)
    wd = ops.fp8_dequant(w, ws, torch.float32) if ws is not None else w.to(torch.float32)
    ref = rows.float() @ wd.t()
    out = ops.w8a16_linear(rows, w, ws, out_dtype=torch.float32)
    rel = ((out - ref).abs().max() / (ref.abs().max() + 1e-9)).item()
    if not rel < 5e-2:
        raise C4QError(f"{TAG} self-check failed (rel={rel:.4f})")
    print(f"{TAG} self-check ok (rel={rel:.2e}); W8A16 MFMA path live.")


def _w8a16_forward(module, input):
    """Kernel-backed replacement for ``Linear.forward_comfy_cast_weights`` on the
    standard-fp8 path (reference ``:151-196``): out = input.dtype(acc_f32 +
    bias_f32), one rounding."""
    global _self_checked
    orig_shape = input.shape
    x2d = input.reshape(-1, orig_shape[-1])
    if not _self_checked:
        _self_check(module, x2d)
        _self_checked = True
    bias = module.bias
    if bias is not None:
        bias = bias.to(torch.float32)          # fp8 / bf16 / f16 biases widen exactly
    out = ops.w8a16_linear(x2d, module.weight, _weight_scale(module), bias, out_dtype=input.dtype)
    return out.reshape(*orig_shape[:-1], module.weight.shape[0])


def _patched_forward(self, input):
    if _eligible(self, input):
        return _w8a16_forward(self, input)
    return _orig_forward(self, input)


def install():
    """Replace ``comfy.ops.disable_weight_init.Linear.forward_comfy_cast_weights``
    (reference ``:222-258``). Returns True when installed (ComfyUI importable
    and a ROCm device present); ``C4Q_W8A16=0`` disables it."""
    global _installed, _orig_forward
    if _installed:
        return True
    if not _common.env_on("C4Q_W8A16") or not _common.rocm_available():
        return False
    try:
        import comfy.ops as comfy_ops
    except Exception:
        return False
    _orig_forward = comfy_ops.disable_weight_init.Linear.forward_comfy_cast_weights
    comfy_ops.disable_weight_init.Linear.forward_comfy_cast_weights = _patched_forward
    _installed = True
    print(f"{TAG} standard-fp8 Linear routed through the W8A16 MFMA kernel.")
    return True
