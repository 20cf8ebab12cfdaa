"""torch._scaled_mm (FP8 x FP8) on ROCm through the fp8 MFMA kernel.

Mirrors the fast route of ``_patches/scaled_mm_fp8.py``: for e4m3fn x e4m3fn
2-D operands (``input`` [M, K], ``other`` [K, N], usually ``W.t()`` of a
[N, K] weight) the result is ``out_dtype(f32(A @ W^T) * scale_a * scale_b *
scale_result + f32(bias))`` -- every step in f32 in that order and one final
rounding (``_fast_route`` ``:123-146``). ``_fast_eligible`` is the shape /
dtype gate (``:66-81``) and ``_get_backend`` the one-time self-check against
a decode + fp32 matmul (``:84-120``, same shapes, seed and 5e-2 bound).
Everything else keeps the stock op.

Differences from the reference, by design: per-row ``scale_a`` [M, 1] and
per-column ``scale_b`` [1, N] vectors are accepted (applied in the same
order); no size gate unless ``C4Q_FP8_MIN_DIM`` sets one; a failed self-check
or kernel error raises instead of falling back to a decode path.
"""
import os

import torch

from .. import ops
from .._lib import C4QError
from . import _common

TAG = "[cdna4q/scaled_mm]"

_original = None
_installed = False
_self_checked = False


def _min_dim():
    try:
        return int(os.environ.get("C4Q_FP8_MIN_DIM", "0"))
    except ValueError:
        return 0


def _fast_eligible(input, other):
    """Pure shape / dtype predicate (reference ``:66-81``)."""
    if input.dtype != torch.float8_e4m3fn or other.dtype != torch.float8_e4m3fn:
        return False
    if not _common.on_device(input, other):
        return False
    if input.dim() != 2 or other.dim() != 2 or input.shape[1] != other.shape[0]:
        return False
    return max(int(other.shape[1]), int(input.shape[1])) >= _min_dim()


def _get_backend(device):
    """One-time self-check (reference ``:84-120``)."""
    global _self_checked
    if _self_checked:
        return
    g = torch.Generator().manual_seed(0)
    a = (torch.randn(64, 2048, generator=g) * 0.3).to(torch.float8_e4m3fn)
    w = (torch.randn(2048, 2048, generator=g) * 0.3).to(torch.float8_e4m3fn)    # [N, K]
    ad, wd = a.to(device), w.to(device)
    ref = ad.to(torch.float32) @ wd.to(torch.float32).t()
    raw = ops.fp8fp8_matmul2d_nt(ad.view(torch.uint8), wd.view(torch.uint8), 2048, 2048)
    rel = ((raw - ref).abs().max() / (ref.abs().max() + 1e-9)).item()
    if not rel < 5e-2:
        raise C4QError(f"{TAG} fp8 self-check failed (rel={rel:.4f})")
    _self_checked = True


def _fast_route(input, other, scale_a, scale_b, scale_result, bias, out_dtype):
    """fp8 x fp8 -> f32 on the MFMA, scales / bias in f32, one rounding
    (reference ``:123-146``)."""
    _get_backend(input.device)
    return ops.scaled_mm(input, other, out_dtype=out_dtype, scale_a=scale_a, scale_b=scale_b,
                         bias=bias, scale_result=scale_result)


def _rocm_scaled_mm(input, other, *, out_dtype=None, scale_a=None, scale_b=None, bias=None,
                    scale_result=None, use_fast_accum=False):
    """Replacement for ``torch._scaled_mm`` (reference ``_mps_scaled_mm``
    ``:149-207``)."""
    if _fast_eligible(input, other):
        return _fast_route(input, other, scale_a, scale_b, scale_result, bias, out_dtype)
    return _original(input, other, out_dtype=out_dtype, scale_a=scale_a, scale_b=scale_b,
                     bias=bias, scale_result=scale_result, use_fast_accum=use_fast_accum)


def install():
    """Replace ``torch._scaled_mm`` (reference ``:210-219``). Returns True when
    installed; ``C4Q_SCALED_MM=0`` disables it."""
    global _original, _installed
    if _installed:
        return True
    if not hasattr(torch, "_scaled_mm") or not _common.env_on("C4Q_SCALED_MM"):
        return False
    if not _common.rocm_available():
        return False
    _get_backend(torch.device("cuda", torch.cuda.current_device()))
    _original = torch._scaled_mm
    torch._scaled_mm = _rocm_scaled_mm
    _installed = True
    print(f"{TAG} torch._scaled_mm fp8 on ROCm routed to the fp8 MFMA kernel.")
    return True


def uninstall():
    global _installed
    if _installed:
        torch._scaled_mm = _original
        _installed = False
