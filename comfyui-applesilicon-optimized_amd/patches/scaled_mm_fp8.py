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
order); no size gate unless ``C4Q_FP8_MIN_DIM`` sets one; a failed one-time
self-check raises (a broken kernel must not go unnoticed). Calls outside the
kernel's argument set (``out_dtype=None`` or fp8, blockwise / MX scales,
other bias shapes) and calls the kernel rejects keep the stock ROCm op.
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


_OUT_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _scale_ok(s, n, layout_shapes, device):
    """None, or an f32 tensor on `device` holding one value (per tensor) or
    one per row / column in one of `layout_shapes`."""
    if s is None:
        return True
    if not isinstance(s, torch.Tensor) or s.dtype != torch.float32 or s.device != device:
        return False
    return s.numel() == 1 or (s.numel() == n and tuple(s.shape) in layout_shapes)


def _fast_eligible(input, other, out_dtype=torch.bfloat16, scale_a=None, scale_b=None,
                   scale_result=None, bias=None):
    """Pure argument predicate, no device work (reference ``:66-81``),
    widened to every argument the fp8 kernel's epilogue takes: e4m3fn 2-D
    operands on the ROCm device, ``out_dtype`` bf16 / f16 / f32 (None keeps
    the stock op, whose output is then fp8), f32 scales per tensor, per row
    ([M, 1] or [M]) for ``scale_a`` and per column ([1, N] or [N]) for
    ``scale_b``, a per-tensor ``scale_result``, and a bf16 / f16 / f32 bias
    of N values. Blockwise or MX (e8m0) scales and fp8 outputs keep the
    stock op."""
    if input.dtype != torch.float8_e4m3fn or other.dtype != torch.float8_e4m3fn:
        return False
    if not _common.on_device(input, other) or input.device != other.device:
        return False
    if input.dim() != 2 or other.dim() != 2 or input.shape[1] != other.shape[0]:
        return False
    if out_dtype not in _OUT_DTYPES:
        return False
    M, N = int(input.shape[0]), int(other.shape[1])
    dev = input.device
    if not (_scale_ok(scale_a, M, ((M, 1), (M,)), dev) and _scale_ok(scale_b, N, ((1, N), (N,)), dev)
            and _scale_ok(scale_result, 1, (), dev)):
        return False
    if bias is not None and not (isinstance(bias, torch.Tensor) and bias.dtype in _OUT_DTYPES
                                 and bias.device == dev and bias.numel() == N
                                 and bias.dim() == 1):
        return False
    return max(N, int(input.shape[1])) >= _min_dim()


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
    ``:149-207``): eligible calls take the fp8 MFMA route; a call the kernel
    rejects falls back to the stock op, as the reference's fast route falls
    back to its decode path (``:172-176``)."""
    if _fast_eligible(input, other, out_dtype, scale_a, scale_b, scale_result, bias):
        try:
            return _fast_route(input, other, scale_a, scale_b, scale_result, bias, out_dtype)
        except C4QError as e:
            print(f"{TAG} fp8 route declined ({e}); using the stock op.")
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
