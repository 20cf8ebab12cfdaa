"""int8-fast's wide-batch forwards on the W8A8 MFMA route.

Mirrors ``_patches/int8_linear_mps.py``. The ``int8-fast`` custom node's
``int8_quant`` module computes its wide-batch Linear with
``int8_forward_dynamic`` (per-tensor weight scale) and
``int8_forward_dynamic_per_row`` (per-output-channel scale), both
``(x, weight, weight_scale, bias, compute_dtype)``: rowwise int8 activation
quant, ``torch._int_mm(x_8, weight.T)``, rescale by ``weight_scale * x_scale``,
``+ bias``, compute dtype. On ROCm the same computation runs as the fused
INT8 GEMM (``int8_linear.int8_forward_dynamic[_per_row]``); other calls
(tensors off the ROCm device, non-int8 weights, fp32 activations) keep
int8-fast's own function.

int8-fast may be imported before this package (then ``_scan_loaded`` finds
its module in ``sys.modules``) or after it (then ``_Finder``, a meta-path
finder placed first, wraps the module's loader and patches it right after
it executes) -- the reference's ``_apply`` / ``_scan_loaded`` / ``_Finder``
(``:66-142``). Differences from the reference, by design: the route keeps
W8A8 (the reference dequantizes to bf16 and calls ``F.linear``, its fastest
GEMM on MPS); the int8-fast quantizer ``quantize_int8_axiswise`` is
third-party code absent from the reference tree, so agreement of its bytes
with this build's rowwise quant is unpinned.
"""
import sys

import torch

from . import _common
from . import int8_linear

TAG = "[cdna4q/int8_fast]"

_installed = False     # install() ran
_patched = False       # an int8_quant module was patched
_orig_dyn = None
_orig_dyn_pr = None
_finder = None


def _served(x, weight):
    return (_common.on_device(x, weight) and isinstance(weight, torch.Tensor)
            and weight.dtype == torch.int8 and weight.dim() == 2
            and x.dtype in (torch.bfloat16, torch.float16) and x.shape[-1] == weight.shape[1])


def _dyn(x, weight, weight_scale, bias, compute_dtype):
    """Replacement for ``int8_quant.int8_forward_dynamic`` (reference ``:54-57``)."""
    if _served(x, weight):
        return int8_linear.int8_forward_dynamic(x, weight, weight_scale, bias, compute_dtype)
    return _orig_dyn(x, weight, weight_scale, bias, compute_dtype)


def _dyn_pr(x, weight, weight_scale, bias, compute_dtype):
    """Replacement for ``int8_quant.int8_forward_dynamic_per_row`` (reference ``:60-63``)."""
    if _served(x, weight):
        return int8_linear.int8_forward_dynamic_per_row(x, weight, weight_scale, bias,
                                                        compute_dtype)
    return _orig_dyn_pr(x, weight, weight_scale, bias, compute_dtype)


def _apply(mod):
    """Patch an ``int8_quant`` module in place, once (reference ``:66-81``).
    A module without both forwards is left alone."""
    global _patched, _orig_dyn, _orig_dyn_pr
    if _patched:
        return
    if not (hasattr(mod, "int8_forward_dynamic") and hasattr(mod, "int8_forward_dynamic_per_row")):
        return
    _orig_dyn = mod.int8_forward_dynamic
    _orig_dyn_pr = mod.int8_forward_dynamic_per_row
    mod.int8_forward_dynamic = _dyn
    mod.int8_forward_dynamic_per_row = _dyn_pr
    _patched = True
    print(f"{TAG} int8-fast wide-batch forwards routed to the INT8 MFMA kernels.")


def _scan_loaded():
    """Patch an already imported ``int8_quant`` module (reference ``:84-94``)."""
    for mod in list(sys.modules.values()):
        try:
            name = getattr(mod, "__name__", "") or ""
            if name.rsplit(".", 1)[-1] == "int8_quant" and hasattr(mod, "int8_forward_dynamic"):
                _apply(mod)
                if _patched:
                    return True
        except Exception:
            continue
    return False


class _Finder:
    """Meta-path finder for a module named ``int8_quant``: finds its spec with
    the other finders and wraps the loader's ``exec_module`` so the module is
    patched as soon as it has executed (reference ``:97-128``). It never
    breaks the import: a failed patch is reported and the module kept."""

    def find_spec(self, fullname, path, target=None):
        if _patched or fullname.rsplit(".", 1)[-1] != "int8_quant":
            return None
        spec = None
        for finder in sys.meta_path:
            if finder is self or not hasattr(finder, "find_spec"):
                continue
            try:
                spec = finder.find_spec(fullname, path, target)
            except Exception:
                spec = None
            if spec is not None:
                break
        if spec is None or spec.loader is None or not hasattr(spec.loader, "exec_module"):
            return None
        orig_exec = spec.loader.exec_module

        def exec_module(module, _orig_exec=orig_exec):
            _orig_exec(module)
            try:
                _apply(module)
            except Exception as e:
                print(f"{TAG} post-import patch failed: {e!r}")

        try:
            spec.loader.exec_module = exec_module
        except Exception:
            return None
        return spec


def install():
    """Patch int8-fast now if it is loaded, else when it is imported
    (reference ``:131-142``). Returns True when installed (a ROCm device is
    present); ``C4Q_INT8_FAST=0`` disables it."""
    global _installed, _finder
    if _installed:
        return True
    if not _common.env_on("C4Q_INT8_FAST") or not _common.rocm_available():
        return False
    _installed = True
    if not _scan_loaded():
        _finder = _Finder()
        sys.meta_path.insert(0, _finder)
    return True
