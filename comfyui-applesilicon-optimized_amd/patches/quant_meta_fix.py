"""Missing ``format`` in per-layer ``comfy_quant`` metadata defaults to
``int8_tensorwise`` for int8 weights with a ``weight_scale``.

Mirrors ``_patches/quant_meta_fix.py``: community int8 ConvRot checkpoints
ship descriptors such as ``{"convrot": true, "convrot_groupsize": 256,
"per_row": true}`` without ``"format"``, which comfy's
``_load_quantized_module`` rejects although the tensors are laid out exactly
like declared ``int8_tensorwise`` layers. ``install`` wraps that loader so
each layer's descriptor is repaired (``formats.fix_quant_meta``) before the
original runs; anything not positively identified (other dtypes, no scale)
is left as it is. Host-side metadata only: it needs ComfyUI, not the GPU.
"""
from .. import formats
from . import _common

TAG = "[cdna4q/quant_meta]"

_installed = False
_fixed_layers = 0


def _maybe_fix(state_dict, prefix):
    """The reference's per-layer repair (``quant_meta_fix.py:34-59``)."""
    global _fixed_layers
    if formats.fix_quant_meta(state_dict, prefix):
        if _fixed_layers == 0:
            print(f"{TAG} comfy_quant metadata without 'format': int8 + weight_scale layers "
                  f"default to int8_tensorwise (first: {prefix.rstrip('.')}).")
        _fixed_layers += 1


def install():
    """Wrap ``comfy.ops._load_quantized_module``; False when ComfyUI (or that
    loader) is absent or the patch is switched off (``C4Q_QUANT_META_FIX=0``)."""
    global _installed
    if _installed:
        return True
    if not _common.env_on("C4Q_QUANT_META_FIX"):
        return False
    try:
        import comfy.ops as comfy_ops
    except Exception:
        return False
    orig = getattr(comfy_ops, "_load_quantized_module", None)
    if orig is None:
        return False

    def wrapper(module, load_fn, state_dict, prefix, *args, **kwargs):
        _maybe_fix(state_dict, prefix)
        return orig(module, load_fn, state_dict, prefix, *args, **kwargs)

    comfy_ops._load_quantized_module = wrapper
    _installed = True
    return True
