"""Helpers shared by the patch modules.

``DEVICE_TYPE`` is the torch device type the patches act on (ROCm tensors
report ``"cuda"``); the predicates compare against this name only, so the
routing logic can be exercised on any device by CPU-only tests.
"""
import os

import torch

TAG = "[cdna4q]"
DEVICE_TYPE = "cuda"


def on_device(*tensors):
    """True when every given tensor is a plain tensor on the patched device."""
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor) or t.device.type != DEVICE_TYPE:
            return False
    return True


def env_on(name, default="1"):
    """Per-patch switch: ``name=0`` disables it."""
    return os.environ.get(name, default) != "0"


def rocm_available():
    """A ROCm device is present (HIP build of torch with a visible GPU)."""
    return bool(getattr(torch.version, "hip", None)) and torch.cuda.is_available()


def is_quantized_int8(w):
    """A comfy_kitchen ``QuantizedTensor`` in ``TensorWiseINT8Layout``: int8
    payload in ``_qdata`` [N, K], f32 scale in ``_params.scale`` ([1] or [N]),
    optional ``convrot`` / ``transposed`` flags (checked by attribute, so the
    kitchen package itself is not needed)."""
    return (getattr(w, "_layout_cls", None) == "TensorWiseINT8Layout"
            and hasattr(w, "_qdata") and hasattr(w, "_params"))
