"""cdna4q: the quantized linear path of the ComfyUI Apple-Silicon pack
(luix93/ComfyUI-AppleSilicon-Optimized), rebuilt for AMD Instinct MI355X.

This directory is a ComfyUI custom-node package (ComfyUI imports it by path,
like the reference's ``__init__.py``). It registers no nodes; importing it
installs the patches of ``patches/`` when ``C4Q_INSTALL=1`` is set.

    ops       tensor-level entry points over libcdna4q.so (HIP / gfx950)
    patches   ComfyUI / torch seams: torch._int_mm, torch._scaled_mm, the
              comfy_kitchen int8_linear route, the fp8 W8A16 Linear forward,
              the Krea2 / MOSS FFN pairs
"""
import os

NODE_CLASS_MAPPINGS = {}
NODE_DISPLAY_NAME_MAPPINGS = {}

if os.environ.get("C4Q_INSTALL") == "1":
    from . import patches as _patches
    _patches.install_all()
