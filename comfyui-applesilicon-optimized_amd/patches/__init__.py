"""ComfyUI / torch seams of the quantized linear path on ROCm, one module per
reference patch:

    int_mm            torch._int_mm                  (_patches/int_mm_mps.py)
    scaled_mm_fp8     torch._scaled_mm, fp8 route    (_patches/scaled_mm_fp8.py)
    int8_linear       comfy_kitchen int8_linear, mixed_precision_ops Linear,
                      linear_input_act SwiGLU        (_patches/int8_linear_kernel_mps.py)
    int8_fast         int8-fast dynamic forwards     (_patches/int8_linear_mps.py)
    linear_fp8_w8a16  standard-fp8 Linear forward    (_patches/linear_fp8_w8a16.py)
    krea2_ffn_pair    Krea2 SwiGLU gate/up pair      (_patches/krea2_ffn_pair.py)
    moss_ffn          MOSS FC1 + SiTU pair           (_patches/moss_ffn_mps.py)
    moss_bf16_ffn_pair  MOSS bf16 FC1 + SiTU pair    (_patches/moss_bf16_ffn_pair.py)
    quant_meta_fix    comfy_quant metadata repair    (_patches/quant_meta_fix.py)

``install_all()`` installs every patch whose host (a ROCm device, ComfyUI for
the model seams) is present and returns the names installed. Each module also
honours its own ``C4Q_<NAME>=0`` switch.
"""
from . import (int8_fast, int8_linear, int_mm, krea2_ffn_pair, linear_fp8_w8a16, moss_bf16_ffn_pair,
               moss_ffn, quant_meta_fix, scaled_mm_fp8)
from . import _common

_ALL = (("int_mm", int_mm), ("scaled_mm_fp8", scaled_mm_fp8), ("int8_linear", int8_linear),
        ("int8_fast", int8_fast), ("linear_fp8_w8a16", linear_fp8_w8a16), ("krea2_ffn_pair", krea2_ffn_pair),
        ("moss_ffn", moss_ffn), ("moss_bf16_ffn_pair", moss_bf16_ffn_pair),
        ("quant_meta_fix", quant_meta_fix))


def install_all():
    done = []
    for name, mod in _ALL:
        if not _common.env_on(f"C4Q_{name.upper()}"):
            continue
        if mod.install():
            done.append(name)
    return done
