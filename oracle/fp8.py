"""FP8 e4m3fn routes (oracle; test infrastructure only).

Accumulation is done in float64 and rounded once to float32: every fp8*fp8
and fp8*bf16 product and partial sum at the sizes the tests use is exactly
representable in float64, so this is the exactly-rounded fp32 dot product
that an fp32-accumulating kernel approximates.
"""
import numpy as np

from .numerics import (F32, bf16_bits_to_f32, e4m3fn_decode, e4m3fn_encode,
                       f16_bits_to_f32, f32_to_bf16_bits, f32_to_f16_bits)


def _round_out(x, out_dtype):
    if out_dtype == "bf16":
        return f32_to_bf16_bits(x)
    if out_dtype == "f16":
        return f32_to_f16_bits(x)
    if out_dtype == "f32":
        return np.asarray(x, dtype=F32)
    raise ValueError(out_dtype)


def _bias_f32(bias, bias_dtype):
    if bias is None:
        return None
    if bias_dtype == "bf16":
        return bf16_bits_to_f32(bias)
    if bias_dtype == "f16":
        return f16_bits_to_f32(bias)
    return np.asarray(bias, dtype=F32)


def scaled_mm(a_codes, w_codes, scale_a=None, scale_b=None, bias=None,
              bias_dtype="bf16", scale_result=None, out_dtype="bf16"):
    """``torch._scaled_mm(input, other=W.t(), ...)`` as the reference's fp8
    route computes it (``_patches/scaled_mm_fp8.py:123-146``):

        out = f32(A @ W^T); out *= scale_a; out *= scale_b; out *= scale_result;
        out += f32(bias); out -> out_dtype (one rounding)

    ``a_codes`` [M,K] and ``w_codes`` [N,K] are e4m3fn bytes. scale_a is a
    scalar or [M] (rowwise), scale_b a scalar or [N] (columnwise)."""
    a = e4m3fn_decode(a_codes).astype(np.float64)
    w = e4m3fn_decode(w_codes).astype(np.float64)
    out = (a @ w.T).astype(F32)
    if scale_a is not None:
        sa = np.asarray(scale_a, dtype=F32).reshape(-1)
        out = out * (sa[0] if sa.size == 1 else sa[:, None])
    if scale_b is not None:
        sb = np.asarray(scale_b, dtype=F32).reshape(-1)
        out = out * (sb[0] if sb.size == 1 else sb[None, :])
    if scale_result is not None:
        out = out * np.asarray(scale_result, dtype=F32).reshape(-1)[0]
    b = _bias_f32(bias, bias_dtype)
    if b is not None:
        out = out + b[None, :]
    return _round_out(out.astype(F32), out_dtype)


def quant_pertensor(x_bits, dtype="bf16"):
    """Dynamic per-tensor e4m3fn activation quant (caller side of
    ``torch._scaled_mm``; the reference clamps before every fp8 cast,
    ``_patches/comfykitchen_fp8.py:96``):

        scale = f32(amax|x|) / 448            (correctly rounded divide)
        q     = e4m3fn(clamp(f32(x) / scale, -448, 448))

    An all-zero tensor would give 0/0; it is defined here as scale = 1,
    q = 0 (the kernel does the same). Returns (codes uint8, scale f32)."""
    xf = bf16_bits_to_f32(x_bits) if dtype == "bf16" else f16_bits_to_f32(x_bits)
    amax = np.abs(xf).max() if xf.size else F32(0)
    scale = F32(amax) / F32(448.0)
    if scale == 0:
        scale = F32(1.0)
    y = np.clip(xf / scale, F32(-448.0), F32(448.0)).astype(F32)
    return e4m3fn_encode(y), F32(scale)


def dequant_pertensor(w_codes, scale, out_dtype="bf16"):
    """comfy_kitchen ``dequantize_per_tensor_fp8``:
    ``x.to(out) * scale.to(out)`` — both factors rounded to the output dtype,
    the product rounded once more (reference ``_patches/comfykitchen_fp8.py:15-17,86-89``).
    ``scale=None`` is the plain decode of a standard (unscaled) fp8 weight
    (``_patches/_common.py:249-273``)."""
    w = e4m3fn_decode(w_codes)
    if out_dtype == "bf16":
        if scale is None:
            return f32_to_bf16_bits(w)
        s = bf16_bits_to_f32(f32_to_bf16_bits(np.asarray([scale], dtype=F32)))[0]
        return f32_to_bf16_bits(w * s)
    if out_dtype == "f16":
        if scale is None:
            return f32_to_f16_bits(w)
        s = f16_bits_to_f32(f32_to_f16_bits(np.asarray([scale], dtype=F32)))[0]
        return f32_to_f16_bits(w * s)
    raise ValueError(out_dtype)


def w8a16_linear(x_bits, w_codes, w_scale=None, bias=None, bias_dtype="bf16",
                 x_dtype="bf16", out_dtype="bf16", act=None):
    """W8A16 linear: dequantize the fp8 weight to the activation dtype (kitchen
    formula above), multiply with fp32 accumulation, add the bias in fp32,
    round once (reference ``_patches/linear_fp8_w8a16.py:151-196`` and the
    fused ``bf16(acc + bias_f32)`` store ``_patches/fp8s_ext/w8a16_gemm.mm:101-119``).
    ``act='gelu_tanh'`` then applies bf16 GELU-tanh to the bf16 result (the
    unfused FLUX MLP order). Returns the output bits (or f32)."""
    from .act import apply_table, gelu_tanh_table
    xf = bf16_bits_to_f32(x_bits) if x_dtype == "bf16" else f16_bits_to_f32(x_bits)
    wd = dequant_pertensor(w_codes, w_scale, x_dtype)
    wf = bf16_bits_to_f32(wd) if x_dtype == "bf16" else f16_bits_to_f32(wd)
    acc = (xf.astype(np.float64) @ wf.astype(np.float64).T).astype(F32)
    b = _bias_f32(bias, bias_dtype)
    if b is not None:
        acc = acc + b[None, :]
    out = _round_out(acc, out_dtype)
    if act == "gelu_tanh":
        assert out_dtype == "bf16"
        out = apply_table(gelu_tanh_table(), out)
    elif act is not None:
        raise ValueError(act)
    return out
