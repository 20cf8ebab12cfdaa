"""INT8 W8A8 arithmetic (oracle; test infrastructure only).

Shapes follow the reference's NT convention: activations A[M,K] int8,
weights B[N,K] int8 (the stored nn.Linear layout), output [M,N].
bf16 tensors are uint16 bit arrays (see ``oracle.numerics``).
"""
import numpy as np

from .numerics import (F32, bf16_bits_to_f32, f16_bits_to_f32, f32_to_bf16_bits,
                       f32_to_f16_bits)


def int_mm(a, b):
    """``torch._int_mm(a, b)``: C[M,N] int32 = a[M,K] int8 @ b[K,N] int8.

    Reference seam ``_patches/int_mm_mps.py:90-110`` (exact integer product;
    its canary compares against an int64 CPU matmul, ``:67-81``).
    Computed in float64: every partial sum is an integer of magnitude
    <= 128*128*K < 2**53, so the BLAS float64 product is exact.
    """
    a = np.asarray(a, dtype=np.int8)
    b = np.asarray(b, dtype=np.int8)
    assert a.shape[1] == b.shape[0]
    assert 16384 * a.shape[1] < 2 ** 53
    c = a.astype(np.float64) @ b.astype(np.float64)
    return c.astype(np.int64).astype(np.int32)


def i8_matmul2d_nt(a, b):
    """NT form ``C = A @ B^T`` with B stored [N,K]
    (reference ``_patches/int8_ext/int8_gemm.mm:1655-1703``)."""
    return int_mm(a, np.asarray(b).T)


def _bias_add_bf16(d_bits, bias_bits):
    # second rounding: bf16(f32(D) + f32(bias[n]))  (int8_gemm.mm:116-118)
    return f32_to_bf16_bits(bf16_bits_to_f32(d_bits) + bf16_bits_to_f32(bias_bits)[None, :])


def epilogue_rowscale(c, row_scale, bias_bits=None):
    """Per-tensor fused epilogue: D = bf16(f32(C) * row_scale[m]) [+ bias, 2nd
    rounding]. Reference ``_patches/int8_ext/int8_gemm.mm:97-122``; the host
    pre-multiplies row_scale = w_scale * x_scale
    (``_patches/int8_linear_kernel_mps.py:171``)."""
    cf = np.asarray(c, dtype=np.int32).astype(F32)
    d = f32_to_bf16_bits(cf * np.asarray(row_scale, dtype=F32)[:, None])
    if bias_bits is not None:
        d = _bias_add_bf16(d, bias_bits)
    return d


def epilogue_rowcolscale(c, row_scale, col_scale, bias_bits=None):
    """Per-channel fused epilogue: s = col_scale[n] * row_scale[m] (f32, this
    product first), D = bf16(f32(C) * s) [+ bias, 2nd rounding].
    Reference ``_patches/int8_ext/int8_gemm.mm:417-443``."""
    cf = np.asarray(c, dtype=np.int32).astype(F32)
    s = np.asarray(col_scale, dtype=F32)[None, :] * np.asarray(row_scale, dtype=F32)[:, None]
    d = f32_to_bf16_bits(cf * s)
    if bias_bits is not None:
        d = _bias_add_bf16(d, bias_bits)
    return d


def epilogue_rowcolscale_half(c, row_scale, col_scale, bias_f16_bits=None):
    """fp16 per-channel epilogue: s = col_scale[n] * row_scale[m] (f32),
    D = half(f32(C) * s), then with a bias D = half(f32(D) + f32(bias[n])),
    bias in fp16. Half rounding is RNE and overflows to +-inf, as Metal's
    half() conversion. Reference ``_patches/int8_ext/int8_gemm.mm:1161-1183``
    (entry ``i8_matmul2d_nt_fused_cs_half`` ``:1965-2010``)."""
    cf = np.asarray(c, dtype=np.int32).astype(F32)
    s = np.asarray(col_scale, dtype=F32)[None, :] * np.asarray(row_scale, dtype=F32)[:, None]
    d = f32_to_f16_bits(cf * s)
    if bias_f16_bits is not None:
        d = f32_to_f16_bits(f16_bits_to_f32(d) + f16_bits_to_f32(bias_f16_bits)[None, :])
    return d


def scatter_qkv(d_bits, heads, head_dim):
    """[M, 3 H D] -> (Q, K, V), each [1, H, M, D]: column kind*H*D + h*D + d
    to out_kind[0, h, m, d] (reference ``int8_gemm.mm:466-471``)."""
    d = np.asarray(d_bits)
    m = d.shape[0]
    x = d.reshape(m, 3, heads, head_dim).transpose(1, 2, 0, 3)
    return [np.ascontiguousarray(x[k][None]) for k in range(3)]


def lora_delta_add(d_bits, delta_bits, delta_scale):
    """Runtime-LoRA delta term of the H3 partition epilogue, added to the
    bf16 projection value d (after its bias): ls = bf16(delta_scale),
    sd = bf16(f32(delta) * f32(ls)), out = bf16(f32(d) + f32(sd)).
    Reference ``_patches/int8_ext/int8_gemm.mm:947,966-968`` (Q/K) and
    ``:1048,1062-1064`` (V); delta_scale arrives as a float32
    (``float ds = (float)delta_scale``, ``:2297``)."""
    ls = bf16_bits_to_f32(f32_to_bf16_bits(np.asarray([delta_scale], dtype=F32)))[0]
    sd = f32_to_bf16_bits(bf16_bits_to_f32(delta_bits) * ls)
    return f32_to_bf16_bits(bf16_bits_to_f32(d_bits) + bf16_bits_to_f32(sd))


def scatter_part(d_bits, heads, head_dim):
    """One partition [M, H D] -> [1, H, M, D]: column h*D + d to
    out[0, h, m, d] (reference ``int8_gemm.mm:1065-1068``)."""
    d = np.asarray(d_bits)
    m = d.shape[0]
    return np.ascontiguousarray(d.reshape(m, heads, head_dim).transpose(1, 0, 2)[None])


BF16_TINY = F32(2.0 ** -126)   # torch.finfo(torch.bfloat16).tiny
F16_TINY = F32(2.0 ** -14)     # torch.finfo(torch.float16).tiny


def quant_rowwise(x_bits, dtype="bf16"):
    """Rowwise symmetric int8 activation quant, bit-exact restatement of
    comfy_kitchen ``quantize_int8_rowwise`` as the reference spells it out
    (``_patches/int8_ext/int8_gemm.mm:1337-1381``):

        amax  = max|x| over the row                (exact)
        scale = max(f32(amax) / 127, 1e-30)        (correctly rounded divide)
        s     = dtype(scale); s == 0 -> finfo(dtype).tiny
        q     = int8(clamp(rint(dtype(f32(x) / f32(s))), -128, 127))

    Returns (q int8 [M,K], scale f32 [M]).
    """
    x_bits = np.asarray(x_bits, dtype=np.uint16)
    if dtype == "bf16":
        xf = bf16_bits_to_f32(x_bits)
        to_bits, from_bits, tiny = f32_to_bf16_bits, bf16_bits_to_f32, BF16_TINY
    elif dtype == "f16":
        xf = f16_bits_to_f32(x_bits)
        to_bits, from_bits, tiny = f32_to_f16_bits, f16_bits_to_f32, F16_TINY
    else:
        raise ValueError(dtype)
    M, K = xf.shape
    amax = np.abs(xf).max(axis=1) if K else np.zeros(M, dtype=F32)
    scale = np.maximum(amax.astype(F32) / F32(127.0), F32(1e-30)).astype(F32)
    s = from_bits(to_bits(scale))
    s = np.where(s == 0, tiny, s).astype(F32)
    d = from_bits(to_bits(xf / s[:, None]))
    q = np.clip(np.rint(d), -128, 127).astype(np.int8)
    return q, scale


def int8_linear(x_bits, w, w_scale, bias_bits=None, x_dtype="bf16"):
    """comfy_kitchen ``int8_linear`` (no convrot) as the reference's kernel
    route computes it (``_patches/int8_linear_kernel_mps.py:152-215``,
    ``:218-263``): rowwise-quantize x, INT8 GEMM against the [N,K] weight,
    then the per-tensor or per-channel fused epilogue; bf16 out."""
    q, xs = quant_rowwise(x_bits, x_dtype)
    c = i8_matmul2d_nt(q, w)
    ws = np.asarray(w_scale, dtype=F32).reshape(-1)
    if ws.size == 1:
        return epilogue_rowscale(c, ws[0] * xs, bias_bits)
    return epilogue_rowcolscale(c, xs, ws, bias_bits)
