"""ConvRot activation rotation + rowwise INT8 quant (oracle; test
infrastructure only).

The reference's fused o-projection pre-pass ``i8_merge_rot_quant_bf16``
(``_patches/int8_ext/int8_gemm.mm:1429-1507``, host ``:2545-2585``) merges
the attention heads of x [B, H, S, D] into rows [B*S, H*D], rotates every
256-element group with a radix-4 fast Walsh-Hadamard transform, rounds to
bf16 and quantizes each row with the exact ``i8_quant_rowwise`` arithmetic.

The transform is the reference kernel's own: four stages at strides 1, 4,
16, 64, each output the row ``digit`` of

    H4 = [[ 1, 1, 1,-1],
          [ 1, 1,-1, 1],
          [ 1,-1, 1, 1],
          [-1, 1, 1, 1]]

applied to the four values base + k*stride, evaluated in fp32 left to right
as written there (``a0 + a1 + a2 - a3`` ...), then times 2^-4 (exact) and
rounded to bf16. The reference states that this equals comfy_kitchen's
normalized Hadamard matmul up to fp32 summation order; comfy_kitchen is not
in the reference tree, so that equivalence is parity unpinned here.
"""
import numpy as np

from .act import apply_table
from .int8 import quant_rowwise
from .numerics import F32, bf16_bits_to_f32, f32_to_bf16_bits

H4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.int64)


def fwht256(v):
    """Radix-4 FWHT of the last axis (length 256) in fp32, stride order 1, 4,
    16, 64 and the reference's per-output operation order
    (``int8_gemm.mm:1467-1483``). Unnormalized."""
    w = np.asarray(v, dtype=F32).copy()
    assert w.shape[-1] == 256
    idx = np.arange(256)
    for stride in (1, 4, 16, 64):
        digit = (idx // stride) % 4
        base = idx - digit * stride
        a0, a1 = w[..., base], w[..., base + stride]
        a2, a3 = w[..., base + 2 * stride], w[..., base + 3 * stride]
        y0 = ((a0 + a1) + a2) - a3
        y1 = ((a0 + a1) - a2) + a3
        y2 = ((a0 - a1) + a2) + a3
        y3 = ((-a0 + a1) + a2) + a3
        w = np.where(digit == 0, y0, np.where(digit == 1, y1, np.where(digit == 2, y2, y3)))
    return w.astype(F32)


def rotate_bf16(x_bits):
    """bf16 rows [M, K] (K a multiple of 256) -> bf16(fwht256(group) * 2^-4)
    per 256-element group."""
    x = bf16_bits_to_f32(x_bits)
    m, k = x.shape
    r = fwht256(x.reshape(m, k // 256, 256)) * F32(0.0625)
    return f32_to_bf16_bits(r.reshape(m, k))


def merge_heads(x_bits):
    """[B, H, S, D] -> [B*S, H*D]: row (b, s), column h*D + d."""
    b, h, s, d = x_bits.shape
    return np.ascontiguousarray(np.asarray(x_bits).transpose(0, 2, 1, 3).reshape(b * s, h * d))


def merge_rot_quant(x_bits, rotate=True):
    """(q [B*S, H*D] int8, scales [B*S] fp32) of the reference's
    ``i8_merge_rot_quant(x, rotate)``."""
    xm = merge_heads(x_bits)
    if rotate:
        xm = rotate_bf16(xm)
    return quant_rowwise(xm, "bf16")


def swiglu_rot(x_bits, silu_table):
    """The reference's ``i8_swiglu_rot(x)`` (``int8_gemm.mm:1521-1554``, host
    ``:2593-2631``): x [M, 2F] bf16, act = bf16(f32(bf16 SiLU(a)) * f32(b))
    with a the gate columns [0, F) and b the up columns [F, 2F) (the bf16 op
    sequence of silu_mul_split_bf16), then every 256-element group of act
    rotated as in ``rotate_bf16``. The SiLU is the bf16 table given (torch's
    F.silu over every bf16 value in the tests; the reference evaluates
    a / (1 + exp(-a)) with Metal's precise::exp, whose last-ulp agreement
    with that table is parity unpinned)."""
    x = np.asarray(x_bits)
    f = x.shape[1] // 2
    a = bf16_bits_to_f32(apply_table(silu_table, x[:, :f]))
    act = f32_to_bf16_bits(a * bf16_bits_to_f32(x[:, f:]))
    return rotate_bf16(act)
