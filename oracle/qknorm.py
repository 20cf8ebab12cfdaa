"""Q/K RMSNorm + partial split-half RoPE of the H3 QKV projection (oracle;
test infrastructure only).

The reference's fused epilogue ``int8_matmul_fused_cs_qkv_rms_rope_impl``
(``_patches/int8_ext/int8_gemm.mm:683-861``, host ``:2111-2209``) takes
the bf16 projection value x of each Q and K head row (D = 128, the exact
per-channel dequant + bias value of the QKV scatter) and computes, in fp32:

    inv = rsqrt(sum_d x_d^2 / 128 + eps)                        (:806-832)
    y_d = bf16((x_d * inv) * w_d)       w: fp32 q or k weight   (:833)
    d < 2R, i = d mod R, r = [d >= R], f = freqs[m, i, r, :]    (:840-854)
        out_d = bf16(bf16(f[r] * y_d) + f[1-r] * y_partner)
        partner = d + R (r = 0) or d - R (r = 1)
    d >= 2R: out_d = y_d

The RoPE step is comfy_kitchen's eager form ``out = y * diag;
out.addcmul_(rotated y, off-diagonal)`` (the reference's comment at
``:848-849``; comfy_kitchen is a third-party package absent from the
reference tree): the diagonal product is rounded to bf16 first, the
off-diagonal product (exact in fp32: bf16 x bf16) is added with one
rounding. Every product here of two bf16 values is exact in fp32.

The reference sums the squares as lane t of a 32-wide SIMD-group over
elements 4t..4t+3, then a hardware ``simd_sum``, whose order Apple does not
publish. This restatement fixes the order the MI355X kernel uses: 8 partial
sums, partial j over columns 8j..8j+7 then 64+8j..64+8j+7 in that order,
combined as ((p0+p4)+(p2+p6)) + ((p1+p5)+(p3+p7)); the reciprocal square
root is 1 / sqrt(.) with correctly rounded sqrt and division. Against the
reference's order these differ only in fp32 rounding of the sum (a few
ulps), which the tests bound against an exact float64 evaluation.
"""
import numpy as np

from .numerics import F32, bf16_bits_to_f32, f32_to_bf16_bits

HEAD_DIM = 128


def _bf16(v):
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(v, dtype=F32)))


def lane_columns(j):
    """Columns whose squares partial sum j adds, in order."""
    return list(range(8 * j, 8 * j + 8)) + list(range(64 + 8 * j, 72 + 8 * j))


def sum_squares(x):
    """fp32 sum of squares over the last axis (128) in the fixed order above."""
    x = np.asarray(x, dtype=F32)
    assert x.shape[-1] == HEAD_DIM
    parts = []
    for j in range(8):
        acc = np.zeros(x.shape[:-1], dtype=F32)
        for c in lane_columns(j):
            acc = (acc + x[..., c] * x[..., c]).astype(F32)
        parts.append(acc)
    p = parts
    return ((p[0] + p[4]) + (p[2] + p[6])) + ((p[1] + p[5]) + (p[3] + p[7]))


def rms_norm(x_bits, weight, eps):
    """bf16 bits [..., 128] -> normalized bf16 values as float32 (step 1-2)."""
    x = bf16_bits_to_f32(np.asarray(x_bits))
    ss = sum_squares(x)
    inv = (F32(1.0) / np.sqrt((ss / F32(HEAD_DIM) + F32(eps)).astype(F32))).astype(F32)
    w = np.asarray(weight, dtype=F32)
    return _bf16((x * inv[..., None]).astype(F32) * w)


def rope_split_half(y, freqs_bits, rows):
    """Partial split-half RoPE of normalized values y [..., M, 128] (float32
    holding bf16 values); freqs_bits [M, R, 2, 2] bf16 bits; ``rows`` the
    token index m of each row of y (y.shape[-2] == M). Returns bf16 bits."""
    y = np.asarray(y, dtype=F32)
    f = bf16_bits_to_f32(np.asarray(freqs_bits)).reshape(rows, -1, 2, 2)
    R = f.shape[1]
    assert 0 <= 2 * R <= HEAD_DIM
    out = y.copy()
    if R:
        y0, y1 = y[..., :R], y[..., R:2 * R]
        # f[m, i, r, 0] multiplies y_i, f[m, i, r, 1] multiplies y_{i+R}
        f00, f01, f10, f11 = f[:, :, 0, 0], f[:, :, 0, 1], f[:, :, 1, 0], f[:, :, 1, 1]
        out[..., :R] = _bf16(_bf16(f00 * y0) + f01 * y1)
        out[..., R:2 * R] = _bf16(_bf16(f11 * y1) + f10 * y0)
    return f32_to_bf16_bits(out)


def qk_rms_rope(x_bits, freqs_bits, weight, eps):
    """One Q or K tensor [1, H, M, 128] (bf16 bits, the projection values)
    -> its normalized, rotated bf16 bits."""
    x = np.asarray(x_bits)
    m = x.shape[-2]
    return rope_split_half(rms_norm(x, weight, eps), freqs_bits, m)


def qkv_rms_rope(q_bits, k_bits, v_bits, freqs_bits, q_weight, k_weight, eps):
    """The reference kernel's outputs from the QKV scatter's (Q, K, V): V is
    stored unchanged (``:714-723``)."""
    return (qk_rms_rope(q_bits, freqs_bits, q_weight, eps),
            qk_rms_rope(k_bits, freqs_bits, k_weight, eps),
            np.asarray(v_bits).copy())
