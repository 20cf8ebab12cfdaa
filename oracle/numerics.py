"""Bit-level number formats (oracle; test infrastructure only).

bf16 and fp16 are carried as uint16 bit patterns, fp8 e4m3fn as uint8 codes,
so every comparison downstream is a bit comparison.
"""
import numpy as np

F32 = np.float32


def f32_to_bf16_bits(x):
    """float32 -> bf16 bits, round-to-nearest-even; NaN -> 0x7FC0 (sign kept
    for the payload-free quiet NaN the way torch's c10::BFloat16 does).

    Restates ``bf16_rte`` (reference ``_patches/int8_ext/int8_gemm.mm:45-53``):
    add 0x7FFF plus the lsb of the kept half, then keep the high 16 bits.
    """
    x = np.ascontiguousarray(x, dtype=F32)
    u = x.view(np.uint32)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    r = ((u + np.uint32(0x7FFF) + lsb) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r = np.where(nan, np.uint16(0x7FC0), r)
    return r


def bf16_bits_to_f32(h):
    h = np.asarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << np.uint32(16)).view(F32)


def bf16_round(x):
    """float32 value of bf16(x) (RNE)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def f32_to_f16_bits(x):
    """float32 -> IEEE half bits, RNE (numpy's astype is RNE); values past the
    half range become +-inf, as in torch."""
    with np.errstate(over="ignore"):
        return np.asarray(x, dtype=F32).astype(np.float16).view(np.uint16)


def f16_bits_to_f32(h):
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(F32)


# --- fp8 e4m3fn (OCP "fn": no inf, NaN = S.1111.111, max 448) -------------

def _e4m3fn_table():
    codes = np.arange(256, dtype=np.uint32)
    s = np.where(codes & 0x80, -1.0, 1.0)
    e = (codes >> 3) & 0xF
    m = (codes & 7).astype(np.float64)
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * 2.0 ** (e.astype(np.float64) - 7.0))
    val = s * val
    val[(codes & 0x7F) == 0x7F] = np.nan
    return val.astype(F32)


E4M3FN_TABLE = _e4m3fn_table()


def e4m3fn_decode(codes):
    """uint8 codes -> float32 (exact). Restates ``fp8_to_float_lut``
    (reference ``_patches/_common.py:203-211``): a 256-entry table of the
    exact values."""
    return E4M3FN_TABLE[np.asarray(codes, dtype=np.uint8)]


def e4m3fn_encode(x):
    """float32 -> e4m3fn code, round-to-nearest-even, NO saturation:
    |x| >= 480 (the first value that rounds past 448) and NaN give NaN
    (0x7F | sign); 464 rounds (tie, even) down to 448.

    This is the cast ``Tensor.to(torch.float8_e4m3fn)`` performs; callers
    clamp to +-448 first, as the reference does before every cast
    (``_patches/comfykitchen_fp8.py:96``).

    Formulated on the magnitude grid: below 2^-6 the grid is uniform with
    step 2^-9 (subnormals), above it each binade [2^e, 2^(e+1)) holds 8
    evenly spaced values.
    """
    x = np.asarray(x, dtype=F32)
    sign = (x.view(np.uint32) >> np.uint32(24)).astype(np.uint8) & np.uint8(0x80)
    a = np.abs(x).astype(np.float64)
    out = np.zeros(x.shape, dtype=np.uint8)
    nan = np.isnan(a) | (a >= 480.0)
    sub = (~nan) & (a < 2.0 ** -6)
    # subnormal grid (q may reach 8 == smallest normal code 0x08: carries naturally)
    q = np.rint(a[sub] * 2.0 ** 9)          # np.rint is half-to-even
    out[sub] = q.astype(np.uint8)
    nrm = (~nan) & (~sub)
    an = a[nrm]
    e = np.floor(np.log2(an)).astype(np.int64)
    # guard log2 rounding at binade edges
    e = np.where(2.0 ** e > an, e - 1, e)
    e = np.where(2.0 ** (e + 1) <= an, e + 1, e)
    mq = np.rint((an / 2.0 ** e - 1.0) * 8.0).astype(np.int64)   # 0..8, exact in f64
    carry = mq == 8
    e = np.where(carry, e + 1, e)
    mq = np.where(carry, 0, mq)
    code = ((e + 7) << 3) | mq
    # (464, 480) rounds to mantissa 7 of the top binade: code 0x7F, the NaN code
    out[nrm] = code.astype(np.uint8)
    out[nan] = 0x7F
    return out | sign
