"""Fused gate/up FFN pair (oracle; test infrastructure only).

Each fused kernel must equal the unfused chain byte for byte: two
per-channel fused INT8 GEMMs (bf16 outputs), then the bf16 activation,
then the bf16 product. The bf16 pair's GEMM accumulates in fp32; here its
sums are exact (fp64) and rounded once to fp32.
"""
import numpy as np

from .act import apply_table, silu_table
from .int8 import epilogue_rowcolscale, i8_matmul2d_nt
from .numerics import bf16_bits_to_f32, f32_to_bf16_bits


def krea2_pair(q, w_gate, w_up, row_scale, gate_scale, up_scale):
    """Krea2 SwiGLU pair (reference ``_patches/krea2_ffn_pair.metal:281-304``):

        g   = bf16(f32(Cg) * (gs[n] * rs[m]))
        u   = bf16(f32(Cu) * (us[n] * rs[m]))
        out = bf16(f32(silu_bf16(g)) * f32(u))
    """
    g = epilogue_rowcolscale(i8_matmul2d_nt(q, w_gate), row_scale, gate_scale)
    u = epilogue_rowcolscale(i8_matmul2d_nt(q, w_up), row_scale, up_scale)
    a = apply_table(silu_table(), g)
    return f32_to_bf16_bits(bf16_bits_to_f32(a) * bf16_bits_to_f32(u))


def moss_pair(q, w, row_scale, col_scale, table_h, table_g):
    """MOSS FC1 + SiTU (reference ``_patches/moss_ffn_mps.metal:278-301``,
    ``_patches/moss_ffn_mps.py:70-79``): one [2F,K] weight, hidden rows [0,F),
    gate rows [F,2F):

        h   = bf16(f32(C[:, :F]) * (cs[n] * rs[m]))
        g   = bf16(f32(C[:, F:]) * (cs[F+n] * rs[m]))
        out = bf16(f32(T_h[h]) * f32(T_g[g]))
    """
    w = np.asarray(w)
    f = w.shape[0] // 2
    cs = np.asarray(col_scale)
    h = epilogue_rowcolscale(i8_matmul2d_nt(q, w[:f]), row_scale, cs[:f])
    g = epilogue_rowcolscale(i8_matmul2d_nt(q, w[f:]), row_scale, cs[f:])
    return f32_to_bf16_bits(bf16_bits_to_f32(apply_table(table_h, h)) *
                            bf16_bits_to_f32(apply_table(table_g, g)))


def moss_bf16_pair(x_bits, w_bits, table_h, table_g):
    """MOSS bf16 FC1 + SiTU (reference ``_patches/moss_bf16_ffn_pair.metal:282-304``
    behind ``project()`` ``_patches/moss_bf16_ffn_pair.py:36-48``): one
    [2F, K] bf16 weight split by ``chunk(2, dim=0)`` into hidden rows [0, F)
    and gate rows [F, 2F):

        h   = bf16(f32(x @ W[:F]^T))
        g   = bf16(f32(x @ W[F:]^T))
        out = bf16(f32(T_h[h]) * f32(T_g[g]))
    """
    xf = bf16_bits_to_f32(x_bits).astype(np.float64)
    wf = bf16_bits_to_f32(w_bits).astype(np.float64)
    f = wf.shape[0] // 2
    h = f32_to_bf16_bits((xf @ wf[:f].T).astype(np.float32))
    g = f32_to_bf16_bits((xf @ wf[f:].T).astype(np.float32))
    return f32_to_bf16_bits(bf16_bits_to_f32(apply_table(table_h, h)) *
                            bf16_bits_to_f32(apply_table(table_g, g)))
