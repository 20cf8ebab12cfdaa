"""MOSS FC1 with the fused SiTU epilogue.

Mirrors ``_patches/moss_ffn_mps.py`` ``project`` (``:70-79``): one int8
weight [2F, K] holds the hidden rows [0, F) and the gate rows [F, 2F)
(``moss_ffn_mps.metal:241``); the pair kernel stores
``bf16(T_h[h] * T_g[g])`` with ``h = bf16(acc_h * cs[n] * rs)``,
``g = bf16(acc_g * cs[F + n] * rs)`` and the SiTU tables
``T_h = 25 tanh(v/25)``, ``T_g = 4 tanh(v/4) sigmoid(v)`` over every bf16 v
(``moss_fast.py:97-99``).
"""
import torch

from .. import ops
from .._lib import C4QError

TAG = "[cdna4q/moss_ffn]"


def tables(device):
    """(T_h, T_g) as 65,536-entry bf16 bit tables on `device`."""
    return ops.situ_tables(device)


def project(q, scales, weight, weight_scale, tables_=None):
    """Prevalidated [M, K] int8 (per-row scales [M]) x [2F, K] int8 (per-row
    scales [2F]) -> [M, F] bf16 SiTU-activated hidden state."""
    if weight.dim() != 2 or weight.shape[0] % 2:
        raise C4QError(f"{TAG} weight must be [2F, K]")
    f = weight.shape[0] // 2
    th, tg = tables_ if tables_ is not None else tables(q.device)
    ws = weight_scale.reshape(-1).float().contiguous()
    return ops.ffn_pair(q, weight[:f], weight[f:], scales.reshape(-1).float().contiguous(),
                        ws[:f], ws[f:], th, tg)


def install():
    """The MOSS block hook needs ComfyUI's MOSS model and the reference's
    owner module; this build exposes ``project`` for that caller and installs
    nothing by itself."""
    return False
