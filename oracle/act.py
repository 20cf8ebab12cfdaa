"""bf16 activation functions (oracle; test infrastructure only).

The reference applies its activations to bf16 tensors through torch ops
(the unfused chains its fused epilogues must reproduce), so the oracle takes
the same torch CPU ops over all 65,536 bf16 inputs and keeps them as tables.
A table lookup is then the exact oracle for any bf16 input.
"""
import functools

import numpy as np


def _all_bf16():
    import torch
    return torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)


def _bits(t):
    import torch
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


@functools.lru_cache(maxsize=None)
def silu_table():
    """bf16 SiLU: ``F.silu`` on a bf16 tensor, as in the Krea2 unfused chain
    (reference ``_patches/krea2_ffn_pair.metal:297-300``: act = bf16(v/(1+exp(-v))))."""
    import torch.nn.functional as F
    return _bits(F.silu(_all_bf16()))


@functools.lru_cache(maxsize=None)
def gelu_tanh_table():
    """bf16 GELU (tanh approximation): ``F.gelu(y, approximate='tanh')`` on a
    bf16 tensor, the FLUX MLP activation after the bf16 up-projection."""
    import torch.nn.functional as F
    return _bits(F.gelu(_all_bf16(), approximate="tanh"))


@functools.lru_cache(maxsize=None)
def situ_tables():
    """MOSS SiTU tables over every bf16 value, same op sequence as the
    reference (``_patches/moss_fast.py:97-99``), each op rounding to bf16:
    T_h = 25*tanh(v/25), T_g = 4*tanh(v/4)*sigmoid(v)."""
    import torch
    v = _all_bf16()
    th = 25.0 * torch.tanh(v / 25.0)
    tg = 4.0 * torch.tanh(v / 4.0) * torch.sigmoid(v)
    return _bits(th), _bits(tg)


def apply_table(table, x_bits):
    return table[np.asarray(x_bits, dtype=np.uint16)]
