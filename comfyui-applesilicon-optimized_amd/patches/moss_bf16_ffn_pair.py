"""MOSS bf16 FC1 with the fused SiTU epilogue.

Mirrors ``_patches/moss_bf16_ffn_pair.py``: ``project(x, weight, tables)``
(``:36-48``) takes the bf16 activation [..., K], the block's ``ffn_up_gate``
weight [2F, K] bf16 (``weight.chunk(2, dim=0)``: hidden rows [0, F), gate
rows [F, 2F)) and the SiTU tables, and returns
``bf16(T_h[bf16(x@Wh^T)] * T_g[bf16(x@Wg^T)])`` [..., F] with fp32
accumulation (``moss_bf16_ffn_pair.metal:282-304``). The reference's
eligibility (``:63-75``) is kept as ``eligible``.
"""
import torch

from .. import ops
from .._lib import C4QError

TAG = "[cdna4q/moss_bf16_ffn_pair]"
calls = 0


def tables(device):
    """(T_h, T_g) as 65,536-entry bf16 bit tables on `device`."""
    return ops.situ_tables(device)


def eligible(x, weight):
    """The reference's shape and dtype gate: one batch of 4096..6656 tokens
    of width 3072, a contiguous [16384, 3072] bf16 weight, no bias."""
    return (isinstance(x, torch.Tensor) and isinstance(weight, torch.Tensor)
            and x.dtype == torch.bfloat16 and x.ndim == 3 and x.shape[0] == 1
            and 4096 <= x.shape[1] <= 6656 and x.is_contiguous() and x.shape[-1] == 3072
            and weight.dtype == torch.bfloat16 and tuple(weight.shape) == (16384, 3072)
            and weight.is_contiguous() and x.device == weight.device
            and x.device.type == "cuda")


def project(x, weight, tables_=None):
    """[..., K] bf16 x [2F, K] bf16 -> [..., F] bf16 SiTU-activated hidden
    state (the reference's ``project``)."""
    global calls
    if weight.dim() != 2 or weight.shape[0] % 2:
        raise C4QError(f"{TAG} weight must be [2F, K]")
    out = ops.moss_bf16_pair(x, weight, tables_ if tables_ is not None else tables(x.device))
    calls += 1
    return out


def install():
    """The block hook needs ComfyUI's MOSS model and the reference's owner
    module (``moss_fast``); this build exposes ``project`` for that caller
    and installs nothing by itself."""
    return False
