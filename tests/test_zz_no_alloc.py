"""The allocation-free MLP bridge entry point against the allocating one.

``c4q_i8_mlp_bridge_prequant_noalloc`` stages FC1's rows in the library's
own per-GPU device array; it must give the same q and scales, byte for byte,
as ``c4q_i8_mlp_bridge_prequant`` with caller scratch. Two calls in a row
(the second smaller) check that nothing left in the array by one call leaks
into the next; the wide case (F > 15360, two-pass route, 128-row chunks)
checks the chunking; an F too wide for one 128-row chunk is rejected.
Both entry points are called through the C ABI.
"""
import ctypes

import numpy as np
import pytest
import torch

from _util import gen

import cdna4q.ops as ops
from cdna4q import _lib
from cdna4q._lib import C4QError

pytestmark = pytest.mark.gpu


def _inputs(M, K, F, seed):
    g = gen(seed)
    a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (2 * F, K), generator=g, dtype=torch.int8)
    rs = torch.rand(M, generator=g) * 0.01
    cs = torch.rand(2 * F, generator=g) * 0.002
    b = torch.randn(2 * F, generator=g).to(torch.bfloat16)
    return a, w, rs, cs, b


def _call_noalloc(dev, a, w, rs, cs, b, silu):
    M, K = a.shape
    W = w.shape[0]
    q = torch.empty((M, W // 2), dtype=torch.int8, device=dev)
    s = torch.empty((M, 1), dtype=torch.float32, device=dev)
    _lib.call("c4q_i8_mlp_bridge_prequant_noalloc", a.data_ptr(), K, w.data_ptr(), K,
              rs.data_ptr(), cs.data_ptr(), b.data_ptr(), silu.data_ptr(), M, K, W, q.data_ptr(),
              s.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
    return q, s


def _call_alloc(dev, a, w, rs, cs, b, silu):
    M, K = a.shape
    W = w.shape[0]
    F = W // 2
    wide = torch.empty((M, W), dtype=torch.bfloat16, device=dev)
    rot = torch.empty((M, F), dtype=torch.bfloat16, device=dev)
    q = torch.empty((M, F), dtype=torch.int8, device=dev)
    s = torch.empty((M, 1), dtype=torch.float32, device=dev)
    _lib.call("c4q_i8_mlp_bridge_prequant", a.data_ptr(), K, w.data_ptr(), K, rs.data_ptr(),
              cs.data_ptr(), b.data_ptr(), silu.data_ptr(), M, K, W, M, wide.data_ptr(),
              rot.data_ptr(), q.data_ptr(), s.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
    return q, s


@pytest.mark.parametrize("shapes", [
    ((2048, 1024, 4096), (300, 512, 1024)),       # one-pass route, all rows in one chunk
    ((6000, 256, 16384), (1500, 512, 16384)),     # two-pass route: 640-row chunks (10 of them)
])
def test_noalloc_bridge_matches_allocating_entry_point(dev, shapes):
    silu = ops.act_table("silu", dev)
    for i, (M, K, F) in enumerate(shapes):
        a, w, rs, cs, b = (t.to(dev) for t in _inputs(M, K, F, 71 + i))
        q0, s0 = _call_alloc(dev, a, w, rs, cs, b, silu)
        q1, s1 = _call_noalloc(dev, a, w, rs, cs, b, silu)
        torch.cuda.synchronize()
        assert torch.equal(q1, q0), f"q differs (call {i}, M={M} K={K} F={F})"
        assert torch.equal(s1.view(torch.int32), s0.view(torch.int32)), f"scales differ (call {i})"


def test_noalloc_bridge_ops_wrapper_and_limit(dev):
    a, w, rs, cs, b = (t.to(dev) for t in _inputs(200, 256, 512, 5))
    q0, s0 = ops.i8_mlp_bridge_prequant(a, w, rs, cs, b)
    q1, s1 = ops.i8_mlp_bridge_prequant_noalloc(a, w, rs, cs, b)
    assert torch.equal(q0, q1) and torch.equal(s0.view(torch.int32), s1.view(torch.int32))
    # F = 87552 (> 87381): a 128-row chunk needs more than the 64 MiB array;
    # rejected before anything is enqueued (the weight is never read)
    silu = ops.act_table("silu", dev)
    F = 87552
    with pytest.raises(C4QError, match="scratch"):
        _lib.call("c4q_i8_mlp_bridge_prequant_noalloc", a.data_ptr(), 256, a.data_ptr(), 256,
                  rs.data_ptr(), rs.data_ptr(), None, silu.data_ptr(), 200, 256, 2 * F,
                  a.data_ptr(), rs.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
