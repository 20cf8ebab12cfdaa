"""Routing logic of the patch layer, CPU only: which kernel entry point each
seam picks for which arguments, and when a call keeps the original op.

The device gate (``patches._common.DEVICE_TYPE``) is pointed at "cpu" and the
``ops`` entry points are replaced by recording fakes, the way the
reference's patch tests exercise their routes with fakes
(tests/test_int8_linear_kernel.py, tests/test_scaled_mm_fp8.py,
tests/test_linear_fp8_w8a16.py). The numerics of the routes are covered by
tests/test_gpu_patches.py on the GPU.
"""
import types

import numpy as np
import pytest
import torch

import cdna4q.ops as ops
from cdna4q import _lib
from cdna4q._lib import C4QError
from cdna4q.patches import (_common, int8_linear, int_mm, krea2_ffn_pair, linear_fp8_w8a16,
                            moss_ffn, scaled_mm_fp8)
import cdna4q.patches as patches


class Rec:
    """Recording fake: remembers calls, returns `fn(*args)`."""

    def __init__(self, fn=None):
        self.calls = []
        self.fn = fn

    def __call__(self, *a, **k):
        self.calls.append((a, k))
        return self.fn(*a, **k) if self.fn else None


@pytest.fixture
def cpu_gate(monkeypatch):
    monkeypatch.setattr(_common, "DEVICE_TYPE", "cpu")


def _i8(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-128, 128, shape, generator=g, dtype=torch.int8)


# ---------------------------------------------------------------- int_mm ---

def test_int_mm_routes_int8_and_runs_canary_once(cpu_gate, monkeypatch):
    fake = Rec(lambda a, b: (a.long() @ b.long()).to(torch.int32))
    monkeypatch.setattr(ops, "int_mm", fake)
    monkeypatch.setattr(int_mm, "_canary_ok", False)
    a, b = _i8((4, 64), 1), _i8((64, 8), 2)
    out = int_mm._int_mm_rocm(a, b)
    assert torch.equal(out, (a.long() @ b.long()).to(torch.int32))
    assert len(fake.calls) == 3            # two canary shapes + the call
    int_mm._int_mm_rocm(a, b)
    assert len(fake.calls) == 4            # canary not repeated


def test_int_mm_canary_mismatch_raises(cpu_gate, monkeypatch):
    monkeypatch.setattr(ops, "int_mm", Rec(lambda a, b: (a.long() @ b.long()).to(torch.int32) + 1))
    monkeypatch.setattr(int_mm, "_canary_ok", False)
    with pytest.raises(_lib.C4QError, match="canary"):
        int_mm._int_mm_rocm(_i8((4, 64), 1), _i8((64, 8), 2))


def test_int_mm_keeps_stock_op_for_other_inputs(cpu_gate, monkeypatch):
    orig = Rec(lambda a, b: "stock")
    monkeypatch.setattr(int_mm, "_orig", orig)
    monkeypatch.setattr(ops, "int_mm", Rec())
    assert int_mm._int_mm_rocm(torch.ones(2, 3), torch.ones(3, 4)) == "stock"          # float
    assert int_mm._int_mm_rocm(_i8((2, 3, 4), 1), _i8((4, 5), 2)) == "stock"           # 3-D
    assert ops.int_mm.calls == []


def test_int_mm_off_device_keeps_stock_op(monkeypatch):
    orig = Rec(lambda a, b: "stock")
    monkeypatch.setattr(int_mm, "_orig", orig)
    assert int_mm._int_mm_rocm(_i8((2, 4), 1), _i8((4, 3), 2)) == "stock"              # CPU tensors


# ----------------------------------------------------------- int8_linear ---

def _fake_int8_ops(monkeypatch):
    rec = {}
    def quant(x):
        rec.setdefault("quant", 0)
        rec["quant"] += 1
        m = x.shape[0]
        return torch.zeros(x.shape, dtype=torch.int8), torch.full((m, 1), 0.5)
    monkeypatch.setattr(ops, "i8_quant_rowwise", quant)
    for name in ("i8_matmul2d_nt_fused", "i8_matmul2d_nt_fused_cs"):
        def f(q, w, *a, _n=name):
            rec.setdefault(_n, []).append(a)
            return torch.zeros(q.shape[0], w.shape[0], dtype=torch.bfloat16)
        monkeypatch.setattr(ops, name, f)
    def raw(q, w):
        rec.setdefault("raw", 0)
        rec["raw"] += 1
        return (q.long() @ w.long().t()).to(torch.int32) + 7
    monkeypatch.setattr(ops, "i8_matmul2d_nt", raw)
    monkeypatch.setattr(int8_linear, "_act_cache", None)
    return rec


def test_int8_linear_dispatch_by_scale_layout(cpu_gate, monkeypatch):
    rec = _fake_int8_ops(monkeypatch)
    x = torch.randn(2, 5, 16).to(torch.bfloat16)
    w = _i8((12, 16), 3)
    out = int8_linear.int8_linear(x, w, torch.tensor([0.25]), None, torch.bfloat16)
    assert out.shape == (2, 5, 12) and len(rec["i8_matmul2d_nt_fused"]) == 1
    row_scale = rec["i8_matmul2d_nt_fused"][0][0]
    assert torch.equal(row_scale, torch.full((10,), 0.125))          # w_scale * x_scale
    out = int8_linear.int8_linear(x, w, torch.rand(12), None, torch.bfloat16)
    assert len(rec["i8_matmul2d_nt_fused_cs"]) == 1
    assert rec["quant"] == 1                                         # same x: quantized once


def test_int8_linear_eager_rescale_for_other_dtypes(cpu_gate, monkeypatch):
    rec = _fake_int8_ops(monkeypatch)
    x = torch.randn(6, 16).to(torch.bfloat16)
    w = _i8((12, 16), 3)
    ws = torch.rand(12)
    bias = torch.randn(12).to(torch.float16)
    out = int8_linear.int8_linear(x, w, ws, bias, torch.float16)
    c = torch.full((6, 12), 7, dtype=torch.int32)                    # fake product of zero q
    ref = (c.float() * (ws * torch.full((6, 1), 0.5))).to(torch.float16) + bias
    assert rec["raw"] == 1 and out.dtype == torch.float16 and torch.equal(out, ref)


def test_int8_linear_activation_cache(cpu_gate, monkeypatch):
    rec = _fake_int8_ops(monkeypatch)
    w = _i8((12, 16), 3)
    x1 = torch.randn(4, 16).to(torch.bfloat16)
    x2 = x1.clone()
    for x in (x1, x1, x2, x2, x1):
        int8_linear.int8_linear(x, w, torch.tensor([1.0]), None, torch.bfloat16)
    assert rec["quant"] == 3                                         # x1, x2, x1 again
    monkeypatch.setenv("C4Q_INT8_ACT_CACHE", "0")
    monkeypatch.setattr(int8_linear, "_act_cache", None)
    int8_linear.int8_linear(x1, w, torch.tensor([1.0]), None, torch.bfloat16)
    int8_linear.int8_linear(x1, w, torch.tensor([1.0]), None, torch.bfloat16)
    assert rec["quant"] == 5


def test_int8_linear_unsupported_calls(cpu_gate, monkeypatch):
    _fake_int8_ops(monkeypatch)
    x = torch.randn(4, 16).to(torch.bfloat16)
    monkeypatch.setattr(int8_linear, "_orig_int8_linear", None)
    with pytest.raises(_lib.C4QError):
        int8_linear.int8_linear(x, _i8((8, 16), 1), torch.tensor([1.0]), None, torch.bfloat16,
                                True, 256)                           # convrot, K % 256
    orig = Rec(lambda *a: "kitchen")
    monkeypatch.setattr(int8_linear, "_orig_int8_linear", orig)
    assert int8_linear.int8_linear(x, _i8((8, 16), 1), torch.tensor([1.0]), None,
                                   torch.bfloat16, True, 256) == "kitchen"
    assert int8_linear.int8_linear(x, torch.randn(8, 16), torch.tensor([1.0])) == "kitchen"


def test_int8_linear_convrot_routes(cpu_gate, monkeypatch):
    """ConvRot activations go through the fused rotate + quant pass, x viewed
    as [M, K/256, 1, 256]; other group sizes, dtypes and widths keep the
    original function."""
    rec = _fake_int8_ops(monkeypatch)
    seen = []

    def mrq(xv):
        seen.append(tuple(xv.shape))
        return torch.zeros(xv.shape[0], xv.shape[1] * xv.shape[3], dtype=torch.int8), \
            torch.ones(xv.shape[0], 1)
    monkeypatch.setattr(ops, "i8_merge_rot_quant", mrq)
    orig = Rec(lambda *a: "kitchen")
    monkeypatch.setattr(int8_linear, "_orig_int8_linear", orig)
    x = torch.randn(2, 3, 512).to(torch.bfloat16)
    w = _i8((8, 512), 1)
    out = int8_linear.int8_linear(x, w, torch.rand(8), None, torch.bfloat16, True, 256)
    assert out.shape == (2, 3, 8) and seen == [(6, 2, 1, 256)] and "quant" not in rec
    assert int8_linear.int8_linear(x, w, torch.rand(8), None, torch.bfloat16, True, 128) == "kitchen"
    assert int8_linear.int8_linear(x.half(), w, torch.rand(8), None, torch.float16, True,
                                   256) == "kitchen"
    xw = torch.randn(2, 16384).to(torch.bfloat16)
    assert int8_linear.int8_linear(xw, _i8((8, 16384), 1), torch.rand(8), None, torch.bfloat16,
                                   True, 256) == "kitchen"           # K > 15360


class FakeQT:
    """Stand-in for comfy_kitchen's QuantizedTensor in TensorWiseINT8Layout."""
    _layout_cls = "TensorWiseINT8Layout"

    def __init__(self, q, scale, convrot=False, transposed=False):
        self._qdata = q
        self._params = types.SimpleNamespace(scale=scale, convrot=convrot, transposed=transposed)


def _layer(w, bias=None, **kw):
    return types.SimpleNamespace(weight=w, bias=bias, weight_function=[], bias_function=[], **kw)


def test_try_int8_kernel_forward_eligibility(cpu_gate, monkeypatch):
    fake = Rec(lambda *a: "kernel")
    monkeypatch.setattr(int8_linear, "_int8_linear_kernel", fake)
    x = torch.randn(3, 16).to(torch.bfloat16)
    q = _i8((8, 16), 1)
    f = int8_linear._try_int8_kernel_forward
    assert f(_layer(FakeQT(q, torch.tensor([0.1]))), x) == "kernel"
    assert f(_layer(FakeQT(q, torch.tensor([0.1]), convrot=True)), x) is None   # K % 256
    q2 = _i8((8, 256), 1)
    x2 = torch.randn(3, 256).to(torch.bfloat16)
    assert f(_layer(FakeQT(q2, torch.tensor([0.1]), convrot=True)), x2) == "kernel"
    assert fake.calls[-1][0][-2:] == (True, 256)
    assert f(_layer(FakeQT(q, torch.tensor([0.1]), transposed=True)), x) is None
    assert f(_layer(q), x) is None                                   # plain int8 weight
    assert f(_layer(FakeQT(q, torch.tensor([0.1])), _full_precision_mm=True), x) is None
    assert f(_layer(FakeQT(q, torch.tensor([0.1])), comfy_force_cast_weights=True), x) is None
    lora = _layer(FakeQT(q, torch.tensor([0.1])))
    lora.weight_function = [lambda w: w]
    assert f(lora, x) is None
    assert f(_layer(FakeQT(q, torch.tensor([0.1]))), x.float()) is None
    assert len(fake.calls) == 2


def test_o_proj_prequant_gate(cpu_gate, monkeypatch):
    calls = {}
    monkeypatch.setattr(ops, "i8_merge_rot_quant",
                        lambda x: calls.setdefault("mrq", (torch.zeros(x.shape[0] * x.shape[2], x.shape[1] * x.shape[3], dtype=torch.int8),
                                                           torch.ones(x.shape[0] * x.shape[2], 1))))
    monkeypatch.setattr(int8_linear, "_int8_linear_prequant",
                        lambda x_8, x_scale, w, ws, b, dt, shape, split_tail=False: ("gemm", shape))
    x = torch.zeros(1, 4, 5, 128, dtype=torch.bfloat16)
    q = _i8((16, 512), 1)
    f = int8_linear.int8_o_proj_prequant
    assert f(_layer(FakeQT(q, torch.rand(16), convrot=True)), x) == ("gemm", (1, 5, 512))
    assert f(_layer(FakeQT(q, torch.rand(16))), x) is None                 # not ConvRot
    assert f(_layer(FakeQT(q, torch.rand(16), convrot=True)), x.float()) is None
    assert f(_layer(FakeQT(_i8((16, 384), 1), torch.rand(16), convrot=True)),
             torch.zeros(1, 3, 5, 128, dtype=torch.bfloat16)) is None     # 384 % 256
    assert f(_layer(FakeQT(q, torch.rand(16), convrot=True, transposed=True)), x) is None
    monkeypatch.setenv("C4Q_INT8_OPROJ_FUSE", "0")
    assert f(_layer(FakeQT(q, torch.rand(16), convrot=True)), x) is None


def test_qkv_prequant_gate(cpu_gate, monkeypatch):
    seen = []
    monkeypatch.setattr(int8_linear, "_quant_cached",
                        lambda x, *a: (torch.zeros(x.shape, dtype=torch.int8), torch.ones(x.shape[0], 1)))
    monkeypatch.setattr(ops, "i8_matmul2d_nt_fused_cs_qkv",
                        lambda *a: seen.append(("scatter", a[-2:])) or "qkv")
    monkeypatch.setattr(ops, "i8_matmul2d_nt_fused_cs_qkv_rms_rope",
                        lambda *a: seen.append(("rope", a[-3:])) or "qkv-rope")
    H, D, K = 2, 128, 64
    x = torch.zeros(70, K, dtype=torch.bfloat16)
    q = _i8((3 * H * D, K), 1)
    layer = _layer(FakeQT(q, torch.rand(3 * H * D)))
    fr = torch.zeros(70, 48, 2, 2, dtype=torch.bfloat16)
    w = torch.ones(D)
    assert int8_linear.int8_qkv_prequant(layer, x, H, D) == "qkv"
    assert int8_linear.int8_qkv_rms_rope_prequant(layer, x, fr, w, w, H, D, 1e-6) == "qkv-rope"
    assert seen == [("scatter", (H, D)), ("rope", (H, D, 1e-6))]
    f = int8_linear.int8_qkv_prequant
    assert f(layer, x.float(), H, D) is None                                   # not bf16
    assert f(layer, x.unsqueeze(0), H, D) is None                              # not 2-D
    assert f(layer, x, 3, D) is None                                           # width != 3HD
    assert f(_layer(FakeQT(q, torch.rand(3 * H * D), convrot=True)), x, H, D) is None
    assert f(_layer(FakeQT(q, torch.rand(7))), x, H, D) is None                 # scale layout
    lora = _layer(FakeQT(q, torch.rand(3 * H * D)))
    lora._asfp8_runtime_lora = object()
    assert f(lora, x, H, D) is None
    monkeypatch.setenv("C4Q_INT8_QKV_NORM_ROPE", "0")
    assert int8_linear.int8_qkv_rms_rope_prequant(layer, x, fr, w, w, H, D, 1e-6) is None
    assert f(layer, x, H, D) == "qkv"
    monkeypatch.setenv("C4Q_INT8_QKV_SCATTER", "0")
    assert f(layer, x, H, D) is None
    # a rejected call (the kernel wrapper raises) falls back
    monkeypatch.delenv("C4Q_INT8_QKV_SCATTER")

    def bad(*a):
        raise C4QError("freqs shape mismatch")
    monkeypatch.setattr(ops, "i8_matmul2d_nt_fused_cs_qkv", bad)
    assert f(layer, x, H, D) is None


def test_mlp_bridge_gate(cpu_gate, monkeypatch):
    seen = []
    monkeypatch.setattr(int8_linear, "_quant_cached",
                        lambda x, *a: (torch.zeros(x.shape, dtype=torch.int8), torch.ones(x.shape[0], 1)))
    monkeypatch.setattr(ops, "i8_mlp_bridge_prequant",
                        lambda x8, w1, rs, cs, b: seen.append(tuple(w1.shape)) or
                        (torch.zeros(x8.shape[0], w1.shape[0] // 2, dtype=torch.int8),
                         torch.ones(x8.shape[0], 1)))
    monkeypatch.setattr(int8_linear, "_int8_linear_prequant",
                        lambda x8, xs, w, ws, b, dt, shape, split_tail=False: ("fc2", shape, split_tail))
    K, F, N2 = 64, 256, 32
    x = torch.zeros(70, K, dtype=torch.bfloat16)
    fc1 = _layer(FakeQT(_i8((2 * F, K), 1), torch.rand(2 * F)))
    fc2 = _layer(FakeQT(_i8((N2, F), 2), torch.rand(N2), convrot=True))
    f = int8_linear.int8_mlp_bridge
    assert f(fc1, fc2, x) == ("fc2", (70, K), True) and seen == [(2 * F, K)]
    assert f(fc1, _layer(FakeQT(_i8((N2, F), 2), torch.rand(N2))), x) is None    # FC2 not ConvRot
    assert f(fc1, fc2, x.float()) is None
    assert f(_layer(FakeQT(_i8((2 * F, K), 1), torch.rand(1))), fc2, x) is None   # per-tensor FC1
    assert f(_layer(FakeQT(_i8((3 * F, K), 1), torch.rand(3 * F))), fc2, x) is None
    lora = _layer(FakeQT(_i8((2 * F, K), 1), torch.rand(2 * F)))
    lora._asfp8_runtime_lora = object()
    assert f(lora, fc2, x) is None
    monkeypatch.setenv("C4Q_INT8_MLP_BRIDGE", "0")
    assert f(fc1, fc2, x) is None


def test_swiglu_forward_routes(cpu_gate, monkeypatch):
    seen = []
    monkeypatch.setattr(ops, "i8_swiglu_rot", lambda x2: seen.append("rot") or torch.zeros(x2.shape[0], x2.shape[1] // 2, dtype=torch.bfloat16))
    monkeypatch.setattr(ops, "i8_quant_rowwise", lambda r: (torch.zeros(r.shape, dtype=torch.int8), torch.ones(r.shape[0], 1)))
    monkeypatch.setattr(int8_linear, "_int8_linear_prequant",
                        lambda x_8, x_scale, w, ws, b, dt, shape, split_tail=False: ("prequant", shape))
    monkeypatch.setattr(int8_linear, "_int8_linear_kernel", lambda act, *a: ("kernel", tuple(act.shape)))
    x = torch.randn(2, 3, 1024).to(torch.bfloat16)
    q = _i8((8, 512), 1)
    f = int8_linear._try_int8_swiglu_forward
    assert f(_layer(FakeQT(q, torch.rand(8), convrot=True)), x) == ("prequant", (2, 3, 512))
    assert seen == ["rot"]
    assert f(_layer(FakeQT(q, torch.rand(8))), x) == ("kernel", (2, 3, 512))
    assert f(_layer(FakeQT(q, torch.rand(8), convrot=True)), x[..., :1000]) is None   # 500 % 256
    assert f(_layer(q), x) is None


def test_int8_fast_seam_uses_w8a8(cpu_gate, monkeypatch):
    rec = _fake_int8_ops(monkeypatch)
    x = torch.randn(40, 16).to(torch.bfloat16)
    w = _i8((8, 16), 1)
    int8_linear.int8_forward_dynamic(x, w, torch.tensor([0.5]), None, torch.bfloat16)
    int8_linear.int8_forward_dynamic_per_row(x, w, torch.rand(8), None, torch.bfloat16)
    assert len(rec["i8_matmul2d_nt_fused"]) == 1 and len(rec["i8_matmul2d_nt_fused_cs"]) == 1


# ---------------------------------------------------------------- W8A16 ---

def _fp8_layer(n=32, k=64, **kw):
    w = torch.nn.Parameter((torch.randn(n, k) * 0.1).to(torch.float8_e4m3fn), requires_grad=False)
    return _layer(w, None, **kw)


def test_w8a16_eligible(cpu_gate, monkeypatch):
    e = linear_fp8_w8a16._eligible
    x = torch.randn(4, 64).to(torch.bfloat16)
    assert e(_fp8_layer(), x)
    assert e(_fp8_layer(), x.half())
    assert not e(_fp8_layer(), x.float())                            # fp32 input
    assert not e(_fp8_layer(), torch.randn(4, 32).to(torch.bfloat16))  # K mismatch
    lora = _fp8_layer()
    lora.bias_function = [lambda b: b]
    assert not e(lora, x)
    assert not e(_fp8_layer(_v=1), x)                                # offloaded weight
    assert e(_fp8_layer(scale_weight=torch.tensor(0.5)), x)          # per-tensor scale
    assert not e(_fp8_layer(scale_weight=torch.rand(32)), x)         # not per-tensor
    nc = _fp8_layer(32, 64)
    nc.weight = torch.nn.Parameter(nc.weight.data.t().contiguous().t(), requires_grad=False)
    assert not e(nc, torch.randn(4, 32).to(torch.bfloat16))          # non-contiguous weight
    monkeypatch.setenv("C4Q_W8A16_MIN_DIM", "128")
    assert not e(_fp8_layer(), x)
    monkeypatch.setenv("C4Q_W8A16_MIN_DIM", "0")
    monkeypatch.setenv("C4Q_W8A16_M_MAX", "2")
    assert not e(_fp8_layer(), x)


def test_w8a16_patched_forward_routes(cpu_gate, monkeypatch):
    orig = Rec(lambda self, x: "decode")
    monkeypatch.setattr(linear_fp8_w8a16, "_orig_forward", orig)
    fwd = Rec(lambda m, x: "kernel")
    monkeypatch.setattr(linear_fp8_w8a16, "_w8a16_forward", fwd)
    x = torch.randn(4, 64).to(torch.bfloat16)
    assert linear_fp8_w8a16._patched_forward(_fp8_layer(), x) == "kernel"
    assert linear_fp8_w8a16._patched_forward(_fp8_layer(), x.float()) == "decode"


# ------------------------------------------------------------- scaled_mm ---

def test_scaled_mm_fast_eligible(cpu_gate, monkeypatch):
    a = torch.randn(8, 64).to(torch.float8_e4m3fn)
    b = torch.randn(64, 32).to(torch.float8_e4m3fn)
    e = scaled_mm_fp8._fast_eligible
    assert e(a, b)
    assert not e(a.to(torch.float8_e5m2), b.to(torch.float8_e5m2))
    assert not e(a, torch.randn(32, 32).to(torch.float8_e4m3fn))     # K mismatch
    assert not e(a.reshape(2, 4, 64), b)
    monkeypatch.setenv("C4Q_FP8_MIN_DIM", "8192")
    assert not e(a, b)


def test_scaled_mm_routes(cpu_gate, monkeypatch):
    orig = Rec(lambda *a, **k: "stock")
    monkeypatch.setattr(scaled_mm_fp8, "_original", orig)
    monkeypatch.setattr(scaled_mm_fp8, "_self_checked", True)
    fake = Rec(lambda *a, **k: "kernel")
    monkeypatch.setattr(ops, "scaled_mm", fake)
    a = torch.randn(8, 64).to(torch.float8_e4m3fn)
    b = torch.randn(64, 32).to(torch.float8_e4m3fn)
    s = torch.tensor(0.5)
    assert scaled_mm_fp8._rocm_scaled_mm(a, b, out_dtype=torch.bfloat16, scale_a=s,
                                         scale_b=s, scale_result=s) == "kernel"
    kw = fake.calls[0][1]
    assert kw["out_dtype"] == torch.bfloat16 and kw["scale_result"] is s
    assert scaled_mm_fp8._rocm_scaled_mm(a.float(), b.float(), scale_a=s, scale_b=s) == "stock"


# ----------------------------------------------------------- FFN pairs ---

def test_moss_project_splits_hidden_and_gate_rows(monkeypatch):
    fake = Rec(lambda *a: "pair")
    monkeypatch.setattr(ops, "ffn_pair", fake)
    q = _i8((4, 16), 1)
    w = _i8((12, 16), 2)
    ws = torch.arange(12, dtype=torch.float32)
    th, tg = torch.zeros(65536, dtype=torch.int16), torch.ones(65536, dtype=torch.int16)
    assert moss_ffn.project(q, torch.ones(4, 1), w, ws, (th, tg)) == "pair"
    a = fake.calls[0][0]
    assert torch.equal(a[1], w[:6]) and torch.equal(a[2], w[6:])
    assert torch.equal(a[4], ws[:6]) and torch.equal(a[5], ws[6:])
    assert a[6] is th and a[7] is tg
    with pytest.raises(_lib.C4QError):
        moss_ffn.project(q, torch.ones(4), _i8((7, 16), 3), torch.ones(7), (th, tg))


def test_moss_bf16_project_and_gate(monkeypatch):
    from cdna4q.patches import moss_bf16_ffn_pair as mb
    fake = Rec(lambda *a: "pair")
    monkeypatch.setattr(ops, "moss_bf16_pair", fake)
    x = torch.zeros(1, 8, 16, dtype=torch.bfloat16)
    w = torch.zeros(12, 16, dtype=torch.bfloat16)
    tabs = (torch.zeros(65536, dtype=torch.int16), torch.ones(65536, dtype=torch.int16))
    assert mb.project(x, w, tabs) == "pair"
    a = fake.calls[0][0]
    assert a[0] is x and a[1] is w and a[2] is tabs
    with pytest.raises(_lib.C4QError):
        mb.project(x, torch.zeros(7, 16, dtype=torch.bfloat16), tabs)
    # the reference's gate: [1, 4096..6656, 3072] bf16 activations, [16384, 3072] bf16 weight
    xs = torch.empty(1, 4096, 3072, dtype=torch.bfloat16)
    ws = torch.empty(16384, 3072, dtype=torch.bfloat16)
    assert not mb.eligible(xs, ws)                                  # CPU tensors
    assert not mb.eligible(xs[:, :10], ws)
    assert not mb.eligible(torch.empty(1, 4096, 3072), ws)
    assert mb.install() is False


def test_krea2_candidate_gate(cpu_gate, monkeypatch):
    monkeypatch.setattr(krea2_ffn_pair, "project", Rec(lambda x, g, u: torch.zeros(2, 8)))
    down = Rec(lambda h: "down(pair)")
    q = _i8((8, 16), 1)
    mod = types.SimpleNamespace(gate=_layer(FakeQT(q, torch.rand(8))),
                                up=_layer(FakeQT(q, torch.rand(8))), down=down)
    original = Rec(lambda self, x: "original")
    x = torch.randn(2, 16).to(torch.bfloat16)
    with torch.no_grad():
        assert krea2_ffn_pair.candidate(original, mod, x) == "down(pair)"
        assert krea2_ffn_pair.candidate(original, mod, x.float()) == "original"
        mod.up = _layer(FakeQT(q, torch.rand(8), convrot=True))
        assert krea2_ffn_pair.candidate(original, mod, x) == "original"


# --------------------------------------------------------------- install ---

def test_install_all_without_rocm_changes_nothing():
    before = (torch._int_mm, torch._scaled_mm)
    if torch.cuda.is_available():
        pytest.skip("ROCm device present")
    assert patches.install_all() == []
    assert (torch._int_mm, torch._scaled_mm) == before
