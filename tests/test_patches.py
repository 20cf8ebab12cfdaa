"""Routing logic of the patch layer, CPU only: which kernel entry point each
seam picks for which arguments, and when a call keeps the original op.

The device gate (``patches._common.DEVICE_TYPE``) is pointed at "cpu" and the
``ops`` entry points are replaced by recording fakes, the way the
reference's patch tests exercise their routes with fakes
(tests/test_int8_linear_kernel.py, tests/test_scaled_mm_fp8.py,
tests/test_linear_fp8_w8a16.py). The numerics of the routes are covered by
tests/test_gpu_patches.py on the GPU.
"""
import sys
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
    for name in ("i8_matmul2d_nt_fused", "i8_matmul2d_nt_fused_cs", "i8_matmul2d_nt_fused_cs_half"):
        def f(q, w, *a, _n=name):
            rec.setdefault(_n, []).append(a)
            dt = torch.float16 if _n.endswith("half") else torch.bfloat16
            return torch.zeros(q.shape[0], w.shape[0], dtype=dt)
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
    """A per-tensor scale with an fp16 (or f32) output takes the raw int32
    GEMM and the reference's eager rescale."""
    rec = _fake_int8_ops(monkeypatch)
    x = torch.randn(6, 16).to(torch.bfloat16)
    w = _i8((12, 16), 3)
    ws = torch.tensor([0.375])
    bias = torch.randn(12).to(torch.float16)
    out = int8_linear.int8_linear(x, w, ws, bias, torch.float16)
    c = torch.full((6, 12), 7, dtype=torch.int32)                    # fake product of zero q
    ref = (c.float() * (ws * torch.full((6, 1), 0.5))).to(torch.float16) + bias
    assert rec["raw"] == 1 and out.dtype == torch.float16 and torch.equal(out, ref)
    out = int8_linear.int8_linear(x, w, torch.rand(12), None, torch.float32)
    assert rec["raw"] == 2 and out.dtype == torch.float32


def test_int8_linear_fp16_per_channel_takes_half_epilogue(cpu_gate, monkeypatch):
    """fp16 output with per-channel scales: the fused half epilogue
    (reference wan_fp16.maybe_prequant), with the x scales as row scales, the
    weight scales as column scales and the bias passed through."""
    rec = _fake_int8_ops(monkeypatch)
    x = torch.randn(2, 3, 16).to(torch.float16)
    w = _i8((12, 16), 3)
    ws = torch.rand(12)
    bias = torch.randn(12).to(torch.float16)
    out = int8_linear.int8_linear(x, w, ws.reshape(12, 1), bias, torch.float16)
    assert out.shape == (2, 3, 12) and out.dtype == torch.float16 and "raw" not in rec
    rs, cs, b = rec["i8_matmul2d_nt_fused_cs_half"][0]
    assert torch.equal(rs, torch.full((6,), 0.5)) and torch.equal(cs, ws) and b is bias


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

    def __init__(self, q, scale, convrot=False, transposed=False, convrot_groupsize=256):
        self._qdata = q
        self._params = types.SimpleNamespace(scale=scale, convrot=convrot, transposed=transposed,
                                             convrot_groupsize=convrot_groupsize)


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


# ------------------------------------------- comfy.ops factory and helper ---

def _fake_comfy_ops():
    """A stand-in ``comfy.ops`` module: ``mixed_precision_ops(quant_config=None,
    compute_dtype=None, full_precision_mm=False, disabled=[])`` returning an
    ops class with a Linear, and the three-argument ``linear_input_act``."""
    seen = {}

    def mixed_precision_ops(quant_config={}, compute_dtype=torch.bfloat16,
                            full_precision_mm=False, disabled=[]):
        seen["disabled"] = list(disabled)
        seen["full_precision_mm"] = full_precision_mm

        class Linear(torch.nn.Module):
            def forward(self, input, *args, **kwargs):
                return "comfy forward"
        return types.SimpleNamespace(Linear=Linear)

    def linear_input_act(linear, x, input_act, *args, **kwargs):
        seen.setdefault("lia", []).append((input_act, args, kwargs))
        return "comfy lia"
    return types.SimpleNamespace(mixed_precision_ops=mixed_precision_ops,
                                 linear_input_act=linear_input_act), seen


def test_factory_wrap_keeps_int8_enabled_and_patches_linear(cpu_gate, monkeypatch):
    """``disabled`` loses "int8_tensorwise" only (reference
    _patches/int8_linear_kernel_mps.py:869-878); the generated Linear tries the
    kernel route first."""
    mod, seen = _fake_comfy_ops()
    int8_linear._patch_comfy_ops(mod)
    int8_linear._patch_comfy_ops(mod)                                 # idempotent
    assert mod.mixed_precision_ops._c4q_wrapped and mod.linear_input_act._c4q_wrapped
    cls = mod.mixed_precision_ops({}, torch.bfloat16, True, ["int8_tensorwise", "float8_e4m3fn"])
    assert seen["disabled"] == ["float8_e4m3fn"] and seen["full_precision_mm"] is True
    mod.mixed_precision_ops(disabled=("int8_tensorwise",))
    assert seen["disabled"] == []
    mod.mixed_precision_ops()                                         # no disabled list given
    assert seen["disabled"] == []
    lin = cls.Linear()
    monkeypatch.setattr(int8_linear, "_try_int8_kernel_forward",
                        lambda self, x: "kernel" if x.dtype == torch.bfloat16 else None)
    assert lin(torch.zeros(2, dtype=torch.bfloat16)) == "kernel"
    assert lin(torch.zeros(2)) == "comfy forward"


def test_try_int8_kernel_forward_falls_back_on_kernel_rejection(cpu_gate, monkeypatch):
    def reject(*a):
        raise C4QError("M must be positive")
    monkeypatch.setattr(int8_linear, "_int8_linear_kernel", reject)
    layer = _layer(FakeQT(_i8((8, 16), 1), torch.tensor([0.1])))
    assert int8_linear._try_int8_kernel_forward(layer, torch.randn(3, 16).to(torch.bfloat16)) is None


def test_linear_input_act_wrap_routes(cpu_gate, monkeypatch):
    """SwiGLU down-projections take the INT8 SwiGLU route; extended calls,
    other activations and declined calls keep comfy's helper; a plain
    ``input_act=None`` call on a module runs the module; a declined SwiGLU on
    a layer with a runtime adapter runs ``linear(swiglu(x))`` (reference
    _patches/int8_linear_kernel_mps.py:897-977)."""
    mod, seen = _fake_comfy_ops()
    int8_linear._patch_comfy_ops(mod)
    lia = mod.linear_input_act
    route = Rec(lambda linear, x: "int8 swiglu" if x.shape[-1] == 8 else None)
    monkeypatch.setattr(int8_linear, "_try_int8_swiglu_forward", route)
    lin = types.SimpleNamespace()
    x = torch.randn(3, 8).to(torch.bfloat16)
    assert lia(lin, x, "swiglu") == "int8 swiglu"
    assert lia(lin, x, "swiglu", torch.ones(4), eps=1e-6) == "comfy lia"    # extended call
    act, args, kwargs = seen["lia"][-1]
    assert act == "swiglu" and torch.equal(args[0], torch.ones(4)) and kwargs == {"eps": 1e-6}
    assert lia(lin, torch.randn(3, 6).to(torch.bfloat16), "swiglu") == "comfy lia"   # declined
    assert lia(lin, x, "gelu") == "comfy lia"
    monkeypatch.setenv("C4Q_INT8_SWIGLU", "0")
    assert lia(lin, x, "swiglu") == "comfy lia"
    monkeypatch.delenv("C4Q_INT8_SWIGLU")
    module = Rec(lambda x: "module call")
    m = torch.nn.Module()
    m.forward = module
    assert lia(m, x, None) == "module call"
    monkeypatch.setenv("ASFP8_INT8_PLAIN_LIA", "0")
    assert lia(m, x, None) == "comfy lia"
    adapted = Rec(lambda act: ("linear", tuple(act.shape)))
    adapted._asfp8_runtime_lora = object()
    y = torch.randn(3, 6).to(torch.bfloat16)
    assert lia(adapted, y, "swiglu") == ("linear", (3, 3))
    assert len(route.calls) == 3          # never for gelu, nor when switched off


def test_swiglu_forward_declines_runtime_lora_and_kernel_errors(cpu_gate, monkeypatch):
    q = _i8((8, 512), 1)
    x = torch.randn(2, 1024).to(torch.bfloat16)
    adapted = _layer(FakeQT(q, torch.rand(8), convrot=True), _asfp8_runtime_lora=object())
    assert int8_linear._try_int8_swiglu_forward(adapted, x) is None

    def reject(x2):
        raise C4QError("x must be contiguous [M,2F]")
    monkeypatch.setattr(ops, "i8_swiglu_rot", reject)
    assert int8_linear._try_int8_swiglu_forward(_layer(FakeQT(q, torch.rand(8), convrot=True)),
                                                x) is None


# -------------------------------------------------------- int8-fast hook ---

def _int8_quant_module(name="int8_quant"):
    m = types.ModuleType(name)
    m.int8_forward_dynamic = Rec(lambda *a: "int8-fast dyn")
    m.int8_forward_dynamic_per_row = Rec(lambda *a: "int8-fast dyn_pr")
    return m


@pytest.fixture
def fresh_int8_fast(monkeypatch):
    from cdna4q.patches import int8_fast
    for name in ("_installed", "_patched", "_orig_dyn", "_orig_dyn_pr", "_finder"):
        monkeypatch.setattr(int8_fast, name, None if name.startswith("_o") or name == "_finder"
                            else False)
    return int8_fast


def test_int8_fast_patches_a_loaded_module(cpu_gate, monkeypatch, fresh_int8_fast):
    """int8-fast imported first: the scan of sys.modules patches it (reference
    _patches/int8_linear_mps.py:84-94); served calls take the W8A8 route,
    the rest int8-fast's own forwards."""
    f8 = fresh_int8_fast
    mod = _int8_quant_module("custom_nodes.int8_fast.int8_quant")
    monkeypatch.setitem(sys.modules, mod.__name__, mod)
    orig_dyn = mod.int8_forward_dynamic
    assert f8._scan_loaded()
    assert mod.int8_forward_dynamic is f8._dyn and mod.int8_forward_dynamic_per_row is f8._dyn_pr
    w8a8 = Rec(lambda *a: "w8a8")
    monkeypatch.setattr(int8_linear, "int8_forward_dynamic", w8a8)
    monkeypatch.setattr(int8_linear, "int8_forward_dynamic_per_row", w8a8)
    x = torch.randn(40, 16).to(torch.bfloat16)
    w = _i8((8, 16), 1)
    assert mod.int8_forward_dynamic(x, w, torch.tensor(0.5), None, torch.bfloat16) == "w8a8"
    assert mod.int8_forward_dynamic_per_row(x, w, torch.rand(8, 1), None, torch.bfloat16) == "w8a8"
    assert mod.int8_forward_dynamic(x.float(), w, torch.tensor(0.5), None, torch.float32) \
        == "int8-fast dyn"
    assert mod.int8_forward_dynamic(x, w.float(), torch.tensor(0.5), None, torch.bfloat16) \
        == "int8-fast dyn"
    assert len(orig_dyn.calls) == 2 and len(w8a8.calls) == 2
    other = _int8_quant_module()
    f8._apply(other)                                                  # patched once only
    assert other.int8_forward_dynamic is not f8._dyn


def test_int8_fast_finder_patches_a_later_import(cpu_gate, monkeypatch, tmp_path,
                                                fresh_int8_fast):
    """int8-fast imported after this package: the meta-path finder wraps the
    module's loader and patches it right after it executes (reference
    _patches/int8_linear_mps.py:97-128)."""
    f8 = fresh_int8_fast
    pkg = tmp_path / "c4q_fake_int8fast"
    pkg.mkdir()
    (pkg / "__init__.py").write_text("")
    (pkg / "int8_quant.py").write_text(
        "def int8_forward_dynamic(x, w, s, b, dt):\n    return 'dyn'\n"
        "def int8_forward_dynamic_per_row(x, w, s, b, dt):\n    return 'dyn_pr'\n")
    monkeypatch.syspath_prepend(str(tmp_path))
    assert not f8._scan_loaded()
    finder = f8._Finder()
    monkeypatch.setattr(sys, "meta_path", [finder] + sys.meta_path)
    import importlib
    mod = importlib.import_module("c4q_fake_int8fast.int8_quant")
    try:
        assert mod.int8_forward_dynamic is f8._dyn and f8._patched
        assert mod.int8_forward_dynamic(torch.randn(2, 4), _i8((3, 4), 1), None, None,
                                        torch.float32) == "dyn"          # CPU float: original
        assert finder.find_spec("c4q_fake_int8fast.other", None) is None
    finally:
        sys.modules.pop("c4q_fake_int8fast.int8_quant", None)
        sys.modules.pop("c4q_fake_int8fast", None)


def test_int8_fast_install_needs_rocm(fresh_int8_fast):
    if torch.cuda.is_available():
        pytest.skip("ROCm device present")
    assert fresh_int8_fast.install() is False


# ------------------------------------------------------ fp8_ext surface ---

def test_fp8_ext_functions_route_to_w8a16(monkeypatch):
    """fp8_matmul2d_nt(a, W[N,K]) and fp8_matmul2d(a, W[K,N]) are the W8A16
    route with f32 output; the [K,N] form hands over the [N,K] transpose
    (reference _patches/fp8_ext/fp8_matmul2d.mm:268-353)."""
    rec = Rec(lambda x, w, out_dtype=None: ("w8a16", tuple(w.shape), out_dtype))
    monkeypatch.setattr(ops, "w8a16_linear", rec)
    a = torch.randn(4, 64).to(torch.float16)
    w = (torch.randn(32, 64) * 0.1).to(torch.float8_e4m3fn)
    assert ops.fp8_matmul2d_nt(a, w.view(torch.uint8), 32) == ("w8a16", (32, 64), torch.float32)
    assert ops.fp8_matmul2d(a, w.t().contiguous().view(torch.uint8), 32) == \
        ("w8a16", (32, 64), torch.float32)
    wt = rec.calls[-1][0][1]
    assert wt.is_contiguous() and torch.equal(wt, w.view(torch.uint8))
    with pytest.raises(C4QError):
        ops.fp8_matmul2d_nt(a, w.view(torch.uint8), 31)
    with pytest.raises(C4QError):
        ops.fp8_matmul2d(a, w.view(torch.uint8), 64)                 # [N,K] given as [K,N]
    assert ops.num_variants() == 4


def test_loader_surface_names():
    """Every function the reference's three native modules export exists in
    ops under the same name."""
    names = ["i8_mlp_bridge_prequant", "i8_swiglu_rot", "i8_merge_rot_quant",
             "i8_matmul2d_nt_fused_cs", "i8_matmul2d_nt_fused_cs_half",
             "i8_matmul2d_nt_fused_cs_qkv", "i8_matmul2d_nt_fused_cs_qkv_rms_rope",
             "i8_matmul2d_nt_fused_cs_qkv_lora_part",
             "i8_quant_rowwise", "i8_matmul2d_nt", "i8_matmul2d_nt_fused", "warmup",
             "fp8_matmul2d", "fp8_matmul2d_nt", "fp8fp8_matmul2d_nt",
             "w8a16_f32", "w8a16_bias_bf16", "num_variants"]
    assert [n for n in names if not callable(getattr(ops, n, None))] == []


def test_activation_tables_are_the_pinned_cpu_tables():
    """The tables the fused epilogues use are built from torch's CPU ops (the
    ones tests/golden/digests.json pins), copied per device."""
    import hashlib
    import json
    import pathlib
    d = json.loads((pathlib.Path(__file__).parent / "golden" / "digests.json").read_text())

    def sha(t):
        return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()
    assert sha(ops.act_table("silu", "cpu")) == d["silu_sha256"]
    assert sha(ops.act_table("gelu_tanh", "cpu")) == d["gelu_tanh_sha256"]
    th, tg = ops.situ_tables("cpu")
    assert (sha(th), sha(tg)) == (d["situ_h_sha256"], d["situ_g_sha256"])
    with pytest.raises(C4QError):
        ops.act_table("relu", "cpu")


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


def test_scaled_mm_eligibility_covers_every_epilogue_argument(cpu_gate):
    """Only calls the fp8 kernel's epilogue can serve take the fast route:
    out dtype bf16/f16/f32, f32 scales per tensor / row / column, per-tensor
    scale_result, an N-element bias. fp8 or unset outputs, blockwise and MX
    scales keep the stock op."""
    a = torch.randn(8, 64).to(torch.float8_e4m3fn)
    b = torch.randn(64, 32).to(torch.float8_e4m3fn)
    e = scaled_mm_fp8._fast_eligible
    one = torch.tensor(0.5)
    for dt in (torch.bfloat16, torch.float16, torch.float32):
        assert e(a, b, dt, one, one)
    assert not e(a, b, None, one, one)                              # stock: fp8 output
    assert not e(a, b, torch.float8_e4m3fn, one, one)
    assert e(a, b, torch.bfloat16, torch.rand(8, 1), torch.rand(1, 32))    # row / column
    assert e(a, b, torch.bfloat16, torch.rand(8), torch.rand(32))
    assert not e(a, b, torch.bfloat16, torch.rand(1, 8), one)       # row scale laid out as a row
    assert not e(a, b, torch.bfloat16, torch.rand(8, 2), one)       # blockwise [M, K/32]
    assert not e(a, b, torch.bfloat16, one, torch.rand(2, 32))      # blockwise over K
    assert not e(a, b, torch.bfloat16, torch.rand(8, 1).half(), one)   # non-f32 scale
    if hasattr(torch, "float8_e8m0fnu"):
        mx = torch.ones(8, 2).to(torch.float8_e8m0fnu)
        assert not e(a, b, torch.bfloat16, mx, one)                 # MX block scales
    assert e(a, b, torch.bfloat16, one, one, one)
    assert not e(a, b, torch.bfloat16, one, one, torch.rand(32))    # scale_result vector
    assert e(a, b, torch.bfloat16, one, one, None, torch.randn(32).half())
    assert not e(a, b, torch.bfloat16, one, one, None, torch.randn(31))
    assert not e(a, b, torch.bfloat16, one, one, None, torch.randn(1, 32))
    assert not e(a, b, torch.bfloat16, one, one, None, torch.randn(32).to(torch.float64))


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
    # out_dtype=None: the stock op's fp8-output semantics, not the kernel's f32
    assert scaled_mm_fp8._rocm_scaled_mm(a, b, scale_a=s, scale_b=s) == "stock"
    assert scaled_mm_fp8._rocm_scaled_mm(a, b, out_dtype=torch.bfloat16, scale_a=torch.rand(8, 2),
                                         scale_b=s) == "stock"
    assert len(fake.calls) == 1
    stock_kw = orig.calls[-1][1]
    assert stock_kw["scale_a"].shape == (8, 2) and stock_kw["use_fast_accum"] is False


def test_scaled_mm_kernel_rejection_falls_back_to_stock(cpu_gate, monkeypatch):
    orig = Rec(lambda *a, **k: "stock")
    monkeypatch.setattr(scaled_mm_fp8, "_original", orig)
    monkeypatch.setattr(scaled_mm_fp8, "_self_checked", True)

    def reject(*a, **k):
        raise C4QError("unsupported layout")
    monkeypatch.setattr(ops, "scaled_mm", reject)
    a = torch.randn(8, 64).to(torch.float8_e4m3fn)
    b = torch.randn(64, 32).to(torch.float8_e4m3fn)
    s = torch.tensor(0.5)
    assert scaled_mm_fp8._rocm_scaled_mm(a, b, out_dtype=torch.bfloat16, scale_a=s,
                                         scale_b=s, use_fast_accum=True) == "stock"
    assert orig.calls[0][1]["use_fast_accum"] is True


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
    """The pair serves ConvRot group-256 INT8 layers only (reference
    _patches/moss_ffn_mps.py:52-53); anything else keeps the SwiGLU forward."""
    monkeypatch.setattr(krea2_ffn_pair, "project", Rec(lambda x, g, u: torch.zeros(2, 8)))
    down = Rec(lambda h: "down(pair)")
    K = 256
    q = _i8((8, K), 1)

    def mod(**kw):
        return types.SimpleNamespace(gate=_layer(FakeQT(q, torch.rand(8), convrot=True), **kw),
                                     up=_layer(FakeQT(q, torch.rand(8), convrot=True)), down=down)
    original = Rec(lambda self, x: "original")
    x = torch.randn(2, K).to(torch.bfloat16)
    with torch.no_grad():
        assert krea2_ffn_pair.candidate(original, mod(), x) == "down(pair)"
        assert krea2_ffn_pair.candidate(original, mod(), x.float()) == "original"
        plain = mod()
        plain.up = _layer(FakeQT(q, torch.rand(8)))                  # not ConvRot
        assert krea2_ffn_pair.candidate(original, plain, x) == "original"
        g128 = mod()
        g128.gate.weight._params.convrot_groupsize = 128
        assert krea2_ffn_pair.candidate(original, g128, x) == "original"
        assert krea2_ffn_pair.candidate(original, mod(bias=torch.zeros(8)), x) == "original"
        assert krea2_ffn_pair.candidate(original, mod(_asfp8_runtime_lora=object()), x) == "original"
        assert krea2_ffn_pair.candidate(original, mod(weight_lowvram_function=[1]), x) == "original"
        assert krea2_ffn_pair.candidate(original, mod(), torch.randn(2, 200).to(torch.bfloat16)) \
            == "original"                                           # K % 256
        pt = mod()
        pt.gate.weight._params.scale = torch.rand(1)                # per-tensor scale
        assert krea2_ffn_pair.candidate(original, pt, x) == "original"
    assert krea2_ffn_pair.candidate(original, mod(), x) == "original"  # grad enabled
    assert len(krea2_ffn_pair.project.calls) == 1


def test_krea2_project_rotates_then_quantizes(cpu_gate, monkeypatch):
    """project = fused ConvRot + rowwise quant of x (group 256), then the
    pair kernel with the SiLU table on the gate (reference
    _patches/krea2_ffn_pair.py:37-49)."""
    seen = {}

    def mrq(xv):
        seen["mrq"] = tuple(xv.shape)
        return torch.zeros(xv.shape[0], xv.shape[1] * xv.shape[3], dtype=torch.int8), \
            torch.full((xv.shape[0], 1), 0.25)
    monkeypatch.setattr(ops, "i8_merge_rot_quant", mrq)
    monkeypatch.setattr(ops, "i8_quant_rowwise", Rec())
    monkeypatch.setattr(ops, "act_table", lambda name, dev: ("table", name))
    pair = Rec(lambda *a: torch.zeros(a[0].shape[0], a[1].shape[0], dtype=torch.bfloat16))
    monkeypatch.setattr(ops, "ffn_pair", pair)
    monkeypatch.setattr(int8_linear, "_act_cache", None)
    q = _i8((8, 512), 1)
    g, u = FakeQT(q, torch.rand(8), convrot=True), FakeQT(q, torch.rand(8), convrot=True)
    x = torch.randn(1, 3, 512).to(torch.bfloat16)
    out = krea2_ffn_pair.project(x, g, u)
    assert out.shape == (1, 3, 8)
    assert seen["mrq"] == (3, 2, 1, 256) and ops.i8_quant_rowwise.calls == []
    a = pair.calls[0][0]
    assert torch.equal(a[3], torch.full((3,), 0.25)) and a[6] == ("table", "silu") and a[7] is None


# --------------------------------------------------------------- install ---

def test_install_all_without_rocm_changes_nothing():
    before = (torch._int_mm, torch._scaled_mm)
    if torch.cuda.is_available():
        pytest.skip("ROCm device present")
    assert patches.install_all() == []
    assert (torch._int_mm, torch._scaled_mm) == before
