"""The patch layer's seams on the GPU against the oracle: exact for the INT8
routes (kitchen int8_linear, int8-fast, torch._int_mm, the FFN pairs), within
the stated bf16 tolerance for the fp8 routes (torch._scaled_mm, the W8A16
Linear forward)."""
import types

import numpy as np
import pytest
import torch

from _util import assert_bits_equal, assert_close, bf16_to_f32, bits16, gen, u8
from oracle import act as oact
from oracle import fp8 as of
from oracle import int8 as oi
from oracle import pair as op

import cdna4q.ops as ops
from cdna4q.patches import int8_linear, int_mm, krea2_ffn_pair, linear_fp8_w8a16, moss_ffn, scaled_mm_fp8

pytestmark = pytest.mark.gpu


def _i8(shape, g):
    return torch.randint(-127, 128, shape, generator=g, dtype=torch.int8)


def test_patched_int_mm_exact(dev):
    g = gen(21)
    a, w = _i8((77, 640), g), _i8((300, 640), g)
    assert int_mm.install()
    try:
        out = torch._int_mm(a.to(dev), w.to(dev).t())     # b = weight.T, the common caller form
        ref = torch._int_mm(a, w.t())                      # CPU stock op (int64-exact)
        assert torch.equal(out.cpu(), ref)
        f = torch._int_mm(torch.ones(32, 32, device=dev, dtype=torch.int8),
                          torch.ones(32, 32, device=dev, dtype=torch.int8))
        assert int(f[0, 0]) == 32
    finally:
        int_mm.uninstall()


@pytest.mark.parametrize("scale", ["tensor", "channel"])
@pytest.mark.parametrize("bias", [False, True])
def test_kitchen_int8_linear_exact(dev, scale, bias):
    g = gen(22)
    x = torch.randn(2, 150, 512, generator=g).to(torch.bfloat16)
    w = _i8((384, 512), g)
    ws = (torch.rand(1, generator=g) * 0.01) if scale == "tensor" else torch.rand(384, generator=g) * 0.01
    b = torch.randn(384, generator=g).to(torch.bfloat16) if bias else None
    int8_linear._act_cache = None
    out = int8_linear.int8_linear(x.to(dev), w.to(dev), ws.to(dev), b.to(dev) if bias else None)
    assert out.shape == (2, 150, 384)
    ref = oi.int8_linear(bits16(x.reshape(-1, 512)), w.numpy(), ws.numpy(),
                         bits16(b) if bias else None)
    assert_bits_equal(bits16(out.reshape(-1, 384)), ref, f"int8_linear {scale} bias={bias}")


def test_kitchen_int8_linear_f16_out_eager_rescale(dev):
    """Non-bf16 output: raw int32 GEMM + comfy_kitchen's eager rescale,
    identical to the same torch ops on the CPU."""
    g = gen(23)
    x = torch.randn(64, 256, generator=g).to(torch.bfloat16)
    w = _i8((96, 256), g)
    ws = torch.rand(96, generator=g) * 0.01
    b = torch.randn(96, generator=g).to(torch.float16)
    int8_linear._act_cache = None
    out = int8_linear.int8_linear(x.to(dev), w.to(dev), ws.to(dev), b.to(dev), torch.float16)
    q, xs = oi.quant_rowwise(bits16(x))
    c = torch.from_numpy(oi.i8_matmul2d_nt(q, w.numpy()))
    ref = (c.float() * (ws * torch.from_numpy(xs).reshape(-1, 1))).to(torch.float16) + b
    assert torch.equal(out.cpu(), ref)


def test_int8_fast_seam_exact(dev):
    g = gen(24)
    x = torch.randn(40, 512, generator=g).to(torch.bfloat16)
    w = _i8((256, 512), g)
    ws = torch.rand(1, generator=g) * 0.01
    int8_linear._act_cache = None
    out = int8_linear.int8_forward_dynamic(x.to(dev), w.to(dev), ws.to(dev), None, torch.bfloat16)
    assert_bits_equal(bits16(out), oi.int8_linear(bits16(x), w.numpy(), ws.numpy()), "int8-fast")


def test_patched_scaled_mm_vs_torch_cpu(dev):
    g = gen(25)
    x = torch.randn(256, 1024, generator=g)
    sa = x.abs().amax() / 448
    a = (x / sa).clamp(-448, 448).to(torch.float8_e4m3fn)
    wf = 0.02 * torch.randn(512, 1024, generator=g)
    sb = wf.abs().amax() / 448
    w = (wf / sb).clamp(-448, 448).to(torch.float8_e4m3fn)
    ref = torch._scaled_mm(a, w.t(), scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)
    assert scaled_mm_fp8.install()
    try:
        out = torch._scaled_mm(a.to(dev), w.to(dev).t(), scale_a=sa.to(dev), scale_b=sb.to(dev),
                               out_dtype=torch.bfloat16)
    finally:
        scaled_mm_fp8.uninstall()
    assert_close(bf16_to_f32(bits16(out)), ref.float().numpy(), "patched _scaled_mm")


@pytest.mark.parametrize("scaled", [False, True])
def test_w8a16_forward_vs_oracle(dev, scaled):
    g = gen(26)
    N, K = 768, 1024
    wf = 0.02 * torch.randn(N, K, generator=g)
    ws = wf.abs().amax() / 448 if scaled else None
    w = ((wf / ws) if scaled else wf * 20).clamp(-448, 448).to(torch.float8_e4m3fn)
    bias = (0.01 * torch.randn(N, generator=g)).to(torch.bfloat16)
    layer = types.SimpleNamespace(
        weight=torch.nn.Parameter(w.to(dev), requires_grad=False), bias=bias.to(dev),
        weight_function=[], bias_function=[])
    if scaled:
        layer.scale_weight = ws.reshape(()).to(dev)
    x = torch.randn(3, 100, K, generator=g).to(torch.bfloat16)
    assert linear_fp8_w8a16._eligible(layer, x.to(dev))
    linear_fp8_w8a16._self_checked = False
    out = linear_fp8_w8a16._w8a16_forward(layer, x.to(dev))
    assert out.shape == (3, 100, N) and out.dtype == torch.bfloat16
    ref = of.w8a16_linear(bits16(x.reshape(-1, K)), u8(w), ws.reshape(1).numpy() if scaled else None,
                          bias.float().numpy(), "f32")
    assert_close(bf16_to_f32(bits16(out.reshape(-1, N))), bf16_to_f32(ref), "w8a16 forward")


def test_krea2_project_exact(dev):
    """Krea2 project: ConvRot rotation of every 256-group + rowwise quant
    (the fused pass), then the pair kernel with the SiLU table, against the
    oracle's rotate + quant and unfused pair chain (reference
    _patches/krea2_ffn_pair.py:37-49)."""
    from oracle import convrot as ocr
    g = gen(27)
    K, F = 512, 384
    x = torch.randn(1, 200, K, generator=g).to(torch.bfloat16)
    wg, wu = _i8((F, K), g), _i8((F, K), g)
    gs, us = torch.rand(F, generator=g) * 0.02, torch.rand(F, generator=g) * 0.02
    int8_linear._act_cache = None
    out = krea2_ffn_pair.project(x.to(dev), (wg.to(dev), gs.to(dev)), (wu.to(dev), us.to(dev)))
    assert out.shape == (1, 200, F)
    xb = bits16(x.reshape(200, K)).reshape(200, K // 256, 1, 256)
    q, rs = ocr.merge_rot_quant(xb)
    ref = op.krea2_pair(q, wg.numpy(), wu.numpy(), np.asarray(rs).reshape(-1), gs.numpy(),
                        us.numpy())
    assert_bits_equal(bits16(out.reshape(-1, F)), ref, "krea2 project (ConvRot)")


def test_krea2_candidate_routes_convrot_layers(dev):
    """The SwiGLU seam on ConvRot group-256 INT8 layers: down(project(x))
    with the pair output bit-exact against the oracle chain."""
    from oracle import convrot as ocr
    g = gen(31)
    K, F = 768, 256
    x = torch.randn(1, 96, K, generator=g).to(torch.bfloat16)
    wg, wu = _i8((F, K), g), _i8((F, K), g)
    gs, us = torch.rand(F, generator=g) * 0.02, torch.rand(F, generator=g) * 0.02

    class QT:
        _layout_cls = "TensorWiseINT8Layout"

        def __init__(self, q, s):
            self._qdata = q
            self._params = types.SimpleNamespace(scale=s, convrot=True, convrot_groupsize=256,
                                                 transposed=False)

    def lin(q, s):
        return types.SimpleNamespace(weight=QT(q.to(dev), s.to(dev)), bias=None,
                                     weight_function=[], bias_function=[])
    seen = []
    mod = types.SimpleNamespace(gate=lin(wg, gs), up=lin(wu, us),
                                down=lambda h: seen.append(h) or "down")
    int8_linear._act_cache = None
    with torch.no_grad():
        assert krea2_ffn_pair.candidate(lambda self, x: "original", mod, x.to(dev)) == "down"
    q, rs = ocr.merge_rot_quant(bits16(x.reshape(96, K)).reshape(96, K // 256, 1, 256))
    ref = op.krea2_pair(q, wg.numpy(), wu.numpy(), np.asarray(rs).reshape(-1), gs.numpy(),
                        us.numpy())
    assert_bits_equal(bits16(seen[0].reshape(-1, F)), ref, "krea2 candidate")


def test_moss_project_exact(dev):
    g = gen(28)
    q, w = _i8((130, 384), g), _i8((2 * 256, 384), g)
    rs, cs = torch.rand(130, generator=g) * 0.01, torch.rand(512, generator=g) * 0.02
    th, tg = oact.situ_tables()
    tabs = tuple(torch.from_numpy(t.view(np.int16)).to(dev) for t in (th, tg))
    out = moss_ffn.project(q.to(dev), rs.to(dev), w.to(dev), cs.to(dev), tabs)
    ref = op.moss_pair(q.numpy(), w.numpy(), rs.numpy(), cs.numpy(), th, tg)
    assert_bits_equal(bits16(out), ref, "moss project")


def test_moss_bf16_project_exact(dev):
    """The reference's MOSS shape (x [1, 4096, 3072], weight [16384, 3072])
    through the patch's gate and project, quarter-integer operands (exact
    fp32 sums in any order): bit-exact against the oracle."""
    from cdna4q.patches import moss_bf16_ffn_pair as mb
    g = gen(29)
    x = (torch.randint(-6, 7, (1, 4096, 3072), generator=g) * 0.25).to(torch.bfloat16)
    w = (torch.randint(-6, 7, (16384, 3072), generator=g) * 0.25).to(torch.bfloat16)
    xd, wd = x.to(dev), w.to(dev)
    assert mb.eligible(xd, wd)
    out = mb.project(xd, wd)
    assert out.shape == (1, 4096, 8192)
    rows = slice(0, 4096, 37)                   # the oracle on a row sample (seconds, not minutes)
    ref = op.moss_bf16_pair(bits16(x[0, rows]), bits16(w), *oact.situ_tables())
    assert_bits_equal(bits16(out[0, rows]), ref, "moss bf16 project")


def test_o_proj_prequant_and_swiglu_forward_exact(dev):
    """The two ConvRot routes of the INT8 linear patch on a stand-in
    TensorWiseINT8Layout weight, bit-exact against the oracle chains."""
    import types
    from oracle import convrot as ocr

    class QT:
        _layout_cls = "TensorWiseINT8Layout"

        def __init__(self, q, scale):
            self._qdata = q
            self._params = types.SimpleNamespace(scale=scale, convrot=True, transposed=False,
                                                 convrot_groupsize=256)

    g = gen(31)
    B, H, S, D, N = 1, 8, 70, 128, 384
    x = (torch.randn(B, H, S, D, generator=g) * 3).to(torch.bfloat16)
    w = _i8((N, H * D), g)
    ws = torch.rand(N, generator=g) * 0.002
    layer = types.SimpleNamespace(weight=QT(w.to(dev), ws.to(dev)), bias=None, weight_function=[],
                                  bias_function=[])
    out = int8_linear.int8_o_proj_prequant(layer, x.to(dev))
    assert out.shape == (B, S, N)
    rq, rs = ocr.merge_rot_quant(bits16(x))
    ref = oi.epilogue_rowcolscale(oi.i8_matmul2d_nt(rq, w.numpy()), rs.reshape(-1), ws.numpy())
    assert_bits_equal(bits16(out.reshape(S, N)), ref, "o_proj patch")
    F = 512
    xf = (torch.randn(2, 35, 2 * F, generator=g) * 2).to(torch.bfloat16)
    w2 = _i8((N, F), g)
    lin = types.SimpleNamespace(weight=QT(w2.to(dev), ws.to(dev)), bias=None, weight_function=[],
                                bias_function=[])
    y = int8_linear._try_int8_swiglu_forward(lin, xf.to(dev))
    assert y.shape == (2, 35, N)
    silu_dev = oact.silu_table()
    rq2, rs2 = oi.quant_rowwise(ocr.swiglu_rot(bits16(xf.reshape(70, 2 * F)), silu_dev), "bf16")
    ref2 = oi.epilogue_rowcolscale(oi.i8_matmul2d_nt(rq2, w2.numpy()), rs2.reshape(-1), ws.numpy())
    assert_bits_equal(bits16(y.reshape(70, N)), ref2, "swiglu fc2 patch")


def test_qkv_prequant_routes_exact(dev):
    """The H3 QKV routes of the INT8 linear patch on a stand-in
    TensorWiseINT8Layout weight: layout-only and with Q/K RMSNorm + partial
    RoPE, bit-exact against the oracle chain (rowwise quant, product,
    per-channel epilogue, scatter, norm/RoPE)."""
    import types
    from oracle import qknorm as oqk

    class QT:
        _layout_cls = "TensorWiseINT8Layout"

        def __init__(self, q, scale):
            self._qdata = q
            self._params = types.SimpleNamespace(scale=scale, convrot=False, transposed=False)

    g = gen(33)
    S, K, H, D, R = 200, 512, 3, 128, 48
    x = (torch.randn(S, K, generator=g) * 2).to(torch.bfloat16)
    w = _i8((3 * H * D, K), g)
    ws = torch.rand(3 * H * D, generator=g) * 0.002
    bias = (torch.randn(3 * H * D, generator=g) * 0.1).to(torch.bfloat16)
    fr = torch.randn(1, S, 1, R, 2, 2, generator=g).to(torch.bfloat16)
    qw = (1 + torch.randn(D, generator=g) * 0.1).float()
    kw = (1 + torch.randn(D, generator=g) * 0.1).float()
    layer = types.SimpleNamespace(weight=QT(w.to(dev), ws.to(dev)), bias=bias.to(dev),
                                  weight_function=[], bias_function=[])
    xq, xs = oi.quant_rowwise(bits16(x), "bf16")
    pre = oi.scatter_qkv(oi.epilogue_rowcolscale(oi.i8_matmul2d_nt(xq, w.numpy()), xs.reshape(-1),
                                                 ws.numpy(), bits16(bias)), H, D)
    outs = int8_linear.int8_qkv_prequant(layer, x.to(dev), H, D)
    for name, o, r in zip("qkv", outs, pre):
        assert_bits_equal(bits16(o), r, f"qkv patch {name}")
    ref = oqk.qkv_rms_rope(*pre, bits16(fr), qw.numpy(), kw.numpy(), 1e-6)
    outs = int8_linear.int8_qkv_rms_rope_prequant(layer, x.to(dev), fr.to(dev), qw.to(dev),
                                                  kw.to(dev), H, D, 1e-6)
    for name, o, r in zip("qkv", outs, ref):
        assert_bits_equal(bits16(o), r, f"qkv rms-rope patch {name}")


def test_qkv_runtime_lora_route_exact(dev):
    """The H3 QKV + norm/RoPE route with a fast runtime LoRA adapter on the
    device: the low-rank deltas come from torch on the GPU (the route's own
    calls), the rest is the oracle chain -- per partition the fused_cs value,
    the rounded delta term, the scatter, Q/K norm + RoPE -- bit-exact."""
    import torch.nn.functional as F
    from oracle import qknorm as oqk

    class QT:
        _layout_cls = "TensorWiseINT8Layout"

        def __init__(self, q, scale):
            self._qdata = q
            self._params = types.SimpleNamespace(scale=scale, convrot=False, transposed=False)

    class Adapter:
        fast = True

        def __init__(self, up, down, scale):
            self.up, self.down, self.scale = up, down, scale

        def linear_parts(self, x):
            return self.up, self.down, self.scale

        def add_qkv_to(self, q, k, v, x, heads, head_dim):
            raise AssertionError("the norm/RoPE route uses the partition kernel")

    g = gen(37)
    S, K, H, D, R, rank = 200, 512, 3, 128, 48, 8
    x = (torch.randn(S, K, generator=g) * 2).to(torch.bfloat16)
    w = _i8((3 * H * D, K), g)
    ws = torch.rand(3 * H * D, generator=g) * 0.002
    bias = (torch.randn(3 * H * D, generator=g) * 0.1).to(torch.bfloat16)
    fr = torch.randn(1, S, 1, R, 2, 2, generator=g).to(torch.bfloat16)
    qw = (1 + torch.randn(D, generator=g) * 0.1).float()
    kw = (1 + torch.randn(D, generator=g) * 0.1).float()
    up = (torch.randn(3 * H * D, rank, generator=g) * 0.2).to(torch.bfloat16).to(dev)
    down = (torch.randn(rank, K, generator=g) * 0.2).to(torch.bfloat16).to(dev)
    layer = types.SimpleNamespace(weight=QT(w.to(dev), ws.to(dev)), bias=bias.to(dev),
                                  weight_function=[], bias_function=[],
                                  _asfp8_runtime_lora=Adapter(up, down, 0.75))
    xd = x.to(dev)
    outs = int8_linear.int8_qkv_rms_rope_prequant(layer, xd, fr.to(dev), qw.to(dev), kw.to(dev),
                                                  H, D, 1e-6)
    xq, xs = oi.quant_rowwise(bits16(x), "bf16")
    base = oi.epilogue_rowcolscale(oi.i8_matmul2d_nt(xq, w.numpy()), xs.reshape(-1), ws.numpy(),
                                   bits16(bias))
    low = F.linear(xd, down)
    width = H * D
    for kind, name in enumerate("qkv"):
        cols = slice(kind * width, (kind + 1) * width)
        delta = bits16(F.linear(low, up[cols]).cpu())
        ref = oi.scatter_part(oi.lora_delta_add(base[:, cols], delta, 0.75), H, D)
        if kind != 2:
            ref = oqk.qk_rms_rope(ref, bits16(fr), (kw if kind == 1 else qw).numpy(), 1e-6)
        assert_bits_equal(bits16(outs[kind]), ref, f"qkv lora patch {name}")


def test_qkv_route_convrot_exact(dev):
    """A ConvRot QKV weight: x rotated + quantized by the fused pass, then
    the QKV scatter -- bit-exact against the oracle chain."""
    from oracle import convrot as ocr

    class QT:
        _layout_cls = "TensorWiseINT8Layout"

        def __init__(self, q, scale):
            self._qdata = q
            self._params = types.SimpleNamespace(scale=scale, convrot=True, transposed=False,
                                                 convrot_groupsize=256)

    g = gen(39)
    S, K, H, D = 150, 512, 2, 128
    x = (torch.randn(S, K, generator=g) * 2).to(torch.bfloat16)
    w = _i8((3 * H * D, K), g)
    ws = torch.rand(3 * H * D, generator=g) * 0.002
    layer = types.SimpleNamespace(weight=QT(w.to(dev), ws.to(dev)), bias=None,
                                  weight_function=[], bias_function=[])
    outs = int8_linear.int8_qkv_prequant(layer, x.to(dev), H, D)
    rq, rs = ocr.merge_rot_quant(bits16(x).reshape(S, K // 256, 1, 256))   # the product's view
    pre = oi.scatter_qkv(oi.epilogue_rowcolscale(oi.i8_matmul2d_nt(rq, w.numpy()), rs.reshape(-1),
                                                 ws.numpy()), H, D)
    for name, o, r in zip("qkv", outs, pre):
        assert_bits_equal(bits16(o), r, f"qkv convrot patch {name}")


def test_mlp_bridge_route_exact(dev):
    """int8_mlp_bridge(fc1, fc2, x) on stand-in TensorWiseINT8Layout weights
    (FC2 ConvRot): the FC2 output of the oracle chain, bit-exact."""
    import types
    from oracle import convrot as ocr

    class QT:
        _layout_cls = "TensorWiseINT8Layout"

        def __init__(self, q, scale, convrot):
            self._qdata = q
            self._params = types.SimpleNamespace(scale=scale, convrot=convrot, transposed=False,
                                                 convrot_groupsize=256)

    g = gen(35)
    M, K, F, N2 = 400, 512, 512, 384
    x = (torch.randn(M, K, generator=g) * 2).to(torch.bfloat16)
    w1, w2 = _i8((2 * F, K), g), _i8((N2, F), g)
    s1, s2 = torch.rand(2 * F, generator=g) * 0.002, torch.rand(N2, generator=g) * 0.002
    b1 = (0.1 * torch.randn(2 * F, generator=g)).to(torch.bfloat16)
    b2 = (0.1 * torch.randn(N2, generator=g)).to(torch.bfloat16)
    fc1 = types.SimpleNamespace(weight=QT(w1.to(dev), s1.to(dev), False), bias=b1.to(dev),
                                weight_function=[], bias_function=[])
    fc2 = types.SimpleNamespace(weight=QT(w2.to(dev), s2.to(dev), True), bias=b2.to(dev),
                                weight_function=[], bias_function=[])
    out = int8_linear.int8_mlp_bridge(fc1, fc2, x.to(dev))
    assert out.shape == (M, N2)
    xq, xs = oi.quant_rowwise(bits16(x), "bf16")
    h = oi.epilogue_rowcolscale(oi.i8_matmul2d_nt(xq, w1.numpy()), xs.reshape(-1), s1.numpy(),
                                bits16(b1))
    silu = oact.silu_table()
    rq, rs = oi.quant_rowwise(ocr.swiglu_rot(h, silu), "bf16")
    ref = oi.epilogue_rowcolscale(oi.i8_matmul2d_nt(rq, w2.numpy()), rs.reshape(-1), s2.numpy(),
                                  bits16(b2))
    assert_bits_equal(bits16(out), ref, "mlp bridge route")
