"""Runtime-LoRA seams of the INT8 routes, CPU only: which adapters each route
serves, which kernel calls it makes, and that the composed result is the
reference's composition (``_patches/int8_linear_kernel_mps.py``: QKV
``:266-412``, o-projection ``:459-531``, MLP bridge ``:538-673``, SwiGLU
``:708-775``). The kernels are replaced by CPU fakes; the partition
kernel's own arithmetic is checked on the GPU in tests/test_gpu_parity.py.
The adapter is a stand-in with the interface the reference's runtime LoRA
class exposes (``fast``, ``linear_parts``, ``add_to``, ``add_bhsd_to``,
``add_qkv_to``)."""
import types

import pytest
import torch
import torch.nn.functional as F

import cdna4q.ops as ops
from cdna4q.patches import _common, int8_linear


@pytest.fixture
def cpu_gate(monkeypatch):
    monkeypatch.setattr(_common, "DEVICE_TYPE", "cpu")


class FakeQT:
    _layout_cls = "TensorWiseINT8Layout"

    def __init__(self, q, scale, convrot=False, convrot_groupsize=256):
        self._qdata = q
        self._params = types.SimpleNamespace(scale=scale, convrot=convrot, transposed=False,
                                             convrot_groupsize=convrot_groupsize)


def _layer(w, bias=None, lora=None):
    layer = types.SimpleNamespace(weight=w, bias=bias, weight_function=[], bias_function=[])
    if lora is not None:
        layer._asfp8_runtime_lora = lora
    return layer


class Adapter:
    """up [N, r], down [r, K], scale; records the calls it receives."""

    def __init__(self, n, k, rank=4, scale=0.5, fast=True, seed=0):
        g = torch.Generator().manual_seed(seed)
        self.up = (torch.randn(n, rank, generator=g) * 0.1).to(torch.bfloat16)
        self.down = (torch.randn(rank, k, generator=g) * 0.1).to(torch.bfloat16)
        self.scale = scale
        self.fast = fast
        self.calls = []

    def linear_parts(self, x):
        self.calls.append("linear_parts")
        return self.up, self.down, self.scale

    def add_to(self, base, x):
        self.calls.append("add_to")
        return base.add_(F.linear(F.linear(x, self.down), self.up), alpha=self.scale)

    def add_bhsd_to(self, base, x):
        self.calls.append("add_bhsd_to")
        b, h, s, d = x.shape
        return self.add_to(base, x.transpose(1, 2).reshape(b, s, h * d))

    def add_qkv_to(self, q, k, v, x, heads, head_dim):
        self.calls.append("add_qkv_to")
        return q, k, v


def _i8(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-128, 128, shape, generator=g, dtype=torch.int8)


def _fake_quant(x, convrot=False, gs=256):
    return torch.zeros(x.shape, dtype=torch.int8), torch.ones(x.shape[0], 1)


# ------------------------------------------------------------------- QKV ---

def _qkv_setup(monkeypatch, convrot=False, k=64):
    seen = []

    def quant(x, convrot=False, gs=256):
        seen.append(("quant", convrot, gs))
        return _fake_quant(x)
    monkeypatch.setattr(int8_linear, "_quant_cached", quant)
    monkeypatch.setattr(ops, "i8_matmul2d_nt_fused_cs_qkv",
                        lambda *a: seen.append("scatter") or ["q", "k", "v"])
    monkeypatch.setattr(ops, "i8_matmul2d_nt_fused_cs_qkv_rms_rope",
                        lambda *a: seen.append("rope") or ["Q", "K", "V"])

    def part(x_8, b, rs, cs, bias, delta, fr, nw, heads, head_dim, kind, scale, eps):
        seen.append(("part", kind, tuple(b.shape), tuple(cs.shape),
                     None if bias is None else tuple(bias.shape), delta, nw, scale))
        return f"part{kind}"
    monkeypatch.setattr(ops, "i8_matmul2d_nt_fused_cs_qkv_lora_part", part)
    H, D = 2, 128
    x = torch.randn(70, k).to(torch.bfloat16)
    q = _i8((3 * H * D, k), 1)
    bias = torch.randn(3 * H * D).to(torch.bfloat16)
    return seen, H, D, x, q, bias


def test_qkv_scatter_route_adds_the_adapter_after_the_scatter(cpu_gate, monkeypatch):
    seen, H, D, x, q, bias = _qkv_setup(monkeypatch)
    lora = Adapter(3 * H * D, x.shape[1])
    out = int8_linear.int8_qkv_prequant(_layer(FakeQT(q, torch.rand(3 * H * D)), bias, lora),
                                        x, H, D)
    assert out == ["q", "k", "v"] and seen[-1] == "scatter" and lora.calls == ["add_qkv_to"]


def test_qkv_norm_route_runs_one_partition_kernel_per_q_k_v(cpu_gate, monkeypatch):
    seen, H, D, x, q, bias = _qkv_setup(monkeypatch)
    lora = Adapter(3 * H * D, x.shape[1], scale=0.25)
    fr = torch.zeros(70, 48, 2, 2, dtype=torch.bfloat16)
    qw, kw = torch.ones(D), torch.full((D,), 2.0)
    out = int8_linear.int8_qkv_rms_rope_prequant(
        _layer(FakeQT(q, torch.rand(3 * H * D)), bias, lora), x, fr, qw, kw, H, D, 1e-6)
    assert out == ["part0", "part1", "part2"]
    parts = [c for c in seen if isinstance(c, tuple) and c[0] == "part"]
    assert [p[1] for p in parts] == [0, 1, 2]
    low = F.linear(x, lora.down)
    w = H * D
    for kind, (_, _, bshape, cshape, bias_shape, delta, nw, scale) in enumerate(parts):
        assert bshape == (w, x.shape[1]) and cshape == (w,) and bias_shape == (w,)
        assert torch.equal(delta, F.linear(low, lora.up[kind * w:(kind + 1) * w]))
        assert nw is (kw if kind == 1 else qw) and scale == 0.25
    assert lora.calls == ["linear_parts"]


def test_qkv_routes_decline_slow_or_incomplete_adapters(cpu_gate, monkeypatch):
    seen, H, D, x, q, bias = _qkv_setup(monkeypatch)
    fr = torch.zeros(70, 48, 2, 2, dtype=torch.bfloat16)
    w = torch.ones(D)
    slow = Adapter(3 * H * D, x.shape[1], fast=False)
    layer = _layer(FakeQT(q, torch.rand(3 * H * D)), bias, slow)
    assert int8_linear.int8_qkv_prequant(layer, x, H, D) is None
    assert int8_linear.int8_qkv_rms_rope_prequant(layer, x, fr, w, w, H, D, 1e-6) is None
    # an adapter without linear_parts: the scatter route only
    partial = types.SimpleNamespace(fast=True, add_qkv_to=lambda q, k, v, *a: (q, k, v))
    layer = _layer(FakeQT(q, torch.rand(3 * H * D)), bias, partial)
    assert int8_linear.int8_qkv_prequant(layer, x, H, D) == ["q", "k", "v"]
    assert int8_linear.int8_qkv_rms_rope_prequant(layer, x, fr, w, w, H, D, 1e-6) is None
    # a low-rank factor of the wrong width
    bad = Adapter(2 * H * D, x.shape[1])
    layer = _layer(FakeQT(q, torch.rand(3 * H * D)), bias, bad)
    assert int8_linear.int8_qkv_rms_rope_prequant(layer, x, fr, w, w, H, D, 1e-6) is None


def test_qkv_routes_serve_convrot_weights_through_the_rotation(cpu_gate, monkeypatch):
    seen, H, D, x, q, bias = _qkv_setup(monkeypatch, k=512)
    layer = _layer(FakeQT(q, torch.rand(3 * H * D), convrot=True), bias)
    assert int8_linear.int8_qkv_prequant(layer, x, H, D) == ["q", "k", "v"]
    assert ("quant", True, 256) in seen
    odd = _layer(FakeQT(q, torch.rand(3 * H * D), convrot=True, convrot_groupsize=128), bias)
    assert int8_linear.int8_qkv_prequant(odd, x, H, D) is None


# ---------------------------------------------------------------- o-proj ---

def test_o_proj_adds_the_adapter_delta(cpu_gate, monkeypatch):
    monkeypatch.setattr(ops, "i8_merge_rot_quant", lambda x: _fake_quant(
        torch.zeros(x.shape[0] * x.shape[2], x.shape[1] * x.shape[3])))
    base = torch.randn(1, 5, 16).to(torch.bfloat16)
    monkeypatch.setattr(int8_linear, "_int8_linear_prequant",
                        lambda *a, **k: base.clone())
    x = torch.randn(1, 4, 5, 128).to(torch.bfloat16)
    q = _i8((16, 512), 1)
    lora = Adapter(16, 512, scale=0.5)
    out = int8_linear.int8_o_proj_prequant(_layer(FakeQT(q, torch.rand(16), convrot=True),
                                                  None, lora), x)
    merged = x.transpose(1, 2).reshape(1, 5, 512)
    want = base.clone().add_(F.linear(F.linear(merged, lora.down), lora.up), alpha=0.5)
    assert torch.equal(out, want) and lora.calls[0] == "add_bhsd_to"
    slow = Adapter(16, 512, fast=False)
    assert int8_linear.int8_o_proj_prequant(_layer(FakeQT(q, torch.rand(16), convrot=True),
                                                   None, slow), x) is None


# ---------------------------------------------------------------- SwiGLU ---

def test_swiglu_forward_projects_the_activation_and_adds_the_adapter(cpu_gate, monkeypatch):
    seen = []
    monkeypatch.setattr(int8_linear, "_int8_linear_kernel",
                        lambda act, w, s, b, dt, convrot, gs: seen.append((convrot, gs)) or
                        torch.zeros(*act.shape[:-1], w.shape[0], dtype=act.dtype))
    x = torch.randn(3, 1024).to(torch.bfloat16)
    q = _i8((8, 512), 1)
    lora = Adapter(8, 512, scale=2.0)
    out = int8_linear._try_int8_swiglu_forward(
        _layer(FakeQT(q, torch.rand(8), convrot=True), None, lora), x)
    act = F.silu(x[:, :512]) * x[:, 512:]
    want = torch.zeros(3, 8, dtype=torch.bfloat16).add_(
        F.linear(F.linear(act, lora.down), lora.up), alpha=2.0)
    assert torch.equal(out, want) and seen == [(True, 256)] and lora.calls == ["add_to"]
    slow = Adapter(8, 512, fast=False)
    assert int8_linear._try_int8_swiglu_forward(
        _layer(FakeQT(q, torch.rand(8), convrot=True), None, slow), x) is None


# ------------------------------------------------------------ MLP bridge ---

def _bridge_fakes(monkeypatch):
    """CPU stand-ins with simple deterministic arithmetic, so the route's
    composition can be recomputed by hand."""
    def fused_cs(x8, w, rs, cs, bias):
        return ((x8.float() @ w.float().t()) * rs[:, None] * cs[None]).to(torch.bfloat16)

    def quant(x, convrot=False, gs=256):
        s = x.float().abs().amax(dim=1).clamp_min(1e-30) / 127
        return torch.round(x.float() / s[:, None]).to(torch.int8), s

    def prequant(x8, xs, w, ws, b, dt, shape, split_tail=False):
        return ((x8.float() @ w.float().t()) * xs.reshape(-1, 1) * ws[None]).to(dt)

    def bridge(*a):
        raise AssertionError("the LoRA route must not use the fused bridge")
    monkeypatch.setattr(ops, "i8_matmul2d_nt_fused_cs", fused_cs)
    monkeypatch.setattr(int8_linear, "_quant_cached", quant)
    monkeypatch.setattr(int8_linear, "_int8_linear_prequant", prequant)
    monkeypatch.setattr(ops, "i8_mlp_bridge_prequant", bridge)
    return fused_cs, quant, prequant


@pytest.mark.parametrize("which", ["fc1", "fc2", "both"])
def test_mlp_bridge_lora_tiles_compose_like_the_reference(cpu_gate, monkeypatch, which):
    fused_cs, quant, prequant = _bridge_fakes(monkeypatch)
    monkeypatch.setenv("ASFP8_INT8_MLP_LORA_TILE_ROWS", "130")     # -> 128-row tiles
    rows, K, Fh, N2 = 300, 64, 256, 32
    x = torch.randn(rows, K).to(torch.bfloat16)
    q1, s1 = _i8((2 * Fh, K), 1), torch.rand(2 * Fh) * 1e-3
    q2, s2 = _i8((N2, Fh), 2), torch.rand(N2) * 1e-3
    l1 = Adapter(2 * Fh, K, scale=0.5, seed=1) if which in ("fc1", "both") else None
    l2 = Adapter(N2, Fh, scale=0.25, seed=2) if which in ("fc2", "both") else None
    fc1 = _layer(FakeQT(q1, s1), None, l1)
    fc2 = _layer(FakeQT(q2, s2, convrot=True), None, l2)
    out = int8_linear.int8_mlp_bridge(fc1, fc2, x)
    # the reference's composition, one 128-row tile at a time
    x8, xs = quant(x)
    fc2_8 = torch.empty(rows, Fh, dtype=torch.int8)
    fc2_s = torch.empty(rows, 1)
    low2 = []
    for lo in range(0, rows, 128):
        hi = min(lo + 128, rows)
        wide = fused_cs(x8[lo:hi], q1, xs[lo:hi], s1, None)
        if l1 is not None:
            wide.add_(F.linear(F.linear(x, l1.down)[lo:hi], l1.up), alpha=0.5)
        act = F.silu(wide[:, :Fh]) * wide[:, Fh:]
        if l2 is not None:
            low2.append(F.linear(act, l2.down))
        a8, a_s = quant(act)
        fc2_8[lo:hi], fc2_s[lo:hi] = a8, a_s.reshape(-1, 1)
    want = prequant(fc2_8, fc2_s, q2, s2, None, x.dtype, x.shape)
    if l2 is not None:
        want.add_(F.linear(torch.cat(low2), l2.up), alpha=0.25)
    assert torch.equal(out, want)


def test_mlp_bridge_declines_slow_adapters(cpu_gate, monkeypatch):
    _bridge_fakes(monkeypatch)
    x = torch.randn(70, 64).to(torch.bfloat16)
    fc1 = _layer(FakeQT(_i8((512, 64), 1), torch.rand(512)), None,
                 Adapter(512, 64, fast=False))
    fc2 = _layer(FakeQT(_i8((32, 256), 2), torch.rand(32), convrot=True))
    assert int8_linear.int8_mlp_bridge(fc1, fc2, x) is None
    no_parts = types.SimpleNamespace(fast=True)
    fc1 = _layer(FakeQT(_i8((512, 64), 1), torch.rand(512)), None, no_parts)
    assert int8_linear.int8_mlp_bridge(fc1, fc2, x) is None
