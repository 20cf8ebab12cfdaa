"""GPU parity: every entry point against the CPU oracle on seeded inputs.

Integer / byte results (INT32 GEMM, fused bf16 epilogues, quantizers,
dequant, FFN pairs) must be bit-exact; fp32-accumulating GEMMs (fp8
scaled_mm, W8A16) meet the tolerance stated in ``_util.assert_close``.
Shapes and edge cases follow the reference's own tests (cited per test).
"""
import numpy as np
import pytest
import torch

from _util import (assert_bits_equal, assert_close, bf16_to_f32, bits16, from_bits16, gen, u8)
from oracle import act as oact
from oracle import convrot as ocr
from oracle import fp8 as of
from oracle import int8 as oi
from oracle import pair as op
from oracle import qknorm as oqk
from oracle.numerics import bf16_bits_to_f32, f16_bits_to_f32

import cdna4q.ops as ops
from cdna4q._lib import C4QError

pytestmark = pytest.mark.gpu


def _randint8(shape, g, lo=-128, hi=128):
    return torch.randint(lo, hi, shape, generator=g, dtype=torch.int8)


# ---------------------------------------------------------------- INT32 ---

# reference canary shapes and corners: _patches/int_mm_mps.py:69-74,
# tests/test_hardening.py:49-65; ragged K/M/N: tests/test_int8_linear_kernel.py:277-283
I8_SHAPES = [
    (3, 129, 5), (16, 4096, 32), (7, 333, 11), (64, 4096, 128), (33, 96, 63), (65, 768, 129),
    (96, 704, 385), (517, 704, 385), (1, 512, 512), (130, 512, 256), (256, 2560, 1024),
    (300, 3072, 700), (1024, 3072, 3072),
]


@pytest.mark.parametrize("M,K,N", I8_SHAPES)
def test_i8_gemm_int32_exact(dev, M, K, N):
    g = gen(M * 7 + K + N)
    a = _randint8((M, K), g)
    b = _randint8((N, K), g)
    a[:, 0] = -128
    b[:, 0] = -128
    if K > 1:
        a[:, 1] = 127
        b[:, 1] = -128
    c = ops.i8_matmul2d_nt(a.to(dev), b.to(dev))
    torch.cuda.synchronize()
    ref = oi.i8_matmul2d_nt(a.numpy(), b.numpy())
    assert_bits_equal(c.cpu().numpy(), ref, f"int32 {M}x{K}x{N}")


def test_int_mm_weight_transpose_view(dev):
    """torch._int_mm(x, weight.T) on [N,K] storage (tests/test_hardening.py:61-65)."""
    g = gen(0)
    w = _randint8((64, 512), g)
    x = _randint8((16, 512), g)
    out = ops.int_mm(x.to(dev), w.to(dev).t())
    ref = torch._int_mm(x, w.t())
    assert_bits_equal(out.cpu().numpy(), ref.numpy(), "int_mm weight.T")
    # contiguous [K,N] right operand takes the copy path
    b = _randint8((512, 48), g)
    out = ops.int_mm(x.to(dev), b.to(dev))
    assert_bits_equal(out.cpu().numpy(), torch._int_mm(x, b).numpy(), "int_mm [K,N]")


# ------------------------------------------------------ fused epilogues ---

FUSED_CASES = [  # tests/test_int8_linear_kernel.py:276-283 (+ C1 and tile tails)
    (256, 2560, 1024, True), (512, 3840, 1152, False), (65, 768, 129, True), (96, 704, 385, False),
    (128, 512, 256, True), (33, 512, 256, True), (1, 2560, 512, False), (1024, 3072, 3072, True),
    (4109, 512, 1536, True), (130, 96, 129, False),
]


@pytest.mark.parametrize("M,K,N,bias", FUSED_CASES)
def test_i8_fused_rowscale_exact(dev, M, K, N, bias):
    g = gen(11 + M + N)
    a, b = _randint8((M, K), g), _randint8((N, K), g)
    rs = torch.rand(M, generator=g) * 0.01
    rs[0] = 0.0
    bb = torch.randn(N, generator=g).to(torch.bfloat16) if bias else None
    d = ops.i8_matmul2d_nt_fused(a.to(dev), b.to(dev), rs.to(dev), bb.to(dev) if bias else None)
    ref = oi.epilogue_rowscale(oi.i8_matmul2d_nt(a.numpy(), b.numpy()), rs.numpy(),
                               bits16(bb) if bias else None)
    assert_bits_equal(bits16(d), ref, f"fused {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N,bias", FUSED_CASES)
def test_i8_fused_cs_exact(dev, M, K, N, bias):
    """Includes zero scales rs[0] = cs[0] = 0 (tests/test_krea2_gemm_tile.py:36-37)."""
    g = gen(23 + M + N)
    a, b = _randint8((M, K), g), _randint8((N, K), g)
    rs = torch.rand(M, generator=g) * 0.01
    cs = torch.rand(N, generator=g) * 0.02
    rs[0] = 0.0
    cs[0] = 0.0
    bb = torch.randn(N, generator=g).to(torch.bfloat16) if bias else None
    d = ops.i8_matmul2d_nt_fused_cs(a.to(dev), b.to(dev), rs.to(dev), cs.to(dev),
                                    bb.to(dev) if bias else None)
    ref = oi.epilogue_rowcolscale(oi.i8_matmul2d_nt(a.numpy(), b.numpy()), rs.numpy(),
                                  cs.numpy(), bits16(bb) if bias else None)
    assert_bits_equal(bits16(d), ref, f"fused_cs {M}x{K}x{N}")


# fp16-output per-channel epilogue (the Wan / MiniMax-VAE INT8 projections)
FUSED_HALF_CASES = [(1, 64, 16, True), (300, 1040, 520, True), (257, 512, 384, False),
                    (1024, 3072, 3072, True)]


@pytest.mark.parametrize("M,K,N,bias", FUSED_HALF_CASES)
def test_i8_fused_cs_half_exact(dev, M, K, N, bias):
    """Column scales spread the results from fp16 subnormals to overflow
    (inf); zero scales in row 0 / column 0."""
    g = gen(41 + M + N)
    a, b = _randint8((M, K), g), _randint8((N, K), g)
    rs = torch.rand(M, generator=g) * 0.01
    cs = torch.rand(N, generator=g) * 0.02 * torch.logspace(-5, 2, N)
    rs[0] = 0.0
    cs[0] = 0.0
    bb = (torch.randn(N, generator=g) * 4).to(torch.float16) if bias else None
    d = ops.i8_matmul2d_nt_fused_cs_half(a.to(dev), b.to(dev), rs.to(dev), cs.to(dev),
                                         bb.to(dev) if bias else None)
    assert d.dtype == torch.float16 and d.shape == (M, N)
    ref = oi.epilogue_rowcolscale_half(oi.i8_matmul2d_nt(a.numpy(), b.numpy()), rs.numpy(),
                                       cs.numpy(), bits16(bb) if bias else None)
    assert_bits_equal(bits16(d), ref, f"fused_cs_half {M}x{K}x{N}")


def test_i8_fused_cs_half_strided_generic(dev):
    """Row strides that are not multiples of 16 take the generic kernel."""
    g = gen(43)
    M, K, N = 70, 200, 90
    a = _randint8((M, K + 3), g)[:, :K]
    b = _randint8((N, K + 5), g)[:, :K]
    rs = torch.rand(M, generator=g) * 0.01
    cs = torch.rand(N, generator=g) * 0.02
    bb = torch.randn(N, generator=g).to(torch.float16)
    d = ops.i8_matmul2d_nt_fused_cs_half(a.to(dev), b.to(dev), rs.to(dev), cs.to(dev), bb.to(dev))
    ref = oi.epilogue_rowcolscale_half(oi.i8_matmul2d_nt(a.numpy(), b.numpy()), rs.numpy(),
                                       cs.numpy(), bits16(bb))
    assert_bits_equal(bits16(d), ref, "fused_cs_half generic")


def test_f16_outputs_round_f32_results_once(dev):
    """fp16 outputs of _scaled_mm and W8A16 over exact integer sums must
    match the oracle bit for bit: their epilogues multiply and add in f32 and
    round the f32 result to half. A conversion fused with the last f32
    operation (v_fma_mixlo_f16) would round the exact value instead, which
    gives another half wherever the f32 result is a half tie."""
    g = gen(61)
    M, K, N = 300, 512, 520
    af = torch.randint(-8, 9, (M, K), generator=g).float().to(torch.float8_e4m3fn)   # small integers: exact e4m3
    wf = torch.randint(-8, 9, (N, K), generator=g).float().to(torch.float8_e4m3fn)
    sa = torch.rand(M, 1, generator=g) * 0.01 + 0.001
    sb = torch.rand(1, N, generator=g) * 0.01 + 0.001
    bias = (torch.randn(N, generator=g) * 2).to(torch.float16)
    o = ops.scaled_mm(af.to(dev), wf.to(dev).t(), out_dtype=torch.float16, scale_a=sa.to(dev),
                      scale_b=sb.to(dev), bias=bias.to(dev))
    ref = of.scaled_mm(u8(af), u8(wf), sa.numpy(), sb.numpy(), bits16(bias), "f16",
                       out_dtype="f16")
    assert_bits_equal(bits16(o), ref, "scaled_mm f16 out")
    x = (torch.randint(-8, 9, (M, K), generator=g) * 0.125).to(torch.float16)
    bw = (torch.randn(N, generator=g) * 0.3).to(torch.float16)
    y = ops.w8a16_linear(x.to(dev), wf.to(dev), None, bw.to(dev))
    ref = of.w8a16_linear(bits16(x), u8(wf), None, bits16(bw), "f16", x_dtype="f16",
                          out_dtype="f16")
    assert_bits_equal(bits16(y), ref, "w8a16 f16 out")


# ConvRot: fused head merge + 256-wide rotation + rowwise quant
MRQ_CASES = [(1, 24, 300, 128), (1, 12, 257, 256), (2, 3, 50, 256), (1, 8, 33, 96),
             (1, 1, 5, 256), (1, 120, 3, 128), (1, 64, 9, 100),   # D=100: 2-byte gathers
             # one workgroup per row: far more workgroups than the device holds at
             # once, so they run in several waves of residency
             (1, 2, 6000, 128), (2, 12, 1100, 256)]


def _bhsd(g, B, H, S, D):
    x = torch.randn(B, H, S, D, generator=g) * torch.logspace(-3, 3, S)[None, None, :, None]
    x[:, :, 0] = 0.0                          # an all-zero row: scale 1e-30, tiny bf16 divisor
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("rotate", [True, False])
@pytest.mark.parametrize("B,H,S,D", MRQ_CASES)
def test_merge_rot_quant_exact(dev, B, H, S, D, rotate):
    g = gen(71 + B + H + S + D)
    x = _bhsd(g, B, H, S, D)
    q, sc = ops.i8_merge_rot_quant(x.to(dev), rotate)
    assert q.shape == (B * S, H * D) and sc.shape == (B * S, 1)
    rq, rs = ocr.merge_rot_quant(bits16(x), rotate)
    assert_bits_equal(q.cpu().numpy(), rq, f"merge_rot_quant q {B}x{H}x{S}x{D} rot={rotate}")
    assert_bits_equal(sc.cpu().numpy().reshape(-1).view(np.uint32),
                      np.asarray(rs, np.float32).reshape(-1).view(np.uint32), "scales")


def test_merge_rot_quant_unaligned_input(dev):
    """x at a 2-byte offset takes the 2-byte gathers."""
    g = gen(77)
    B, H, S, D = 1, 6, 40, 128
    x = _bhsd(g, B, H, S, D)
    flat = torch.empty(x.numel() + 1, dtype=torch.bfloat16, device=dev)
    xd = flat[1:].view(B, H, S, D)
    xd.copy_(x.to(dev))
    q, sc = ops.i8_merge_rot_quant(xd)
    rq, rs = ocr.merge_rot_quant(bits16(x))
    assert_bits_equal(q.cpu().numpy(), rq, "merge_rot_quant unaligned q")
    assert_bits_equal(sc.cpu().numpy().reshape(-1).view(np.uint32),
                      np.asarray(rs, np.float32).reshape(-1).view(np.uint32), "scales")


def test_o_proj_prequant_chain_exact(dev):
    """The reference's fused o-projection (int8_o_proj_prequant, per-channel
    weight scales): merge + rotate + quant, then the fused_cs GEMM."""
    g = gen(79)
    B, H, S, D, N = 1, 24, 130, 128, 3072
    x = _bhsd(g, B, H, S, D)
    w = _randint8((N, H * D), g, -127, 128)
    ws = torch.rand(N, generator=g) * 0.002
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    q, sc = ops.i8_merge_rot_quant(x.to(dev))
    out = ops.i8_matmul2d_nt_fused_cs(q, w.to(dev), sc.reshape(-1), ws.to(dev), bias.to(dev))
    rq, rs = ocr.merge_rot_quant(bits16(x))
    ref = oi.epilogue_rowcolscale(oi.i8_matmul2d_nt(rq, w.numpy()), np.asarray(rs).reshape(-1),
                                  ws.numpy(), bits16(bias))
    assert_bits_equal(bits16(out), ref, "o_proj chain")


@pytest.mark.parametrize("M,F", [(130, 8192), (1, 256), (37, 768), (9, 4352)])
def test_swiglu_rot_exact(dev, M, F):
    g = gen(81 + M + F)
    x = (torch.randn(M, 2 * F, generator=g) * torch.logspace(-2, 2, M)[:, None]).to(torch.bfloat16)
    silu = torch.from_numpy(oact.silu_table().view(np.int16))
    rot = ops.i8_swiglu_rot(x.to(dev), silu.to(dev))
    assert rot.shape == (M, F) and rot.dtype == torch.bfloat16
    assert_bits_equal(bits16(rot), ocr.swiglu_rot(bits16(x), oact.silu_table()),
                      f"swiglu_rot {M}x{F}")


def test_fc2_swiglu_rot_chain_exact(dev):
    """The reference's INT8 fc2 route (int8_linear_kernel_mps.py:756-770):
    swiglu_rot, rowwise quant, fused INT8 GEMM with per-channel scales."""
    g = gen(83)
    M, F, N = 96, 1024, 512
    x = (torch.randn(M, 2 * F, generator=g) * 2).to(torch.bfloat16)
    w = _randint8((N, F), g, -127, 128)
    ws = torch.rand(N, generator=g) * 0.002
    silu = torch.from_numpy(oact.silu_table().view(np.int16)).to(dev)
    rot = ops.i8_swiglu_rot(x.to(dev), silu)
    q, sc = ops.i8_quant_rowwise(rot)
    out = ops.i8_matmul2d_nt_fused_cs(q, w.to(dev), sc.reshape(-1), ws.to(dev))
    rq, rs = oi.quant_rowwise(ocr.swiglu_rot(bits16(x), oact.silu_table()), "bf16")
    ref = oi.epilogue_rowcolscale(oi.i8_matmul2d_nt(rq, w.numpy()), rs.reshape(-1), ws.numpy())
    assert_bits_equal(bits16(out), ref, "fc2 chain")


# MOSS bf16 FC1/SiTU pair
def _moss_tables(dev):
    return tuple(torch.from_numpy(t.view(np.int16)).to(dev) for t in oact.situ_tables())


@pytest.mark.parametrize("M,K,F", [(129, 3072, 8192), (300, 1040, 520), (1, 64, 64),
                                   (77, 136, 100)])
def test_moss_bf16_pair_integer_exact(dev, M, K, F):
    """Quarter-integer operands: every fp32 sum is exact in any order, so the
    kernel must equal the oracle bit for bit (first case: the reference's
    MOSS weight [16384, 3072])."""
    g = gen(51 + M + F)
    x = (torch.randint(-6, 7, (M, K), generator=g) * 0.25).to(torch.bfloat16)
    w = (torch.randint(-6, 7, (2 * F, K), generator=g) * 0.25).to(torch.bfloat16)
    out = ops.moss_bf16_pair(x.to(dev), w.to(dev), _moss_tables(dev))
    assert out.shape == (M, F) and out.dtype == torch.bfloat16
    ref = op.moss_bf16_pair(bits16(x), bits16(w), *oact.situ_tables())
    assert_bits_equal(bits16(out), ref, f"moss bf16 pair {M}x{K}x{F}")


def test_moss_bf16_pair_random(dev):
    g = gen(55)
    M, K, F = 512, 3072, 1024
    x = torch.randn(1, M, K, generator=g).to(torch.bfloat16)
    w = (0.02 * torch.randn(2 * F, K, generator=g)).to(torch.bfloat16)
    out = ops.moss_bf16_pair(x.to(dev), w.to(dev), _moss_tables(dev))
    assert out.shape == (1, M, F)
    ref = op.moss_bf16_pair(bits16(x[0]), bits16(w), *oact.situ_tables())
    assert_close(bf16_to_f32(bits16(out[0])), bf16_to_f32(ref), "moss bf16 pair random")


def test_moss_bf16_pair_generic_and_split_k(dev, monkeypatch):
    """A row stride that is not a multiple of 8 takes the generic kernel; the
    forced split-K tile runs the same pair on 64x64 pieces."""
    g = gen(57)
    M, K, F = 100, 264, 96
    x = (torch.randint(-6, 7, (M, K + 3), generator=g) * 0.25).to(torch.bfloat16)[:, :K]
    w = (torch.randint(-6, 7, (2 * F, K), generator=g) * 0.25).to(torch.bfloat16)
    ref = op.moss_bf16_pair(bits16(x), bits16(w), *oact.situ_tables())
    out = ops.moss_bf16_pair(x.to(dev), w.to(dev), _moss_tables(dev))
    assert_bits_equal(bits16(out), ref, "moss bf16 pair generic")
    monkeypatch.setenv("C4Q_TILE", "7")
    xc = x.contiguous()
    out = ops.moss_bf16_pair(xc.to(dev), w.to(dev), _moss_tables(dev))
    assert_bits_equal(bits16(out), ref, "moss bf16 pair split-K")


@pytest.mark.parametrize("tile", [None, "5", "7"])
@pytest.mark.parametrize("M,K,H,D", [(300, 1024, 4, 128), (77, 512, 3, 64), (1024, 3072, 24, 128)])
def test_i8_fused_cs_qkv_exact(dev, monkeypatch, tile, M, K, H, D):
    """H3 QKV scatter: the fused_cs bytes stored into [1, H, M, D] Q/K/V."""
    if tile is not None:
        monkeypatch.setenv("C4Q_TILE", tile)
    g = gen(91 + M + H * D)
    N = 3 * H * D
    a, b = _randint8((M, K), g), _randint8((N, K), g)
    rs = torch.rand(M, generator=g) * 0.01
    cs = torch.rand(N, generator=g) * 0.02
    bb = torch.randn(N, generator=g).to(torch.bfloat16)
    outs = ops.i8_matmul2d_nt_fused_cs_qkv(a.to(dev), b.to(dev), rs.to(dev), cs.to(dev),
                                           bb.to(dev), H, D)
    ref = oi.scatter_qkv(oi.epilogue_rowcolscale(oi.i8_matmul2d_nt(a.numpy(), b.numpy()),
                                                 rs.numpy(), cs.numpy(), bits16(bb)), H, D)
    for name, o, r in zip("qkv", outs, ref):
        assert o.shape == (1, H, M, D)
        assert_bits_equal(bits16(o), r, f"qkv {name} {M}x{K} H{H} D{D} tile {tile}")


def _qkv_rope_case(M, K, H, R, seed, unaligned=False):
    g = gen(seed)
    N = 3 * H * 128
    a, b = _randint8((M, K), g), _randint8((N, K), g)
    rs = torch.rand(M, generator=g) * 0.01
    cs = torch.rand(N, generator=g) * 0.02
    bb = torch.randn(N, generator=g).to(torch.bfloat16)
    freqs = torch.randn(1, M, 1, R, 2, 2, generator=g).to(torch.bfloat16)
    qw = (1 + torch.randn(128, generator=g) * 0.1).float()
    kw = (1 + torch.randn(128, generator=g) * 0.1).float()
    pre = oi.scatter_qkv(oi.epilogue_rowcolscale(oi.i8_matmul2d_nt(a.numpy(), b.numpy()),
                                                 rs.numpy(), cs.numpy(), bits16(bb)), H, 128)
    ref = oqk.qkv_rms_rope(*pre, bits16(freqs), qw.numpy(), kw.numpy(), 1e-6)
    return (a, b, rs, cs, bb, freqs, qw, kw), ref


@pytest.mark.parametrize("route", ["two-pass", "fused", "fused-0", "fused-1", "fused-2"])
@pytest.mark.parametrize("M,K,H,R", [(300, 1024, 4, 48), (1024, 3072, 24, 48), (777, 512, 3, 64),
                                     (130, 256, 1, 8), (2100, 640, 7, 16), (130, 256, 1, 1),
                                     (513, 128, 5, 33)])
def test_i8_fused_cs_qkv_rms_rope_exact(dev, monkeypatch, route, M, K, H, R):
    """H3 QKV + Q/K RMSNorm + partial RoPE: bit-exact to the oracle on both
    routes -- the QKV scatter then the in-place norm/RoPE pass (default),
    and the fused epilogue (R a multiple of 8; else it takes the two-pass
    route too) with its default plan (256x256 8-wave tiles + 128x128 2-wave
    tail) and each head tile forced. Odd head counts leave half of the last
    256-column tile past N."""
    if route != "two-pass":
        monkeypatch.setenv("C4Q_QKV_NORM_FUSE", "1")
    if route.startswith("fused-"):
        monkeypatch.setenv("C4Q_HEAD_TILE", route[-1])
    ins, ref = _qkv_rope_case(M, K, H, R, 7 + M + H + R)
    a, b, rs, cs, bb, freqs, qw, kw = (t.to(dev) for t in ins)
    outs = ops.i8_matmul2d_nt_fused_cs_qkv_rms_rope(a, b, rs, cs, bb, freqs, qw, kw, H, 128, 1e-6)
    for name, o, r in zip("qkv", outs, ref):
        assert o.shape == (1, H, M, 128)
        assert_bits_equal(bits16(o), r, f"qkv-rms-rope {name} {M}x{K} H{H} R{R} {route}")


@pytest.mark.parametrize("M,K,H,R", [(100, 200, 2, 48), (333, 1000, 3, 64)])
def test_i8_fused_cs_qkv_rms_rope_generic_path(dev, M, K, H, R):
    """K not a multiple of 16: the generic product + scatter, then the
    in-place norm/RoPE pass -- the same bytes."""
    ins, ref = _qkv_rope_case(M, K, H, R, 3 + M + R)
    a, b, rs, cs, bb, freqs, qw, kw = (t.to(dev) for t in ins)
    outs = ops.i8_matmul2d_nt_fused_cs_qkv_rms_rope(a, b, rs, cs, None if H == 3 else bb, freqs,
                                                    qw, kw, H, 128, 1e-6)
    if H == 3:
        a0, b0, rs0, cs0 = ins[:4]
        pre = oi.scatter_qkv(oi.epilogue_rowcolscale(oi.i8_matmul2d_nt(a0.numpy(), b0.numpy()),
                                                     rs0.numpy(), cs0.numpy(), None), H, 128)
        ref = oqk.qkv_rms_rope(*pre, bits16(ins[5]), ins[6].numpy(), ins[7].numpy(), 1e-6)
    for name, o, r in zip("qkv", outs, ref):
        assert_bits_equal(bits16(o), r, f"qkv-rms-rope generic {name} {M}x{K} H{H} R{R}")


@pytest.mark.parametrize("tile", [None, "5", "7"])
@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("M,K,H,R,bias,scale", [(300, 1024, 4, 48, True, 0.3),
                                                (777, 512, 3, 20, False, 1.0),
                                                (130, 200, 2, 48, True, 0.0123),  # generic path
                                                (2100, 640, 7, 64, True, 2.5)])
def test_i8_qkv_lora_part_exact(dev, monkeypatch, tile, kind, M, K, H, R, bias, scale):
    """H3 runtime-LoRA partition: the partition's fused_cs bytes plus the
    rounded delta term, scattered to [1, H, M, 128]; Q and K then through
    the RMSNorm + partial RoPE -- bit-exact to the oracle chain, on the
    default tile plan and with the 64x128 and split-K tiles forced."""
    if tile is not None:
        monkeypatch.setenv("C4Q_TILE", tile)
    g = gen(17 + M + H + R + kind)
    N = H * 128
    a, b = _randint8((M, K), g), _randint8((N, K), g)
    rs = torch.rand(M, generator=g) * 0.01
    cs = torch.rand(N, generator=g) * 0.02
    bb = torch.randn(N, generator=g).to(torch.bfloat16) if bias else None
    delta = (torch.randn(M, N, generator=g) * 0.5).to(torch.bfloat16)
    freqs = torch.randn(1, M, 1, R, 2, 2, generator=g).to(torch.bfloat16)
    nw = (1 + torch.randn(128, generator=g) * 0.1).float()
    base = oi.epilogue_rowcolscale(oi.i8_matmul2d_nt(a.numpy(), b.numpy()), rs.numpy(),
                                   cs.numpy(), bits16(bb) if bias else None)
    ref = oi.scatter_part(oi.lora_delta_add(base, bits16(delta), scale), H, 128)
    if kind != 2:
        ref = oqk.qk_rms_rope(ref, bits16(freqs), nw.numpy(), 1e-6)
    out = ops.i8_matmul2d_nt_fused_cs_qkv_lora_part(
        a.to(dev), b.to(dev), rs.to(dev), cs.to(dev), bb.to(dev) if bias else None,
        delta.to(dev), freqs.to(dev), nw.to(dev), H, 128, kind, scale, 1e-6)
    assert out.shape == (1, H, M, 128)
    assert_bits_equal(bits16(out), ref, f"qkv lora part kind {kind} {M}x{K} H{H} R{R} tile {tile}")


def test_i8_qkv_lora_part_zero_delta_is_the_scatter_route(dev):
    """With a zero delta the partitions equal the QKV + norm/RoPE route's
    Q, K and V (the delta term then adds +0 and rounds nothing)."""
    M, K, H, R = 512, 1024, 6, 48
    ins, _ = _qkv_rope_case(M, K, H, R, 23)
    a, b, rs, cs, bb, freqs, qw, kw = (t.to(dev) for t in ins)
    full = ops.i8_matmul2d_nt_fused_cs_qkv_rms_rope(a, b, rs, cs, bb, freqs, qw, kw, H, 128, 1e-6)
    zero = torch.zeros(M, H * 128, dtype=torch.bfloat16, device=dev)
    w = H * 128
    for kind in range(3):
        part = ops.i8_matmul2d_nt_fused_cs_qkv_lora_part(
            a, b[kind * w:(kind + 1) * w].contiguous(), rs, cs[kind * w:(kind + 1) * w].contiguous(),
            bb[kind * w:(kind + 1) * w].contiguous(), zero, freqs, kw if kind == 1 else qw,
            H, 128, kind, 0.7, 1e-6)
        assert torch.equal(part, full[kind]), f"kind {kind}"


def test_i8_qkv_lora_part_rejects_bad_arguments(dev):
    g = gen(3)
    M, K, H = 100, 256, 2
    a, b = _randint8((M, K), g).to(dev), _randint8((H * 128, K), g).to(dev)
    rs, cs = torch.ones(M, device=dev), torch.ones(H * 128, device=dev)
    delta = torch.zeros(M, H * 128, dtype=torch.bfloat16, device=dev)
    fr = torch.zeros(M, 8, 2, 2, dtype=torch.bfloat16, device=dev)
    nw = torch.ones(128, device=dev)
    call = ops.i8_matmul2d_nt_fused_cs_qkv_lora_part
    with pytest.raises(C4QError, match="kind"):
        call(a, b, rs, cs, None, delta, fr, nw, H, 128, 3, 1.0, 1e-6)
    with pytest.raises(C4QError, match="delta shape"):
        call(a, b, rs, cs, None, delta[:, :128].contiguous(), fr, nw, H, 128, 0, 1.0, 1e-6)
    with pytest.raises(C4QError, match="M > 64"):
        call(a[:64].contiguous(), b, rs[:64].contiguous(), cs, None, delta[:64].contiguous(),
             fr[:64].contiguous(), nw, H, 128, 0, 1.0, 1e-6)


def test_i8_fused_cs_qkv_rms_rope_matches_scatter_then_norm(dev):
    """V equals the plain QKV scatter's V; Q/K equal the oracle applied to
    the scatter kernel's own Q/K (the epilogue adds norm/RoPE only)."""
    M, K, H, R = 512, 1024, 6, 48
    ins, _ = _qkv_rope_case(M, K, H, R, 99)
    a, b, rs, cs, bb, freqs, qw, kw = (t.to(dev) for t in ins)
    q, k, v = ops.i8_matmul2d_nt_fused_cs_qkv(a, b, rs, cs, bb, H, 128)
    outs = ops.i8_matmul2d_nt_fused_cs_qkv_rms_rope(a, b, rs, cs, bb, freqs, qw, kw, H, 128, 1e-6)
    assert_bits_equal(bits16(outs[2]), bits16(v), "V")
    assert_bits_equal(bits16(outs[0]), oqk.qk_rms_rope(bits16(q), bits16(freqs), ins[6].numpy(),
                                                       1e-6), "Q")
    assert_bits_equal(bits16(outs[1]), oqk.qk_rms_rope(bits16(k), bits16(freqs), ins[7].numpy(),
                                                       1e-6), "K")


def test_i8_fused_cs_qkv_rms_rope_rejects_bad_shapes(dev):
    a = torch.zeros(100, 64, dtype=torch.int8, device=dev)
    b = torch.zeros(3 * 2 * 64, 64, dtype=torch.int8, device=dev)
    rs = torch.ones(100, device=dev)
    cs = torch.ones(384, device=dev)
    fr = torch.zeros(100, 16, 2, 2, dtype=torch.bfloat16, device=dev)
    w = torch.ones(128, device=dev)
    with pytest.raises(C4QError, match="D=128"):
        ops.i8_matmul2d_nt_fused_cs_qkv_rms_rope(a, b, rs, cs, None, fr, w, w, 2, 64, 1e-6)
    b = torch.zeros(3 * 2 * 128, 64, dtype=torch.int8, device=dev)
    cs = torch.ones(768, device=dev)
    with pytest.raises(C4QError, match="freqs"):
        ops.i8_matmul2d_nt_fused_cs_qkv_rms_rope(a, b, rs, cs, None, fr[:50], w, w, 2, 128, 1e-6)


@pytest.mark.parametrize("M,K,F,tile_rows", [(300, 512, 256, -1), (1000, 256, 512, 128),
                                              (1000, 256, 512, 200), (700, 128, 256, 0),
                                              (2500, 384, 256, -1), (90, 128, 15360, -1),
                                              (100, 128, 15616, 0)])
def test_i8_mlp_bridge_prequant_exact(dev, M, K, F, tile_rows):
    """FC1 -> SwiGLU -> ConvRot -> rowwise quant, chunk by chunk: the bytes of
    the unfused oracle chain for every chunking (auto, 128-row chunks, 200
    rounded down to 128, all rows at once; ragged last chunks), through the
    one-pass rotate + quant (F <= 15360) and the two-pass route (F 15616)."""
    g = gen(5 + M + F)
    W = 2 * F
    a, w1 = _randint8((M, K), g), _randint8((W, K), g)
    rs = torch.rand(M, generator=g) * 0.01
    cs = torch.rand(W, generator=g) * 0.02
    bb = torch.randn(W, generator=g).to(torch.bfloat16)
    q, sc = ops.i8_mlp_bridge_prequant(a.to(dev), w1.to(dev), rs.to(dev), cs.to(dev), bb.to(dev),
                                       tile_rows=tile_rows)
    fc1 = oi.epilogue_rowcolscale(oi.i8_matmul2d_nt(a.numpy(), w1.numpy()), rs.numpy(), cs.numpy(),
                                  bits16(bb))
    silu = oact.silu_table()
    rq, rsc = oi.quant_rowwise(ocr.swiglu_rot(fc1, silu), "bf16")
    assert q.shape == (M, F) and sc.shape == (M, 1)
    assert np.array_equal(q.cpu().numpy(), rq), f"bridge q {M}x{K} F{F} tile {tile_rows}"
    assert np.array_equal(sc.cpu().numpy().reshape(-1), np.asarray(rsc).reshape(-1)), "bridge scales"


def test_c1_golden_digest_full_size(dev):
    """BASELINE C1 at full size (seed 1): the kernel's INT32 product and
    per-channel bf16 epilogue hash to the digests written from torch._int_mm
    and torch's eager epilogue by tests/golden/make_golden.py."""
    import hashlib, json, pathlib
    d = json.loads((pathlib.Path(__file__).parent / "golden" / "digests.json").read_text())
    g = gen(d["c1_seed"])
    M, K, N = 1024, 3072, 3072
    x = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    rs = 0.005 + 0.015 * torch.rand(M, generator=g)
    cs = 0.0005 + 0.0015 * torch.rand(N, generator=g)
    c = ops.i8_matmul2d_nt(x.to(dev), w.to(dev)).cpu().numpy()
    assert hashlib.sha256(c.tobytes()).hexdigest() == d["c1_int32_sha256"]
    e = ops.i8_matmul2d_nt_fused_cs(x.to(dev), w.to(dev), rs.to(dev), cs.to(dev))
    assert hashlib.sha256(bits16(e).view(np.int16).tobytes()).hexdigest() == d["c1_epilogue_bf16_sha256"]


def test_c1_config_exact(dev):
    """X, W int8 uniform in [-127,127] (seed 1),
    rs U[0.005,0.02] [1024], cs U[0.0005,0.002] [3072]."""
    g = gen(1)
    x = _randint8((1024, 3072), g, -127, 128)
    w = _randint8((3072, 3072), g, -127, 128)
    rs = 0.005 + 0.015 * torch.rand(1024, generator=g)
    cs = 0.0005 + 0.0015 * torch.rand(3072, generator=g)
    c = ops.i8_matmul2d_nt(x.to(dev), w.to(dev))
    ref_c = torch._int_mm(x, w.t()).numpy()
    assert_bits_equal(c.cpu().numpy(), ref_c, "C1 int32 vs torch._int_mm")
    d = ops.i8_matmul2d_nt_fused_cs(x.to(dev), w.to(dev), rs.to(dev), cs.to(dev))
    assert_bits_equal(bits16(d), oi.epilogue_rowcolscale(ref_c, rs.numpy(), cs.numpy()), "C1 bf16")


# --------------------------------------------------------- rowwise quant ---

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K", [(33, 6144), (7, 100), (1, 256), (128, 300), (64, 16384),
                                 (8, 3072)])
def test_quant_rowwise_exact(dev, dtype, M, K):
    """tests/test_int8_linear_kernel.py:223-235 (seed 3, x*3)."""
    g = gen(3 + M + K)
    x = (torch.randn((M, K), generator=g) * 3).to(dtype)
    if M > 2:
        x[1] = 0.0
        x[2] = 1e-30 if dtype == torch.bfloat16 else 0.0
    q, s = ops.i8_quant_rowwise(x.to(dev))
    qr, sr = oi.quant_rowwise(bits16(x), "bf16" if dtype == torch.bfloat16 else "f16")
    assert_bits_equal(q.cpu().numpy(), qr, "q")
    assert_bits_equal(s.cpu().numpy().reshape(-1).view(np.uint32), sr.view(np.uint32), "scale")


def test_quant_rowwise_strided_and_offset(dev):
    """Row stride not a multiple of 8, and rows at a 2-byte offset: the
    2-byte path."""
    g = gen(9)
    x = (torch.randn(40, 1027, generator=g) * 3).to(torch.bfloat16)
    xs = x.to(dev)[:, :1024]
    q, s = ops.i8_quant_rowwise(xs)
    qr, sr = oi.quant_rowwise(bits16(x[:, :1024]), "bf16")
    assert_bits_equal(q.cpu().numpy(), qr, "strided q")
    flat = torch.empty(40 * 1024 + 1, dtype=torch.bfloat16, device=dev)
    xo = flat[1:].view(40, 1024)
    xo.copy_(x[:, :1024].to(dev))
    q, s = ops.i8_quant_rowwise(xo)
    assert_bits_equal(q.cpu().numpy(), qr, "offset q")
    assert_bits_equal(s.cpu().numpy().reshape(-1).view(np.uint32), sr.view(np.uint32), "scale")
    flat8 = torch.empty(40 * 1024 + 3, dtype=torch.bfloat16, device=dev)
    xf = flat8[3:].view(-1)
    xf.copy_(x[:, :1024].reshape(-1).to(dev))
    qf, sf = ops.fp8_quant_pertensor(xf)
    qfr, sfr = of.quant_pertensor(bits16(x[:, :1024].reshape(-1)))
    assert sf.item() == sfr
    assert_bits_equal(u8(qf), qfr, "fp8 quant offset")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_quant_rowwise_edges(dev, dtype):
    for x in (torch.zeros(4, 512), torch.full((4, 512), 1e-30)):
        x = x.to(dtype)
        q, s = ops.i8_quant_rowwise(x.to(dev))
        qr, sr = oi.quant_rowwise(bits16(x), "bf16" if dtype == torch.bfloat16 else "f16")
        assert_bits_equal(q.cpu().numpy(), qr, "edge q")
        assert_bits_equal(s.cpu().numpy().reshape(-1), sr, "edge scale")


# ------------------------------------------------------------ fp8 dequant ---

@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scale", [None, 1.0, 0.0123, 3.3e-4, 2.0 ** -5, 7.77])
def test_fp8_dequant_all_codes_exact(dev, out_dtype, scale):
    """All 256 codes (tests/test_scaled_mm_fp8.py:12-20), through the same
    conversion routine the W8A16 GEMM uses while staging weights."""
    codes = torch.arange(256, dtype=torch.uint8).repeat(5)[:1021]   # ragged tail too
    w = codes.view(torch.float8_e4m3fn)
    s = None if scale is None else torch.tensor([scale], dtype=torch.float32)
    out = ops.fp8_dequant(w.to(dev), s.to(dev) if s is not None else None, out_dtype)
    ref = of.dequant_pertensor(codes.numpy(), None if s is None else s.numpy()[0],
                               "bf16" if out_dtype == torch.bfloat16 else "f16")
    got = bits16(out)
    finite = (codes.numpy() & 0x7F) != 0x7F
    assert_bits_equal(got[finite], ref[finite], f"dequant scale={scale}")
    vals = bf16_bits_to_f32(got[~finite]) if out_dtype == torch.bfloat16 else f16_bits_to_f32(got[~finite])
    assert np.isnan(vals).all()


# ------------------------------------------------------------- fp8 quant ---

@pytest.mark.parametrize("shape,mult", [((16384 // 16, 5120 // 4), 1.0), ((333, 77), 40.0),
                                        ((1, 7), 1e-3)])
def test_fp8_quant_pertensor_exact(dev, shape, mult):
    g = gen(3)
    x = (torch.randn(shape, generator=g) * mult).to(torch.bfloat16)
    q, s = ops.fp8_quant_pertensor(x.to(dev))
    qr, sr = of.quant_pertensor(bits16(x))
    assert s.item() == sr
    assert_bits_equal(u8(q), qr, "fp8 quant")


@pytest.mark.parametrize("dtype,mult", [
    (torch.bfloat16, 1e-24),    # scale below 2^-80: the IEEE-divide path
    (torch.bfloat16, 3e-21),    # just above it: the reciprocal path
    (torch.bfloat16, 1e30),     # large scale
    (torch.bfloat16, 2e-38),    # subnormal-heavy bf16 input, IEEE path
    (torch.float16, 1.0),
    (torch.float16, 3e-5),      # f16 subnormals
    (torch.float16, 1e4),       # toward the f16 maximum (no infinities)
])
def test_fp8_quant_pertensor_scale_ranges(dev, dtype, mult):
    """Both quotient paths of the per-tensor fp8 quantizer (reciprocal step
    for 2^-80 <= scale <= 2^126, IEEE divide otherwise) against the oracle,
    bit-exact, with a ragged length for the scalar tail."""
    g = gen(31)
    x = (torch.randn(777, 301, generator=g) * mult).to(dtype)
    q, s = ops.fp8_quant_pertensor(x.to(dev))
    qr, sr = of.quant_pertensor(bits16(x), "bf16" if dtype == torch.bfloat16 else "f16")
    assert s.item() == sr
    assert_bits_equal(u8(q), qr, f"fp8 quant {dtype} x{mult}")


def test_fp8_quant_zero_tensor(dev):
    x = torch.zeros(64, 64, dtype=torch.bfloat16)
    q, s = ops.fp8_quant_pertensor(x.to(dev))
    assert s.item() == 1.0 and (u8(q) == 0).all()


# ------------------------------------------------------------ scaled_mm ---

def _fp8(t):
    return t.clamp(-448, 448).to(torch.float8_e4m3fn)


@pytest.mark.parametrize("M,K,N,out_dtype", [
    (64, 128, 32, torch.bfloat16), (64, 128, 32, torch.float32), (1024, 3072, 1280, torch.bfloat16),
    (333, 2048, 200, torch.bfloat16), (7, 96, 5, torch.float32), (512, 5120, 1024, torch.bfloat16),
])
def test_scaled_mm_vector_scales(dev, M, K, N, out_dtype):
    """tests/test_scaled_mm_fp8.py:57-80: rowwise scale_a [M,1], colwise
    scale_b [1,N], f32 bias."""
    g = gen(M + K + N)
    a = _fp8(torch.randn(M, K, generator=g) * 0.3)
    w = _fp8(torch.randn(N, K, generator=g) * 0.3)
    sa = torch.rand(M, 1, generator=g) + 0.5
    sb = torch.rand(1, N, generator=g) + 0.5
    bias = torch.randn(N, generator=g)
    out = ops.scaled_mm(a.to(dev), w.to(dev).t(), out_dtype=out_dtype, scale_a=sa.to(dev),
                        scale_b=sb.to(dev), bias=bias.to(dev))
    od = "bf16" if out_dtype == torch.bfloat16 else "f32"
    ref = of.scaled_mm(u8(a), u8(w), sa.numpy(), sb.numpy(), bias.numpy(), "f32", None, od)
    got = bf16_to_f32(bits16(out)) if od == "bf16" else out.cpu().numpy()
    ref = bf16_to_f32(ref) if od == "bf16" else ref
    # f32 outputs expose the accumulator itself: the gfx950 fp8 MFMA sums
    # with ~2^-18 relative error (measured), inside the reference's own 1e-3
    # bound for this route (tests/test_scaled_mm_fp8.py:76-78).
    tol = {} if od == "bf16" else dict(maxabs_rel=2.0 ** -14, rel_l2=2.0 ** -16)
    assert_close(got, ref, f"scaled_mm {M}x{K}x{N}", **tol)


def test_scaled_mm_pertensor_vs_torch_cpu(dev):
    """Per-tensor scales against CPU torch._scaled_mm itself."""
    g = gen(5)
    x = torch.randn(512, 5120, generator=g).to(torch.bfloat16)
    sa = x.float().abs().amax() / 448
    a = _fp8(x.float() / sa)
    wf = 0.02 * torch.randn(768, 5120, generator=g)
    sb = wf.abs().amax() / 448
    w = _fp8(wf / sb)
    ref = torch._scaled_mm(a, w.t(), scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)
    out = ops.scaled_mm(a.to(dev), w.to(dev).t(), out_dtype=torch.bfloat16, scale_a=sa.to(dev),
                        scale_b=sb.to(dev))
    assert_close(bf16_to_f32(bits16(out)), ref.float().numpy(), "scaled_mm vs torch CPU")


# fp8 GEMMs whose plan takes the 256x256 tile run the one-wave-per-SIMD
# kernel when K >= 5120 (C4Q_W4 forces either kernel; C4Q_TILE=0 forces the
# 256x256 tile for small shapes). Each output takes its K steps in the same
# order on both kernels: bits equal, and close to the oracle. Cases: whole
# tiles; ragged M and N with K % 128 = 80 and 16 (zero-filled K tail);
# vector and per-tensor scales; bias; bf16, f16 and f32 outputs; several
# tiles per workgroup (M x N beyond one round).
W4_CASES = [
    (512, 5120, 768, "tensor", torch.bfloat16, False, True),
    (700, 5200, 900, "vector", torch.bfloat16, True, True),
    (300, 6160, 260, "vector", torch.float32, True, True),
    (256, 1024, 512, "tensor", torch.float16, False, True),
    (1000, 2048, 1100, "vector", torch.bfloat16, True, True),
    (4352, 640, 4480, "tensor", torch.bfloat16, True, True),
]


@pytest.mark.parametrize("M,K,N,scales,out_dtype,with_bias,force_tile", W4_CASES)
def test_scaled_mm_one_wave_kernel(dev, monkeypatch, M, K, N, scales, out_dtype, with_bias,
                                   force_tile):
    g = gen(3 * M + K + N)
    a = _fp8(torch.randn(M, K, generator=g) * 0.3)
    w = _fp8(torch.randn(N, K, generator=g) * 0.3)
    if scales == "vector":
        sa, sb = torch.rand(M, 1, generator=g) + 0.5, torch.rand(1, N, generator=g) + 0.5
    else:
        sa, sb = torch.tensor(0.7), torch.tensor(1.3)
    bias = torch.randn(N, generator=g) if with_bias else None
    if force_tile:
        monkeypatch.setenv("C4Q_TILE", "0")
    ad, wd = a.to(dev), w.to(dev)

    def run(route):
        monkeypatch.setenv("C4Q_W4", route)
        out = ops.scaled_mm(ad, wd.t(), out_dtype=out_dtype, scale_a=sa.to(dev), scale_b=sb.to(dev),
                            bias=None if bias is None else bias.to(dev))
        return out.cpu()

    one_wave, eight_wave = run("1"), run("0")
    od = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[out_dtype]
    if od == "f32":
        assert np.array_equal(one_wave.numpy().view(np.uint32), eight_wave.numpy().view(np.uint32)), \
            f"one-wave vs 8-wave {M}x{K}x{N}"
        got = one_wave.numpy()
    else:
        assert_bits_equal(bits16(one_wave), bits16(eight_wave), f"one-wave vs 8-wave {M}x{K}x{N}")
        got = (bf16_to_f32 if od == "bf16" else f16_bits_to_f32)(bits16(one_wave))
    ref = of.scaled_mm(u8(a), u8(w), sa.numpy(), sb.numpy(),
                       None if bias is None else bias.numpy(), "f32", None, od)
    if od == "bf16":
        ref = bf16_to_f32(ref)
    elif od == "f16":
        ref = f16_bits_to_f32(ref)
    tol = {} if od != "f32" else dict(maxabs_rel=2.0 ** -14, rel_l2=2.0 ** -16)
    assert_close(got, ref, f"one-wave scaled_mm {M}x{K}x{N}", **tol)


# ---------------------------------------------------------------- W8A16 ---

@pytest.mark.parametrize("M,K,N,xdt,scaled,bias_dt", [
    (64, 512, 384, torch.bfloat16, False, torch.bfloat16),   # tests/test_linear_fp8_w8a16.py:132-156
    (257, 384, 512, torch.bfloat16, True, torch.float32),
    (1, 512, 512, torch.bfloat16, True, None),
    (96, 384, 512, torch.float16, False, torch.float32),
    (66, 3072, 700, torch.bfloat16, True, torch.bfloat16),
    (1024, 3072, 3072, torch.bfloat16, True, torch.bfloat16),
    (33, 100, 17, torch.bfloat16, True, torch.bfloat16),       # generic path (K % 16 != 0)
])
def test_w8a16_linear(dev, M, K, N, xdt, scaled, bias_dt):
    g = gen(2 + M + N)
    x = torch.randn(M, K, generator=g).to(xdt)
    wf = 0.02 * torch.randn(N, K, generator=g)
    ws = wf.abs().amax() / 448 if scaled else None
    w = _fp8(wf / ws) if scaled else _fp8(wf * 20)
    bias = (0.01 * torch.randn(N, generator=g)).to(bias_dt) if bias_dt is not None else None
    out = ops.w8a16_linear(x.to(dev), w.to(dev), ws.reshape(1).to(dev) if scaled else None,
                           bias.to(dev) if bias is not None else None)
    xd = "bf16" if xdt == torch.bfloat16 else "f16"
    bd = {torch.bfloat16: "bf16", torch.float32: "f32", None: "f32"}[bias_dt]
    braw = None if bias is None else (bits16(bias) if bias_dt == torch.bfloat16 else bias.numpy())
    ref = of.w8a16_linear(bits16(x), u8(w), ws.numpy() if scaled else None, braw, bd, xd, xd)
    tof = bf16_bits_to_f32 if xd == "bf16" else f16_bits_to_f32
    assert_close(tof(bits16(out)), tof(ref), f"w8a16 {M}x{K}x{N}")


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scale", [None, 0.0123, 2.0 ** -7, 3.7])
@pytest.mark.parametrize("M", [256, 8])
def test_w8a16_dequant_exact_every_code(dev, xdt, scale, M):
    """The in-register weight dequant, bit for bit: with an identity
    activation each output y[i, n] is the single product 1 * W'[n, i], exact
    in fp32 and in the output type, so y is the dequantized weight
    T(decode(w) * T(scale)) (comfykitchen_fp8.py:86-89) of every finite
    e4m3fn code. M = 256 takes the MFMA-tiled route, M = 8 the small-M one."""
    K = N = 256
    codes = (np.arange(N)[:, None] + np.arange(K)[None, :]) % 256
    codes[(codes & 0x7F) == 0x7F] = 0                     # the two NaN codes
    w = torch.from_numpy(codes.astype(np.uint8)).view(torch.float8_e4m3fn)
    x = torch.zeros(M, K, dtype=xdt)
    x[torch.arange(M), torch.arange(M)] = 1
    ws = None if scale is None else torch.tensor([scale], dtype=torch.float32)
    y = ops.w8a16_linear(x.to(dev), w.to(dev), None if ws is None else ws.to(dev))
    od = "bf16" if xdt == torch.bfloat16 else "f16"
    deq = of.dequant_pertensor(codes.astype(np.uint8), None if ws is None else ws.numpy(), od)
    want = np.ascontiguousarray(deq.T[:M])
    want[want == 0x8000] = 0      # -0 (code 0x80) plus the +0 products of the sum is +0
    assert_bits_equal(bits16(y), want, f"dequant {od} scale={scale} M={M}")


@pytest.mark.parametrize("M,K,N,xdt,scaled,bias_dt,out_dt", [
    (1, 3072, 3072, torch.bfloat16, True, torch.bfloat16, None),     # decode shapes (16 waves)
    (4, 3072, 8200, torch.bfloat16, True, torch.bfloat16, None),     # 8-wave split, ragged N
    (16, 3072, 3072, torch.bfloat16, False, None, None),
    (16, 1040, 17, torch.bfloat16, True, torch.float32, None),       # K tail inside a chunk
    (3, 24, 40, torch.bfloat16, True, torch.bfloat16, None),         # K < one chunk
    (7, 4160, 300, torch.float16, True, torch.float32, None),        # f16 activations
    (5, 3072, 260, torch.bfloat16, True, torch.bfloat16, torch.float32),
    (17, 3072, 512, torch.bfloat16, True, torch.bfloat16, None),     # two row groups, one row in the second
    (32, 3072, 3072, torch.bfloat16, True, torch.bfloat16, None),    # two full row groups
    (24, 3072, 18432, torch.bfloat16, True, torch.float32, None),    # two groups, several blocks per workgroup
    (32, 4096, 20000, torch.bfloat16, True, torch.bfloat16, None),   # two groups on the 16-wave variant
    (29, 1040, 17, torch.float16, False, torch.float16, None),       # two groups, K tail, f16, ragged N
    (20, 3000, 33333, torch.bfloat16, True, None, torch.float32),    # two groups, ragged K, f32 out
    (33, 3072, 512, torch.bfloat16, True, torch.bfloat16, None),     # two passes: 16 + 17 rows
    (48, 3072, 6000, torch.bfloat16, True, torch.float32, None),     # two passes of two groups
    (64, 1040, 17, torch.float16, False, torch.float16, None),       # two passes, K tail, f16
    (57, 3000, 12288, torch.bfloat16, True, None, torch.float32),    # two passes at the largest N, f32 out
    (40, 3072, 12289, torch.bfloat16, True, torch.bfloat16, None),   # N past the two-pass route: tiled
    (65, 3072, 512, torch.bfloat16, True, torch.bfloat16, None),     # first M past the small-M route
    (2, 4096, 96, torch.bfloat16, True, torch.bfloat16, None),       # largest K of the small-M route
    (2, 4112, 96, torch.bfloat16, True, torch.bfloat16, None),       # K past it: tiled route
    (16, 3072, 18432, torch.bfloat16, True, torch.bfloat16, None),   # several blocks per workgroup
    (2, 512, 100000, torch.bfloat16, True, torch.bfloat16, None),    # several reduction groups
    (16, 4096, 20000, torch.bfloat16, True, torch.float32, None),    # 16-wave variant, two groups
    (9, 3000, 33333, torch.float16, False, torch.bfloat16, None),    # ragged K and N, last group short
])
def test_w8a16_small_m(dev, M, K, N, xdt, scaled, bias_dt, out_dt):
    """Small-M (split-K) route against the oracle's dequant + fp32-accumulated
    linear, within the bf16 output tolerance."""
    g = gen(7 + M + K + N)
    x = torch.randn(M, K, generator=g).to(xdt)
    wf = 0.02 * torch.randn(N, K, generator=g)
    ws = wf.abs().amax() / 448 if scaled else None
    w = _fp8(wf / ws) if scaled else _fp8(wf * 20)
    bias = (0.01 * torch.randn(N, generator=g)).to(bias_dt) if bias_dt is not None else None
    out = ops.w8a16_linear(x.to(dev), w.to(dev), ws.reshape(1).to(dev) if scaled else None,
                           bias.to(dev) if bias is not None else None, out_dtype=out_dt)
    xd = "bf16" if xdt == torch.bfloat16 else "f16"
    bd = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32", None: "f32"}[bias_dt]
    braw = None if bias is None else (bias.numpy() if bias_dt == torch.float32 else bits16(bias))
    od = "f32" if out_dt == torch.float32 else xd
    ref = of.w8a16_linear(bits16(x), u8(w), ws.numpy() if scaled else None, braw, bd, xd, od)
    if od == "f32":
        assert_close(out.cpu().numpy(), ref, f"w8a16 small-M f32 {M}x{K}x{N}")
    else:
        tof = bf16_bits_to_f32 if xd == "bf16" else f16_bits_to_f32
        assert_close(tof(bits16(out)), tof(ref), f"w8a16 small-M {M}x{K}x{N}")


@pytest.mark.parametrize("M,K,N", [(128, 3072, 3072), (200, 3072, 1000), (65, 12288, 3072),
                                   (130, 1040, 2000)])
def test_w8a16_few_tiles_split_k_main(dev, monkeypatch, M, K, N):
    """Few-tile W8A16 GEMMs whose plan runs the split-K 64x64 tile as the main
    launch: against the oracle, and against the 64x128 tile (C4Q_TILE=5)
    within one bf16 ulp plus the fp32 reordering (the K groups sum in another
    order)."""
    info = _w8a16_plan(M, N, K)
    assert info[0] == 1 and info[1] == TILE_SPLIT_K, info.tolist()
    g = gen(3 * M + K + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    wf = 0.02 * torch.randn(N, K, generator=g)
    ws = (wf.abs().amax() / 448).reshape(1)
    w = _fp8(wf / ws)
    bias = (0.01 * torch.randn(N, generator=g)).to(torch.bfloat16)
    args = (x.to(dev), w.to(dev), ws.to(dev), bias.to(dev))
    y = bits16(ops.w8a16_linear(*args))
    ref = of.w8a16_linear(bits16(x), u8(w), ws.numpy(), bits16(bias))
    assert_close(bf16_to_f32(y), bf16_to_f32(ref), f"w8a16 split-K main {M}x{K}x{N}")
    monkeypatch.setenv("C4Q_TILE", "5")
    assert_reordered_sum_close(y, bits16(ops.w8a16_linear(*args)), "split-K main vs 64x128")


@pytest.mark.parametrize("M", [20, 50])    # one pass of two groups; two passes over the row halves
def test_w8a16_small_m_strided_output(dev, M):
    """Small-M route through the C ABI with padded activation and output rows
    (lda = K + 24, ldd = N + 8): the result equals the contiguous call's, and
    the padding columns keep their sentinel (the second pass of M > 32 writes
    its rows at M // 2 of the strided output)."""
    from cdna4q import _lib
    g = gen(31 + M)
    K, N = 3072, 1000
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    wf = 0.02 * torch.randn(N, K, generator=g)
    ws = (wf.abs().amax() / 448).reshape(1)
    w = _fp8(wf / ws)
    bias = (0.01 * torch.randn(N, generator=g)).to(torch.bfloat16)
    xd, wd, sd, bd = x.to(dev), w.to(dev), ws.to(dev), bias.to(dev)
    ref = ops.w8a16_linear(xd, wd, sd, bd)
    xp = torch.zeros(M, K + 24, dtype=torch.bfloat16, device=dev)
    xp[:, :K] = xd
    out = torch.full((M, N + 8), -7.0, dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    _lib.call("c4q_w8a16_gemm_nt", xp.data_ptr(), 0, K + 24, wd.view(torch.uint8).data_ptr(), K,
              sd.data_ptr(), out.data_ptr(), 0, N + 8, bd.data_ptr(), 0, None, M, N, K,
              torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize()
    assert_bits_equal(bits16(out[:, :N].contiguous()), bits16(ref), f"strided small-M M={M}")
    assert (out[:, N:].float() == -7.0).all(), "padding columns written"


@pytest.mark.parametrize("M", [4, 27, 50])    # one and two 16-row activation groups; two passes
def test_w8a16_small_m_gelu_table(dev, M):
    """Activation table on the small-M route: exact lookup of its own bf16 linear output."""
    g = gen(11)
    K, N = 3072, 1000
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    wf = 0.02 * torch.randn(N, K, generator=g)
    ws = (wf.abs().amax() / 448).reshape(1)
    w = _fp8(wf / ws)
    table = torch.from_numpy(oact.gelu_tanh_table().view(np.int16))
    lin = ops.w8a16_linear(x.to(dev), w.to(dev), ws.to(dev))
    act = ops.w8a16_linear(x.to(dev), w.to(dev), ws.to(dev), act_table=table.to(dev))
    assert_bits_equal(bits16(act), oact.apply_table(oact.gelu_tanh_table(), bits16(lin)), "gelu small-M")


def test_w8a16_gelu_table_exact_on_bf16_result(dev):
    """GELU-tanh epilogue = table lookup of the rounded bf16 linear output."""
    g = gen(5)
    M, K, N = 256, 3072, 768
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    wf = 0.02 * torch.randn(N, K, generator=g)
    ws = (wf.abs().amax() / 448).reshape(1)
    w = _fp8(wf / ws)
    table = torch.from_numpy(oact.gelu_tanh_table().view(np.int16))
    lin = ops.w8a16_linear(x.to(dev), w.to(dev), ws.to(dev))
    act = ops.w8a16_linear(x.to(dev), w.to(dev), ws.to(dev), act_table=table.to(dev))
    assert_bits_equal(bits16(act), oact.apply_table(oact.gelu_tanh_table(), bits16(lin)), "gelu")


# --------------------------------------------------------------- FFN pair ---

@pytest.mark.parametrize("M,K,N", [(129, 3072, 512), (256, 512, 384), (4095, 256, 256),
                                   (3, 129, 5), (1, 3072, 1024)])
def test_krea2_pair_exact(dev, M, K, N):
    g = gen(917 + M)
    q = _randint8((M, K), g, -127, 128)
    wg = _randint8((N, K), g, -127, 128)
    wu = _randint8((N, K), g, -127, 128)
    rs = torch.rand(M, generator=g) * 0.001
    gs = torch.rand(N, generator=g) * 0.005
    us = torch.rand(N, generator=g) * 0.005
    silu = torch.from_numpy(oact.silu_table().view(np.int16))
    out = ops.ffn_pair(q.to(dev), wg.to(dev), wu.to(dev), rs.to(dev), gs.to(dev), us.to(dev),
                       silu.to(dev), None)
    ref = op.krea2_pair(q.numpy(), wg.numpy(), wu.numpy(), rs.numpy(), gs.numpy(), us.numpy())
    assert_bits_equal(bits16(out), ref, f"krea2 pair {M}x{K}x{N}")


def test_moss_pair_exact(dev):
    """tests/test_moss_ffn_mps.py:38-55 (seed 917, M=129, [16384,3072] weight)."""
    g = gen(917)
    M, K, F2 = 129, 3072, 16384
    q = _randint8((M, K), g, -127, 128)
    w = _randint8((F2, K), g, -127, 128)
    rs = torch.rand(M, generator=g) * 0.001
    cs = torch.rand(F2, generator=g) * 0.005
    th, tg = (torch.from_numpy(t.view(np.int16)) for t in oact.situ_tables())
    f = F2 // 2
    wd = w.to(dev)
    csd = cs.to(dev)
    out = ops.ffn_pair(q.to(dev), wd[:f], wd[f:], rs.to(dev), csd[:f], csd[f:], th.to(dev),
                       tg.to(dev))
    ref = op.moss_pair(q.numpy(), w.numpy(), rs.numpy(), cs.numpy(), *oact.situ_tables())
    assert_bits_equal(bits16(out), ref, "moss pair")


# ---------------------------------------------------- every tile variant ---

@pytest.mark.parametrize("tile", [str(t) for t in range(8)])
def test_every_tile_variant(dev, monkeypatch, tile):
    """Force each MFMA tile variant (C4Q_TILE) on ragged shapes: INT8 fused
    epilogue and pair bit-exact, fp8 / W8A16 within tolerance."""
    monkeypatch.setenv("C4Q_TILE", tile)
    g = gen(100 + int(tile))
    M, K, N = 300, 1040, 520          # ragged M and N tails, K tail inside a 128-byte stage
    a, b = _randint8((M, K), g), _randint8((N, K), g)
    rs = torch.rand(M, generator=g) * 0.01
    cs = torch.rand(N, generator=g) * 0.02
    bb = torch.randn(N, generator=g).to(torch.bfloat16)
    c = ops.i8_matmul2d_nt(a.to(dev), b.to(dev))
    ref_c = oi.i8_matmul2d_nt(a.numpy(), b.numpy())
    assert_bits_equal(c.cpu().numpy(), ref_c, f"tile {tile} int32")
    d = ops.i8_matmul2d_nt_fused_cs(a.to(dev), b.to(dev), rs.to(dev), cs.to(dev), bb.to(dev))
    assert_bits_equal(bits16(d), oi.epilogue_rowcolscale(ref_c, rs.numpy(), cs.numpy(), bits16(bb)),
                      f"tile {tile} fused_cs")
    bh = bb.to(torch.float16)
    h = ops.i8_matmul2d_nt_fused_cs_half(a.to(dev), b.to(dev), rs.to(dev), cs.to(dev), bh.to(dev))
    assert_bits_equal(bits16(h), oi.epilogue_rowcolscale_half(ref_c, rs.numpy(), cs.numpy(),
                                                              bits16(bh)), f"tile {tile} fused_cs_half")
    xq = (torch.randint(-6, 7, (M, K), generator=g) * 0.25).to(torch.bfloat16)
    wq = (torch.randint(-6, 7, (2 * N, K), generator=g) * 0.25).to(torch.bfloat16)
    mp = ops.moss_bf16_pair(xq.to(dev), wq.to(dev), _moss_tables(dev))
    assert_bits_equal(bits16(mp), op.moss_bf16_pair(bits16(xq), bits16(wq), *oact.situ_tables()),
                      f"tile {tile} moss bf16 pair")
    wu = _randint8((N, K), g)
    us = torch.rand(N, generator=g) * 0.02
    silu = torch.from_numpy(oact.silu_table().view(np.int16))
    p = ops.ffn_pair(a.to(dev), b.to(dev), wu.to(dev), rs.to(dev), cs.to(dev), us.to(dev),
                     silu.to(dev), None)
    assert_bits_equal(bits16(p), op.krea2_pair(a.numpy(), b.numpy(), wu.numpy(), rs.numpy(),
                                               cs.numpy(), us.numpy()), f"tile {tile} pair")
    af = _fp8(torch.randn(M, K, generator=g))
    wf = _fp8(torch.randn(N, K, generator=g) * 0.1)
    sa, sb = torch.tensor(0.7), torch.tensor(1.3)
    o = ops.scaled_mm(af.to(dev), wf.to(dev).t(), out_dtype=torch.bfloat16, scale_a=sa.to(dev),
                      scale_b=sb.to(dev))
    ref = of.scaled_mm(u8(af), u8(wf), sa.numpy(), sb.numpy())
    assert_close(bf16_to_f32(bits16(o)), bf16_to_f32(ref), f"tile {tile} fp8")
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    ws = (wf.float().abs().amax() / 448).reshape(1)
    y = ops.w8a16_linear(x.to(dev), wf.to(dev), ws.to(dev), bb.to(dev))
    ref = of.w8a16_linear(bits16(x), u8(wf), ws.numpy(), bits16(bb))
    assert_close(bf16_to_f32(bits16(y)), bf16_to_f32(ref), f"tile {tile} w8a16")


# ------------------------------------------------- W8A16 224-row tile ---
# W8A16 GEMMs may run on 224 x 256 tiles (seven 32-row blocks per wave of
# the one-wave-per-SIMD kernel). Forced (C4Q_TILE=8) on ragged shapes, each
# output is checked against the oracle and, bit for bit, against the same
# GEMM on 256 x 256 tiles (C4Q_TILE=0): both accumulate every element's K
# products in the same order.

W8A16_224_CASES = [
    # M, K, N, x dtype, scaled, bias dtype, out dtype, GELU table
    (300, 1040, 520, torch.bfloat16, True, torch.bfloat16, None, False),    # ragged M, N, K tail
    (449, 3072, 700, torch.bfloat16, True, torch.bfloat16, None, True),     # last tile: one row
    (224, 3072, 3072, torch.bfloat16, False, torch.float32, None, False),   # one whole tile row
    (1000, 16, 256, torch.float16, True, None, None, False),                # one K step
    (672, 12288, 300, torch.bfloat16, True, torch.bfloat16, torch.float32, False),  # long K, f32 out
    (2100, 3072, 3072, torch.float16, False, torch.float16, None, False),   # several rounds
]


@pytest.mark.parametrize("M,K,N,xdt,scaled,bias_dt,out_dt,gelu", W8A16_224_CASES)
def test_w8a16_224_row_tile_exact(dev, monkeypatch, M, K, N, xdt, scaled, bias_dt, out_dt, gelu):
    g = gen(224 + M + K + N)
    x = torch.randn(M, K, generator=g).to(xdt)
    wf = 0.02 * torch.randn(N, K, generator=g)
    ws = wf.abs().amax() / 448 if scaled else None
    w = _fp8(wf / ws) if scaled else _fp8(wf * 20)
    bias = (0.01 * torch.randn(N, generator=g)).to(bias_dt) if bias_dt is not None else None
    table = ops.act_table("gelu_tanh", dev) if gelu else None
    xd_, wd_ = x.to(dev), w.to(dev)
    sd_ = ws.reshape(1).to(dev) if scaled else None
    bd_ = bias.to(dev) if bias is not None else None

    def run(tile):
        monkeypatch.setenv("C4Q_TILE", tile)
        return ops.w8a16_linear(xd_, wd_, sd_, bd_, out_dtype=out_dt, act_table=table).cpu()

    y224, y256 = run("8"), run("0")
    assert y224.dtype == y256.dtype and y224.shape == (M, N)
    assert torch.equal(y224.view(torch.int16) if y224.dtype != torch.float32 else y224.view(torch.int32),
                       y256.view(torch.int16) if y256.dtype != torch.float32 else y256.view(torch.int32)), \
        f"224-row tile != 256-row tile ({M}x{K}x{N})"
    xd = "bf16" if xdt == torch.bfloat16 else "f16"
    od = "f32" if out_dt == torch.float32 else xd
    bd = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32", None: "f32"}[bias_dt]
    braw = None if bias is None else (bias.numpy() if bias_dt == torch.float32 else bits16(bias))
    ref = of.w8a16_linear(bits16(x), u8(w), ws.numpy() if scaled else None, braw, bd, xd, od,
                          act="gelu_tanh" if gelu else None)
    if od == "f32":
        assert_close(y224.numpy(), ref, f"w8a16 224-row tile {M}x{K}x{N} f32")
        return
    tof = bf16_bits_to_f32 if xd == "bf16" else f16_bits_to_f32
    assert_close(tof(bits16(y224)), tof(ref), f"w8a16 224-row tile {M}x{K}x{N}")


# ------------------------------------------------------ split tile plans ---
# Shapes whose last round of 256x256 tiles would leave most CUs idle: the
# library runs the whole rounds as one launch and splits the leftover tiles
# into 64x128 or 128x128 pieces run by a second launch. Each case is checked
# against the oracle and, bit for bit, against the single-launch plan
# (C4Q_TILE=0): every output element accumulates its K products in the same
# order in every tile variant.

def _device_plan(M, n_rows_b, K):
    import ctypes, pathlib
    lib = ctypes.CDLL(str(pathlib.Path(__file__).resolve().parent / "native" / "libc4q_probe.so"))
    f = lib.c4q_probe_tile_plan
    f.argtypes = [ctypes.c_int64] * 3 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                         ctypes.c_void_p]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    cover = np.zeros(-(-M // 64) * -(-n_rows_b // 64), np.int32)
    info = np.zeros(8, np.int64)
    assert f(M, n_rows_b, K, cus, cover.ctypes.data, cover.size, info.ctypes.data) == 0
    if info[0] != 2:
        pytest.skip(f"no split plan for {M}x{n_rows_b} on {cus} CUs")
    return info


TILE_SPLIT_K = 7   # 64x64 pieces, K split over 4 wave groups


def _w8a16_plan(M, N, K):
    """The W8A16 tile set's plan on this device (info as in _device_plan)."""
    import ctypes, pathlib
    lib = ctypes.CDLL(str(pathlib.Path(__file__).resolve().parent / "native" / "libc4q_probe.so"))
    f = lib.c4q_probe_w8a16_tile_plan
    f.argtypes = [ctypes.c_int64] * 3 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                         ctypes.c_void_p]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    cover = np.zeros(-(-M // 32) * -(-N // 64), np.int32)
    info = np.zeros(8, np.int64)
    assert f(M, N, K, cus, cover.ctypes.data, cover.size, info.ctypes.data) == 0
    return info


def assert_reordered_sum_close(out, ref, what):
    """bf16 results of the same products summed in another fp32 order: equal
    up to the final rounding (one bf16 ulp, 2^-7 relative) plus the fp32
    reordering error, which matters only where the sum cancels."""
    o, r = bf16_to_f32(out).astype(np.float64), bf16_to_f32(ref).astype(np.float64)
    scale = np.abs(r).max() if r.size else 0.0
    bad = np.abs(o - r) > 2.0 ** -7 * np.abs(r) + 1e-5 * scale
    assert not bad.any(), f"{what}: {int(bad.sum())} elements differ by more than one ulp"


# 64x128, 64x128, 128x128, split-K 64x64 (ragged K), split-K 64x64 (ragged M, N, K) pieces
SPLIT_CASES = [(4352, 512, 4352), (4312, 1040, 4280), (4608, 1024, 4608), (4352, 1008, 4096),
               (4300, 1040, 4090)]


@pytest.mark.parametrize("M,K,N", SPLIT_CASES)
def test_split_plan_int8_exact(dev, monkeypatch, M, K, N):
    _device_plan(M, N, K)
    g = gen(M + K + N)
    a, b = _randint8((M, K), g), _randint8((N, K), g)
    rs = torch.rand(M, generator=g) * 0.01
    cs = torch.rand(N, generator=g) * 0.02
    bb = torch.randn(N, generator=g).to(torch.bfloat16)
    ad, bd = a.to(dev), b.to(dev)
    c = ops.i8_matmul2d_nt(ad, bd).cpu().numpy()
    d = bits16(ops.i8_matmul2d_nt_fused_cs(ad, bd, rs.to(dev), cs.to(dev), bb.to(dev)))
    ref_c = oi.i8_matmul2d_nt(a.numpy(), b.numpy())
    assert_bits_equal(c, ref_c, f"split int32 {M}x{K}x{N}")
    assert_bits_equal(d, oi.epilogue_rowcolscale(ref_c, rs.numpy(), cs.numpy(), bits16(bb)),
                      f"split fused_cs {M}x{K}x{N}")
    monkeypatch.setenv("C4Q_TILE", "0")
    d1 = bits16(ops.i8_matmul2d_nt_fused_cs(ad, bd, rs.to(dev), cs.to(dev), bb.to(dev)))
    assert_bits_equal(d, d1, "split plan vs one launch")


@pytest.mark.parametrize("N_out", [2176, 2048])    # 64x128 pieces, split-K 64x64 pieces
def test_split_plan_pair_exact(dev, monkeypatch, N_out):
    M, K = 4352, 512
    _device_plan(M, 2 * N_out, K)
    g = gen(77)
    a, wg, wu = _randint8((M, K), g), _randint8((N_out, K), g), _randint8((N_out, K), g)
    rs = torch.rand(M, generator=g) * 0.01
    gs = torch.rand(N_out, generator=g) * 0.02
    us = torch.rand(N_out, generator=g) * 0.02
    silu = torch.from_numpy(oact.silu_table().view(np.int16))
    args = (a.to(dev), wg.to(dev), wu.to(dev), rs.to(dev), gs.to(dev), us.to(dev), silu.to(dev), None)
    p = bits16(ops.ffn_pair(*args))
    assert_bits_equal(p, op.krea2_pair(a.numpy(), wg.numpy(), wu.numpy(), rs.numpy(), gs.numpy(),
                                       us.numpy()), "split pair")
    monkeypatch.setenv("C4Q_TILE", "0")
    assert_bits_equal(p, bits16(ops.ffn_pair(*args)), "split pair vs one launch")


@pytest.mark.parametrize("M,K,N", SPLIT_CASES)
def test_split_plan_fp8_and_w8a16(dev, monkeypatch, M, K, N):
    info = _device_plan(M, N, K)
    g = gen(5 * M + N)
    af = _fp8(torch.randn(M, K, generator=g))
    wf = _fp8(torch.randn(N, K, generator=g) * 0.1)
    sa, sb = torch.tensor(0.7), torch.tensor(1.3)
    bb = torch.randn(N, generator=g).to(torch.bfloat16)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    ws = (wf.float().abs().amax() / 448).reshape(1)
    afd, wfd, xd = af.to(dev), wf.to(dev), x.to(dev)

    def run():
        o = ops.scaled_mm(afd, wfd.t(), out_dtype=torch.bfloat16, scale_a=sa.to(dev),
                          scale_b=sb.to(dev))
        y = ops.w8a16_linear(xd, wfd, ws.to(dev), bb.to(dev))
        return bits16(o), bits16(y)

    o, y = run()
    assert_close(bf16_to_f32(o), bf16_to_f32(of.scaled_mm(u8(af), u8(wf), sa.numpy(), sb.numpy())),
                 f"split fp8 {M}x{K}x{N}")
    assert_close(bf16_to_f32(y), bf16_to_f32(of.w8a16_linear(bits16(x), u8(wf), ws.numpy(), bits16(bb))),
                 f"split w8a16 {M}x{K}x{N}")
    wi = _w8a16_plan(M, N, K)            # W8A16 plans over its own tile set
    monkeypatch.setenv("C4Q_TILE", "0")
    o1, y1 = run()
    if info[3] == TILE_SPLIT_K:
        assert_reordered_sum_close(o, o1, "split-K fp8 vs one launch")
    else:
        assert_bits_equal(o, o1, "split fp8 vs one launch")
    if TILE_SPLIT_K in (wi[1], wi[3] if wi[0] == 2 else -1):
        assert_reordered_sum_close(y, y1, "split-K w8a16 vs one launch")
    else:
        assert_bits_equal(y, y1, "split w8a16 vs one launch")


# Whole GEMMs forced through the split-K kernel: K shorter than one stage per
# group, K not a multiple of the stage, ragged M and N, several pieces per
# workgroup (M x N beyond one round of 64x64 pieces).
FORCED_SPLIT_K = [(64, 16, 64), (100, 80, 130), (257, 1008, 190), (1000, 2064, 700),
                  (2048, 256, 2112)]


@pytest.mark.parametrize("M,K,N", FORCED_SPLIT_K)
def test_forced_split_k_every_family(dev, monkeypatch, M, K, N):
    g = gen(11 * M + 7 * K + N)
    a, b = _randint8((M, K), g), _randint8((N, K), g)
    rs = torch.rand(M, generator=g) * 0.01
    cs = torch.rand(N, generator=g) * 0.02
    bb = torch.randn(N, generator=g).to(torch.bfloat16)
    af = _fp8(torch.randn(M, K, generator=g))
    wf = _fp8(torch.randn(N, K, generator=g) * 0.1)
    sa, sb = torch.tensor(0.7), torch.tensor(1.3)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    ws = (wf.float().abs().amax() / 448).reshape(1)
    ad, bd, afd, wfd, xd = a.to(dev), b.to(dev), af.to(dev), wf.to(dev), x.to(dev)

    def run():
        c = ops.i8_matmul2d_nt(ad, bd).cpu().numpy()
        d = bits16(ops.i8_matmul2d_nt_fused_cs(ad, bd, rs.to(dev), cs.to(dev), bb.to(dev)))
        o = bits16(ops.scaled_mm(afd, wfd.t(), out_dtype=torch.bfloat16, scale_a=sa.to(dev),
                                 scale_b=sb.to(dev)))
        y = bits16(ops.w8a16_linear(xd, wfd, ws.to(dev), bb.to(dev)))
        return c, d, o, y

    monkeypatch.setenv("C4Q_TILE", str(TILE_SPLIT_K))
    c, d, o, y = run()
    ref_c = oi.i8_matmul2d_nt(a.numpy(), b.numpy())
    assert_bits_equal(c, ref_c, f"split-K int32 {M}x{K}x{N}")
    assert_bits_equal(d, oi.epilogue_rowcolscale(ref_c, rs.numpy(), cs.numpy(), bits16(bb)),
                      f"split-K fused_cs {M}x{K}x{N}")
    assert_close(bf16_to_f32(o), bf16_to_f32(of.scaled_mm(u8(af), u8(wf), sa.numpy(), sb.numpy())),
                 f"split-K fp8 {M}x{K}x{N}")
    assert_close(bf16_to_f32(y), bf16_to_f32(of.w8a16_linear(bits16(x), u8(wf), ws.numpy(), bits16(bb))),
                 f"split-K w8a16 {M}x{K}x{N}")
    monkeypatch.setenv("C4Q_TILE", "0")
    c0, d0, o0, y0 = run()
    assert_bits_equal(d, d0, "split-K fused_cs vs 256x256")
    assert_reordered_sum_close(o, o0, "split-K fp8 vs 256x256")
    assert_reordered_sum_close(y, y0, "split-K w8a16 vs 256x256")


@pytest.mark.parametrize("M,K,N_out", [(100, 80, 96), (600, 1040, 200)])
def test_forced_split_k_pair(dev, monkeypatch, M, K, N_out):
    g = gen(3 * M + K + N_out)
    a, wg, wu = _randint8((M, K), g), _randint8((N_out, K), g), _randint8((N_out, K), g)
    rs = torch.rand(M, generator=g) * 0.01
    gs = torch.rand(N_out, generator=g) * 0.02
    us = torch.rand(N_out, generator=g) * 0.02
    silu = torch.from_numpy(oact.silu_table().view(np.int16))
    args = (a.to(dev), wg.to(dev), wu.to(dev), rs.to(dev), gs.to(dev), us.to(dev), silu.to(dev), None)
    monkeypatch.setenv("C4Q_TILE", str(TILE_SPLIT_K))
    p = bits16(ops.ffn_pair(*args))
    assert_bits_equal(p, op.krea2_pair(a.numpy(), wg.numpy(), wu.numpy(), rs.numpy(), gs.numpy(),
                                       us.numpy()), f"split-K pair {M}x{K}x{N_out}")
