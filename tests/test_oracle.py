"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

Every oracle function is checked against something that does not share its
code: torch CPU library routines (``torch._int_mm``, ``torch._scaled_mm``,
dtype casts, ``F.silu`` / ``F.gelu``), the golden fixtures of tests/golden/
(written from torch CPU by tests/golden/make_golden.py, never from the
oracle), closed forms and brute force. Each check is chosen so that a
plausible mistake fails it -- several tests plant such a mistake in a copy
of the oracle and assert that the same check rejects it.

The reference stores no known-answer vectors for this path (its kernels are
Metal and its tests need an M5 GPU), so these checks are the pin.
"""
import hashlib
import json
import pathlib

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import act as oact
from oracle import convrot as ocr
from oracle import fp8 as of
from oracle import int8 as oi
from oracle import pair as op
from oracle import qknorm as oqk
from oracle import torch_path as tp
from oracle.numerics import (bf16_bits_to_f32, e4m3fn_decode, e4m3fn_encode, f16_bits_to_f32,
                             f32_to_bf16_bits, f32_to_f16_bits)

GOLD = pathlib.Path(__file__).resolve().parent / "golden"


def tbits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def f32_sample(n=1 << 20, seed=0):
    """Random float32 bit patterns (all exponents) plus special values and
    round-to-nearest-even ties of the bf16 / f16 grids."""
    rng = np.random.default_rng(seed)
    u = rng.integers(0, 2 ** 32, size=n, dtype=np.uint64).astype(np.uint32)
    ties = (rng.integers(0, 2 ** 16, size=4096, dtype=np.uint64).astype(np.uint32) << 16) | 0x8000
    specials = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x7F7FFFFF, 0x00000001,
                         0x007FFFFF, 0x00800000, 0x3F808000, 0x3F818000, 0x477FE000, 0x477FF000],
                        dtype=np.uint32)
    return np.concatenate([u, ties, specials]).view(np.float32)


# ------------------------------------------------------------- numerics ---

def test_bf16_rounding_matches_torch():
    x = f32_sample()
    want = tbits(torch.from_numpy(x).to(torch.bfloat16))
    got = f32_to_bf16_bits(x)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.isnan(bf16_bits_to_f32(got[nan])).all()
    # a truncating conversion (the plausible mistake) disagrees with torch
    trunc = (x.view(np.uint32) >> 16).astype(np.uint16)
    assert (trunc[~nan] != want[~nan]).sum() > 1000


def test_f16_rounding_matches_torch():
    x = f32_sample(seed=1)
    x = x[np.isfinite(x)]
    want = tbits(torch.from_numpy(x).to(torch.float16))
    assert np.array_equal(f32_to_f16_bits(x), want)
    assert np.array_equal(f16_bits_to_f32(want), torch.from_numpy(want.view(np.int16)).view(
        torch.float16).float().numpy())


def test_e4m3fn_decode_all_codes_golden():
    g = np.load(GOLD / "fp8_e4m3fn.npz")
    got = e4m3fn_decode(np.arange(256, dtype=np.uint8))
    want = g["decode"]
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan) and nan.sum() == 2          # 0x7F, 0xFF
    assert np.array_equal(got[~nan], want[~nan])
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6


def test_e4m3fn_encode_golden_and_torch():
    g = np.load(GOLD / "fp8_e4m3fn.npz")
    got = e4m3fn_encode(g["x"])
    want = g["encode"]
    # NaN codes: torch yields 0x7F or 0xFF; compare as NaN-ness, the rest exactly
    gn, wn = (got & 0x7F) == 0x7F, (want & 0x7F) == 0x7F
    assert np.array_equal(gn, wn)
    assert np.array_equal(got[~gn], want[~wn])
    # saturating instead of NaN at |x| >= 480 (plausible mistake) is caught
    x = np.array([480.0, -1e6], dtype=np.float32)
    assert ((e4m3fn_encode(x) & 0x7F) == 0x7F).all()


# ----------------------------------------------------------------- INT8 ---

@pytest.mark.parametrize("M,K,N", [(3, 129, 5), (16, 4096, 32), (70, 1000, 33)])
def test_int_mm_matches_torch(M, K, N):
    g = torch.Generator().manual_seed(M)
    a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    b = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8)
    a[:, 0] = -128
    b[0, :] = -128                   # -128 * -128 corners (the int_mm canary's adversarial case)
    want = torch._int_mm(a, b).numpy() if M > 16 and K % 8 == 0 and N % 8 == 0 else \
        (a.long() @ b.long()).to(torch.int32).numpy()
    assert np.array_equal(oi.int_mm(a.numpy(), b.numpy()), want)
    assert np.array_equal(oi.i8_matmul2d_nt(a.numpy(), b.t().numpy()), want)


def test_c1_golden_digest():
    """Full C1 config (seed 1): INT32 product and per-channel epilogue
    against the digests of torch._int_mm and torch's eager epilogue."""
    d = json.loads((GOLD / "digests.json").read_text())
    g = torch.Generator().manual_seed(d["c1_seed"])
    M, K, N = 1024, 3072, 3072
    x = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    rs = 0.005 + 0.015 * torch.rand(M, generator=g)
    cs = 0.0005 + 0.0015 * torch.rand(N, generator=g)
    c = oi.i8_matmul2d_nt(x.numpy(), w.numpy())
    assert sha(c) == d["c1_int32_sha256"]
    e = oi.epilogue_rowcolscale(c, rs.numpy(), cs.numpy())
    assert sha(e.view(np.int16)) == d["c1_epilogue_bf16_sha256"]


def _epi_case(seed, M=64, N=96):
    g = torch.Generator().manual_seed(seed)
    c = torch.randint(-2 ** 24, 2 ** 24, (M, N), generator=g, dtype=torch.int32)
    rs = torch.rand(M, generator=g) * 0.01
    cs = torch.rand(N, generator=g) * 0.002
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    return c, rs, cs, bias


def test_epilogue_rowscale_matches_torch_eager():
    c, rs, _, bias = _epi_case(1)
    d = (c.float() * rs[:, None]).to(torch.bfloat16)
    assert np.array_equal(oi.epilogue_rowscale(c.numpy(), rs.numpy()), tbits(d))
    db = (d.float() + bias.float()).to(torch.bfloat16)        # second rounding (bias)
    assert np.array_equal(oi.epilogue_rowscale(c.numpy(), rs.numpy(), tbits(bias)), tbits(db))
    # one rounding instead of two (plausible mistake) differs somewhere
    one = (c.float() * rs[:, None] + bias.float()).to(torch.bfloat16)
    assert not np.array_equal(tbits(one), tbits(db))


def test_epilogue_rowcolscale_order_matches_torch_eager():
    # large enough that the other association order changes some bf16 results
    c, rs, cs, bias = _epi_case(2, 1024, 1024)
    want = (c.float() * (cs[None, :] * rs[:, None])).to(torch.bfloat16)   # scale product first
    assert np.array_equal(oi.epilogue_rowcolscale(c.numpy(), rs.numpy(), cs.numpy()), tbits(want))
    other = ((c.float() * cs[None, :]) * rs[:, None]).to(torch.bfloat16)  # the other order
    assert not np.array_equal(tbits(other), tbits(want))
    wb = (want.float() + bias.float()).to(torch.bfloat16)
    got = oi.epilogue_rowcolscale(c.numpy(), rs.numpy(), cs.numpy(), tbits(bias))
    assert np.array_equal(got, tbits(wb))


def test_epilogue_rowcolscale_half_matches_torch_eager():
    c, rs, cs, _ = _epi_case(21, 256, 512)
    cs = cs * torch.logspace(-5, 3, 512)          # results from fp16 subnormals to overflow
    bias = (torch.randn(512, generator=torch.Generator().manual_seed(22)) * 4).to(torch.float16)
    want = (c.float() * (cs[None, :] * rs[:, None])).to(torch.float16)
    got = oi.epilogue_rowcolscale_half(c.numpy(), rs.numpy(), cs.numpy())
    assert np.array_equal(got, tbits(want))
    wf = want.float()
    assert torch.isinf(wf).any() and ((wf != 0) & (wf.abs() < 2.0 ** -14)).any()
    wb = (want.float() + bias.float()).to(torch.float16)      # second rounding (bias)
    got_b = oi.epilogue_rowcolscale_half(c.numpy(), rs.numpy(), cs.numpy(), tbits(bias))
    assert np.array_equal(got_b, tbits(wb))
    # one rounding instead of two, and a bf16 first rounding, each differ somewhere
    one = (c.float() * (cs[None, :] * rs[:, None]) + bias.float()).to(torch.float16)
    assert not np.array_equal(tbits(one), tbits(wb))
    via_bf16 = ((c.float() * (cs[None, :] * rs[:, None])).to(torch.bfloat16).float()
                + bias.float()).to(torch.float16)
    assert not np.array_equal(tbits(via_bf16), tbits(wb))


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_quant_rowwise_golden_edges(dt):
    g = np.load(GOLD / "quant_rowwise.npz")
    q, s = oi.quant_rowwise(g[f"x_{dt}"], dt)
    assert np.array_equal(q, g[f"q_{dt}"])
    assert np.array_equal(s.view(np.uint32), g[f"scale_{dt}"].view(np.uint32))


def _torch_quant(x):
    dt = x.dtype
    xf = x.float()
    scale = torch.clamp(xf.abs().amax(dim=1) / 127.0, min=1e-30)
    s = scale.to(dt)
    s = torch.where(s == 0, torch.full_like(s, torch.finfo(dt).tiny), s)
    q = torch.clamp(torch.round((xf / s.float()[:, None]).to(dt).float()), -128, 127).to(torch.int8)
    return q.numpy(), scale.numpy()


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_quant_rowwise_random_matches_torch(dt):
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(300, 513, generator=g) * torch.logspace(-3, 3, 300)[:, None]).to(dt)
    q, s = oi.quant_rowwise(tbits(x), "bf16" if dt == torch.bfloat16 else "f16")
    tq, ts = _torch_quant(x)
    assert np.array_equal(q, tq) and np.array_equal(s, ts)
    # property: the row maximum lands within one step of the int8 range edge
    # (the bf16-rounded scale is within 2^-9 of amax/127: 126 .. 128 reachable)
    row_max = np.abs(q.astype(np.int32)).max(axis=1)
    assert ((row_max >= 126) & (row_max <= 128)).all()


def test_int8_linear_equals_its_parts():
    g = torch.Generator().manual_seed(6)
    x = torch.randn(20, 256, generator=g).to(torch.bfloat16)
    w = torch.randint(-127, 128, (48, 256), generator=g, dtype=torch.int8)
    ws = torch.rand(48, generator=g) * 0.01
    q, xs = _torch_quant(x)
    c = torch._int_mm(torch.from_numpy(q), w.t())
    want = (c.float() * (ws[None, :] * torch.from_numpy(xs)[:, None])).to(torch.bfloat16)
    assert np.array_equal(oi.int8_linear(tbits(x), w.numpy(), ws.numpy()), tbits(want))
    wt = torch.tensor([0.004])
    want = (c.float() * (wt * torch.from_numpy(xs))[:, None]).to(torch.bfloat16)
    assert np.array_equal(oi.int8_linear(tbits(x), w.numpy(), wt.numpy()), tbits(want))


# ------------------------------------------------------------------ FP8 ---

def test_scaled_mm_golden_torch():
    """torch._scaled_mm (CPU) rounds the fp32 product once after the scales;
    the oracle rounds the exactly-rounded fp32 dot product, so they agree up
    to one bf16 rounding step of an fp32 accumulation-order difference."""
    g = np.load(GOLD / "scaled_mm.npz")
    got = of.scaled_mm(g["a"], g["w"], g["sa"], g["sb"])
    want = g["y"]
    gf, wf = bf16_bits_to_f32(got), bf16_bits_to_f32(want)
    assert (got == want).mean() > 0.99
    ulp = np.abs(wf) * 2.0 ** -7
    assert (np.abs(gf - wf) <= ulp + 1e-30).all()


def test_scaled_mm_scale_order_and_vectors():
    """out = ((acc * sa) * sb) * sr + bias, in f32, one final rounding: a
    closed-form fp64 -> f32 restatement with vector scales."""
    rng = np.random.default_rng(7)
    a = e4m3fn_encode((rng.standard_normal((8, 64)) * 4).astype(np.float32))
    w = e4m3fn_encode((rng.standard_normal((5, 64)) * 4).astype(np.float32))
    sa = rng.random(8).astype(np.float32)
    sb = rng.random(5).astype(np.float32)
    sr = np.float32(0.37)
    bias = (rng.standard_normal(5)).astype(np.float32)
    acc = (e4m3fn_decode(a).astype(np.float64) @ e4m3fn_decode(w).astype(np.float64).T).astype(np.float32)
    want = ((acc * sa[:, None]) * sb[None, :]) * sr + bias[None, :]
    got = of.scaled_mm(a, w, sa, sb, bias, "f32", sr, "f32")
    assert np.array_equal(got, want.astype(np.float32))


def test_quant_pertensor_matches_torch():
    g = torch.Generator().manual_seed(8)
    x = (torch.randn(64, 333, generator=g) * 7).to(torch.bfloat16)
    codes, scale = of.quant_pertensor(tbits(x))
    s = x.float().abs().amax() / 448
    q = (x.float() / s).clamp(-448, 448).to(torch.float8_e4m3fn)
    assert np.float32(scale) == s.item()
    assert np.array_equal(codes, q.view(torch.uint8).numpy())
    z, zs = of.quant_pertensor(np.zeros((2, 3), dtype=np.uint16))
    assert zs == 1.0 and not z.any()


@pytest.mark.parametrize("scale", [None, 0.0123, 3.0e-5, 17.5])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_dequant_matches_kitchen_formula(scale, dt):
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    codes = codes[(codes & 0x7F) != 0x7F]                      # finite codes
    w = codes.view(torch.float8_e4m3fn)
    want = w.to(tdt) if scale is None else w.to(tdt) * torch.tensor(scale).to(tdt)
    got = of.dequant_pertensor(codes.numpy(), scale, dt)
    assert np.array_equal(got, tbits(want))


def test_w8a16_linear_closed_form():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(24, 256, generator=g).to(torch.bfloat16)
    wf = 0.02 * torch.randn(40, 256, generator=g)
    ws = wf.abs().amax() / 448
    w = (wf / ws).clamp(-448, 448).to(torch.float8_e4m3fn)
    bias = (0.01 * torch.randn(40, generator=g)).to(torch.bfloat16)
    wd = w.to(torch.bfloat16) * ws.to(torch.bfloat16)           # kitchen dequant
    # exactly-rounded fp32 dot product, then the f32 bias add (two roundings)
    want = (x.double() @ wd.double().t()).float() + bias.float()
    got = of.w8a16_linear(tbits(x), w.view(torch.uint8).numpy(), ws.reshape(1).numpy(), tbits(bias),
                          "bf16", "bf16", "f32")
    assert np.array_equal(got, want.numpy())
    out = of.w8a16_linear(tbits(x), w.view(torch.uint8).numpy(), ws.reshape(1).numpy(), tbits(bias))
    assert np.array_equal(out, f32_to_bf16_bits(got))


# ---------------------------------------------------- activations, pairs ---

def test_activation_tables_digests():
    d = json.loads((GOLD / "digests.json").read_text())
    assert sha(oact.silu_table().view(np.int16)) == d["silu_sha256"]
    assert sha(oact.gelu_tanh_table().view(np.int16)) == d["gelu_tanh_sha256"]
    th, tg = oact.situ_tables()
    assert sha(th.view(np.int16)) == d["situ_h_sha256"]
    assert sha(tg.view(np.int16)) == d["situ_g_sha256"]
    v = torch.randn(5000).to(torch.bfloat16)
    assert np.array_equal(oact.apply_table(oact.silu_table(), tbits(v)), tbits(F.silu(v)))


def _pair_case(seed, M=40, K=128, N=48):
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    wg = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    wu = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    rs = torch.rand(M, generator=g) * 0.01
    gs = torch.rand(N, generator=g) * 0.02
    us = torch.rand(N, generator=g) * 0.02
    return q, wg, wu, rs, gs, us


def test_krea2_pair_is_the_unfused_torch_chain():
    q, wg, wu, rs, gs, us = _pair_case(10)
    want = tp.c4_ffn_pair(q, wg, wu, rs, gs, us)       # two eager epilogues, F.silu, * (bf16)
    got = op.krea2_pair(q.numpy(), wg.numpy(), wu.numpy(), rs.numpy(), gs.numpy(), us.numpy())
    assert np.array_equal(got, tbits(want))


def test_moss_pair_is_the_unfused_torch_chain():
    q, wg, wu, rs, gs, us = _pair_case(11)
    w = torch.cat([wg, wu])
    cs = torch.cat([gs, us])
    h = tp.c1_int8_linear(q, wg, rs, gs)
    gg = tp.c1_int8_linear(q, wu, rs, us)
    want = (25.0 * torch.tanh(h / 25.0)) * (4.0 * torch.tanh(gg / 4.0) * torch.sigmoid(gg))
    th, tg = oact.situ_tables()
    got = op.moss_pair(q.numpy(), w.numpy(), rs.numpy(), cs.numpy(), th, tg)
    assert np.array_equal(got, tbits(want))


def _situ(h, g):
    return (25.0 * torch.tanh(h / 25.0)) * (4.0 * torch.tanh(g / 4.0) * torch.sigmoid(g))


def test_moss_bf16_pair_is_the_unfused_torch_chain():
    """Integer-valued bf16 operands (multiples of 1/4): every fp32 sum is
    exact in any order, so torch's CPU bf16 linear is exact and the chain
    linear -> SiTU (bf16 ops) must match bit for bit."""
    g = torch.Generator().manual_seed(31)
    M, K, F_ = 40, 384, 72
    x = (torch.randint(-6, 7, (M, K), generator=g) * 0.25).to(torch.bfloat16)
    w = (torch.randint(-6, 7, (2 * F_, K), generator=g) * 0.25).to(torch.bfloat16)
    wh, wg = w.chunk(2, dim=0)
    want = _situ(F.linear(x, wh), F.linear(x, wg))
    th, tg = oact.situ_tables()
    got = op.moss_bf16_pair(tbits(x), tbits(w), th, tg)
    assert np.array_equal(got, tbits(want))
    # swapped halves or swapped tables (plausible mistakes) differ
    assert not np.array_equal(op.moss_bf16_pair(tbits(x), tbits(torch.cat([wg, wh])), th, tg), got)
    assert not np.array_equal(op.moss_bf16_pair(tbits(x), tbits(w), tg, th), got)


def test_moss_bf16_pair_random_within_one_rounding_of_torch():
    """Random operands: torch's fp32 summation order differs from the exact
    sum, so h / g may differ by one bf16 ulp; the outputs then agree to the
    slope of SiTU times that ulp."""
    g = torch.Generator().manual_seed(32)
    x = torch.randn(32, 512, generator=g).to(torch.bfloat16)
    w = (0.05 * torch.randn(160, 512, generator=g)).to(torch.bfloat16)
    wh, wg = w.chunk(2, dim=0)
    want = bf16_bits_to_f32(tbits(_situ(F.linear(x, wh), F.linear(x, wg))))
    th, tg = oact.situ_tables()
    got = bf16_bits_to_f32(op.moss_bf16_pair(tbits(x), tbits(w), th, tg))
    scale = np.abs(want).max()
    assert (np.abs(got - want) <= 2.0 ** -6 * np.abs(want) + 2.0 ** -9 * scale).all()
    assert (got == want).mean() > 0.9


def test_cpu_baseline_paths_compute_the_oracle_results():
    """The timed CPU baseline (oracle/torch_path.py) computes what the oracle
    does: C1 exactly, C2 within one bf16 rounding of an fp32-order change."""
    g = torch.Generator().manual_seed(12)
    x = torch.randint(-127, 128, (32, 256), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (64, 256), generator=g, dtype=torch.int8)
    rs, cs = torch.rand(32, generator=g) * 0.01, torch.rand(64, generator=g) * 0.002
    want = oi.epilogue_rowcolscale(oi.i8_matmul2d_nt(x.numpy(), w.numpy()), rs.numpy(), cs.numpy())
    assert np.array_equal(tbits(tp.c1_int8_linear(x, w, rs, cs)), want)
    xb = torch.randn(16, 256, generator=g).to(torch.bfloat16)
    wf = 0.02 * torch.randn(48, 256, generator=g)
    ws = wf.abs().amax() / 448
    wq = (wf / ws).clamp(-448, 448).to(torch.float8_e4m3fn)
    b = (0.01 * torch.randn(48, generator=g)).to(torch.bfloat16)
    cpu = bf16_bits_to_f32(tbits(tp.c2_w8a16_linear(xb, wq, ws, b)))
    ref = bf16_bits_to_f32(of.w8a16_linear(tbits(xb), wq.view(torch.uint8).numpy(),
                                           ws.reshape(1).numpy(), tbits(b)))
    assert (np.abs(cpu - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-30).all()


# ----------------------------------------------------------- ConvRot ---

def _h256():
    h = ocr.H4
    return np.kron(h, np.kron(h, np.kron(h, h)))


def test_h4_is_a_symmetric_hadamard_matrix():
    h = _h256()
    assert np.array_equal(ocr.H4, ocr.H4.T)
    assert np.array_equal(h @ h.T, 256 * np.eye(256, dtype=np.int64))


def test_fwht256_unit_vectors_give_the_kronecker_rows():
    """One nonzero input: every sum is exact, so each output row must equal
    the Kronecker power of H4 exactly (pins the stage strides, the digit
    order and the H4 rows; the Sylvester H4 fails this)."""
    got = ocr.fwht256(np.eye(256, dtype=np.float32))
    assert np.array_equal(got.astype(np.int64), _h256())
    sylv = np.array([[1, 1, 1, 1], [1, -1, 1, -1], [1, 1, -1, -1], [1, -1, -1, 1]])
    assert not np.array_equal(np.kron(sylv, np.kron(sylv, np.kron(sylv, sylv))), _h256())


def test_fwht256_random_is_the_matmul_within_fp32_rounding():
    rng = np.random.default_rng(3)
    v = rng.standard_normal((64, 256)).astype(np.float32)
    exact = v.astype(np.float64) @ _h256().T.astype(np.float64)
    got = ocr.fwht256(v)
    assert np.abs(got - exact).max() <= 1e-5 * np.abs(exact).max()
    # the butterfly order is observable: another association differs somewhere
    w = v.copy()
    idx = np.arange(256)
    for stride in (1, 4, 16, 64):
        digit = (idx // stride) % 4
        base = idx - digit * stride
        a = [w[:, base + k * stride] for k in range(4)]
        sgn = ocr.H4[digit]
        w = (a[0] * sgn[:, 0]).astype(np.float32) + ((a[1] * sgn[:, 1]) + ((a[2] * sgn[:, 2]) + (a[3] * sgn[:, 3])))
    assert not np.array_equal(w.astype(np.float32), got)


def test_merge_heads_is_the_torch_permute():
    g = torch.Generator().manual_seed(40)
    x = torch.randn(2, 3, 5, 128, generator=g).to(torch.bfloat16)
    want = x.permute(0, 2, 1, 3).reshape(10, 384)
    assert np.array_equal(ocr.merge_heads(tbits(x)), tbits(want))


def test_merge_rot_quant_unrotated_is_rowwise_quant_of_the_merge():
    g = torch.Generator().manual_seed(41)
    x = torch.randn(1, 4, 7, 64, generator=g).to(torch.bfloat16)
    q, s = ocr.merge_rot_quant(tbits(x), rotate=False)
    q2, s2 = _torch_quant(x.permute(0, 2, 1, 3).reshape(7, 256))
    assert np.array_equal(q, q2) and np.array_equal(s.reshape(-1), s2.reshape(-1))


def test_swiglu_rot_is_torch_swiglu_then_the_rotation():
    g = torch.Generator().manual_seed(42)
    x = (torch.randn(6, 1024, generator=g) * 3).to(torch.bfloat16)
    act = F.silu(x[:, :512]) * x[:, 512:]                      # bf16 ops, torch CPU
    got = ocr.swiglu_rot(tbits(x), oact.silu_table())
    assert np.array_equal(got, ocr.rotate_bf16(tbits(act)))
    # gate and up swapped (a plausible mistake) differs
    xs = torch.cat([x[:, 512:], x[:, :512]], dim=1)
    assert not np.array_equal(ocr.swiglu_rot(tbits(xs), oact.silu_table()), got)


def test_scatter_qkv_is_the_torch_split_and_head_transpose():
    g = torch.Generator().manual_seed(45)
    m, h, d = 5, 3, 8
    y = torch.randn(m, 3 * h * d, generator=g).to(torch.bfloat16)
    q, k, v = y.split(h * d, dim=1)
    want = [t.reshape(m, h, d).transpose(0, 1).unsqueeze(0).contiguous() for t in (q, k, v)]
    got = oi.scatter_qkv(tbits(y), h, d)
    for a, b in zip(got, want):
        assert np.array_equal(a, tbits(b))


@pytest.mark.parametrize("scale", [1.0, 0.3, 0.0123, 5.7])
def test_lora_delta_add_is_torch_bf16_mul_then_add(scale):
    """The runtime-LoRA term against torch's CPU bf16 ops, which round each
    operation: value + delta * bf16(scale)."""
    g = torch.Generator().manual_seed(46)
    base = (torch.randn(64, 96, generator=g) * 4).to(torch.bfloat16)
    delta = (torch.randn(64, 96, generator=g) * 0.05).to(torch.bfloat16)
    base[0, :4] = torch.tensor([0.0, -0.0, 3.0e38, -1.0e-40]).to(torch.bfloat16)
    ls = torch.tensor(scale, dtype=torch.float32).to(torch.bfloat16)
    want = base + delta * ls
    got = oi.lora_delta_add(tbits(base), tbits(delta), scale)
    assert np.array_equal(got, tbits(want))


def test_lora_delta_add_rounds_the_scaled_delta_and_the_scale():
    """Dropping either intermediate rounding (the bf16 scale, the bf16
    scaled delta) changes some outputs, so the pin above sees both."""
    g = torch.Generator().manual_seed(47)
    base = (torch.randn(4096, generator=g) * 4).to(torch.bfloat16)
    delta = (torch.randn(4096, generator=g) * 0.5).to(torch.bfloat16)
    got = oi.lora_delta_add(tbits(base), tbits(delta), 0.3)
    fused = (base.float() + delta.float() * torch.tensor(0.3).to(torch.bfloat16).float()).to(
        torch.bfloat16)
    raw_scale = (base.float() + (delta.float() * 0.3).to(torch.bfloat16).float()).to(torch.bfloat16)
    assert not np.array_equal(got, tbits(fused))
    assert not np.array_equal(got, tbits(raw_scale))


def test_scatter_part_is_the_torch_head_transpose():
    g = torch.Generator().manual_seed(48)
    m, h, d = 5, 3, 8
    y = torch.randn(m, h * d, generator=g).to(torch.bfloat16)
    want = y.reshape(m, h, d).transpose(0, 1).unsqueeze(0).contiguous()
    assert np.array_equal(oi.scatter_part(tbits(y), h, d), tbits(want))


# ------------------------------------------------ Q/K RMSNorm + RoPE (H3) ---

def _qk_inputs(seed, rows=37, heads=2, pairs=48):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(1, heads, rows, 128, generator=g) * 2).to(torch.bfloat16)
    freqs = torch.randn(rows, pairs, 2, 2, generator=g).to(torch.bfloat16)
    w = (1 + torch.randn(128, generator=g) * 0.1).float()
    return x, freqs, w


def test_qknorm_sum_order_is_a_permutation_of_all_columns():
    cols = sorted(c for j in range(8) for c in oqk.lane_columns(j))
    assert cols == list(range(128))


def test_qknorm_sum_of_squares_close_to_exact():
    """The fixed fp32 order vs the float64 sum: 16 sequential adds plus 3
    tree levels bound the relative error by 19 * 2^-24; a dropped or doubled
    column moves it by far more."""
    x, _, _ = _qk_inputs(51, rows=300)
    xf = x.float().numpy()
    exact = (xf.astype(np.float64) ** 2).sum(-1)
    got = oqk.sum_squares(xf).astype(np.float64)
    assert np.max(np.abs(got - exact) / exact) <= 19 * 2.0 ** -24
    bad = xf.copy()
    bad[..., 127] = 0
    assert np.max(np.abs(oqk.sum_squares(bad) - exact) / exact) > 1e-4


def test_qknorm_rms_against_torch_rms_norm():
    """Against torch's F.rms_norm in fp32 (its own sum order), then bf16:
    at most 1 bf16 ulp apart, and almost everywhere equal."""
    x, _, w = _qk_inputs(52, rows=400)
    got = oqk.rms_norm(tbits(x), w.numpy(), 1e-6)
    want = F.rms_norm(x.float(), (128,), w, eps=1e-6).to(torch.bfloat16).float().numpy()
    ulp = np.abs(tbits(torch.from_numpy(got).to(torch.bfloat16)).astype(np.int32)
                 - tbits(torch.from_numpy(want).to(torch.bfloat16)).astype(np.int32))
    assert ulp.max() <= 1
    assert (ulp != 0).mean() < 0.01
    # the weight on the wrong side of the rounding, or a missing eps, fails
    assert not np.array_equal(oqk.rms_norm(tbits(x), np.ones(128, np.float32), 1e-6), got)


def test_qknorm_eps_dominates_tiny_rows():
    """A zero row stays zero; a tiny row is scaled by 1/sqrt(eps)."""
    x = torch.zeros(1, 1, 2, 128, dtype=torch.bfloat16)
    x[0, 0, 1, 0] = 2.0 ** -20
    y = oqk.rms_norm(tbits(x), np.ones(128, np.float32), 1e-6)
    assert np.all(y[0, 0, 0] == 0)
    want = np.float32(2.0 ** -20) / np.sqrt(np.float32(2.0 ** -40 / 128 + 1e-6).astype(np.float32))
    assert y[0, 0, 1, 0] == bf16_bits_to_f32(f32_to_bf16_bits(np.float32(want)))


def test_rope_split_half_matches_torch_eager_form():
    """comfy_kitchen's eager form on torch CPU bf16 tensors: out = y * diag;
    out.addcmul_(partner, off) -- bit-exact."""
    x, freqs, w = _qk_inputs(53, rows=64, pairs=48)
    y = torch.from_numpy(oqk.rms_norm(tbits(x), w.numpy(), 1e-6)).to(torch.bfloat16)
    R = 48
    f = freqs                                   # [M, R, 2, 2]
    y0, y1 = y[..., :R], y[..., R:2 * R]
    o0 = y0 * f[:, :, 0, 0]
    o0.addcmul_(y1, f[:, :, 0, 1])
    o1 = y1 * f[:, :, 1, 1]
    o1.addcmul_(y0, f[:, :, 1, 0])
    want = torch.cat([o0, o1, y[..., 2 * R:]], dim=-1)
    got = oqk.rope_split_half(y.float().numpy(), tbits(freqs), 64)
    assert np.array_equal(got, tbits(want))


def test_rope_closed_forms_pin_partner_and_row():
    """Swap matrices [[0,1],[1,0]] exchange the halves exactly; a quarter
    turn [[0,-1],[1,0]] gives (-y1, y0); identity keeps y; columns past 2R
    are untouched."""
    g = torch.Generator().manual_seed(54)
    M, R = 5, 20
    y = torch.randn(1, 3, M, 128, generator=g).to(torch.bfloat16).float()
    yn = y.numpy()

    def run(mat):
        f = torch.tensor(mat, dtype=torch.bfloat16).expand(M, R, 2, 2).contiguous()
        return bf16_bits_to_f32(oqk.rope_split_half(yn, tbits(f), M))

    sw = run([[0.0, 1.0], [1.0, 0.0]])
    assert np.array_equal(sw[..., :R], yn[..., R:2 * R]) and np.array_equal(sw[..., R:2 * R], yn[..., :R])
    qt = run([[0.0, -1.0], [1.0, 0.0]])
    assert np.array_equal(qt[..., :R], -yn[..., R:2 * R]) and np.array_equal(qt[..., R:2 * R], yn[..., :R])
    ident = run([[1.0, 0.0], [0.0, 1.0]])
    assert np.array_equal(ident, yn)
    assert np.array_equal(sw[..., 2 * R:], yn[..., 2 * R:])


def test_rope_rotation_preserves_pair_norm():
    """cos/sin rotation matrices: |(out_i, out_{i+R})| = |(y_i, y_{i+R})| up
    to bf16 rounding of the inputs and outputs."""
    g = torch.Generator().manual_seed(55)
    M, R = 16, 48
    y = torch.randn(1, 2, M, 128, generator=g).to(torch.bfloat16).float()
    th = torch.rand(M, R, generator=g) * 6.28
    f = torch.stack([torch.stack([th.cos(), -th.sin()], -1), torch.stack([th.sin(), th.cos()], -1)], -2)
    out = bf16_bits_to_f32(oqk.rope_split_half(y.numpy(), tbits(f.to(torch.bfloat16)), M))
    n_in = np.hypot(y.numpy()[..., :R], y.numpy()[..., R:2 * R])
    n_out = np.hypot(out[..., :R], out[..., R:2 * R])
    assert np.allclose(n_out, n_in, rtol=3e-2, atol=1e-2)


def test_qkv_rms_rope_keeps_v_and_uses_each_weight():
    x, freqs, w = _qk_inputs(56, rows=9)
    q, k, v = oqk.qkv_rms_rope(tbits(x), tbits(x), tbits(x), tbits(freqs), w.numpy(),
                               np.ones(128, np.float32), 1e-6)
    assert np.array_equal(v, tbits(x))
    assert np.array_equal(q, oqk.qk_rms_rope(tbits(x), tbits(freqs), w.numpy(), 1e-6))
    assert not np.array_equal(q, k)
