"""Writes the golden fixtures of tests/golden/ from torch CPU library routines
only (never from the oracle), so that tests/test_oracle.py can pin the
oracle against them:

  fp8_e4m3fn.npz      decode of all 256 codes (torch cast to float32) and the
                      torch e4m3fn encode of rounding-edge and random float32s
  quant_rowwise.npz   edge rows (zeros, 1e-30, tiny, huge, all-equal, exact
                      halves, +-127*s boundaries) through the comfy_kitchen
                      rowwise quant formula spelled with torch ops
                      (reference _patches/int8_ext/int8_gemm.mm:1337-1345)
  scaled_mm.npz       torch._scaled_mm (CPU, per-tensor scales) on a seeded case
  digests.json        sha256 of large results: the C1 config's
                      torch._int_mm INT32 output and its eager bf16 epilogue
                      (seed 1, BASELINE C1), the bf16 activation tables
                      (F.silu, F.gelu tanh, the MOSS SiTU pair), and the C4
                      config's rowwise-quantized activation, its scales and
                      the unfused gate/up chain's bf16 output (seed 4,
                      BASELINE C4: two torch._int_mm GEMMs with the eager
                      per-channel epilogue, F.silu, then the bf16 product)

Run from the repository root:  python tests/golden/make_golden.py
"""
import hashlib
import json
import pathlib

import numpy as np
import torch
import torch.nn.functional as F

OUT = pathlib.Path(__file__).resolve().parent


def sha(t):
    return hashlib.sha256(np.ascontiguousarray(t).tobytes()).hexdigest()


def fp8():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    dec = codes.view(torch.float8_e4m3fn).to(torch.float32).numpy()
    edges = [0.0, 2.0 ** -10, 2.0 ** -9 * 0.5, 2.0 ** -9 * 1.5, 2.0 ** -9 * 2.5, 2.0 ** -6 * 0.999,
             2.0 ** -6, 1.0, 1.0625, 1.1875, 1.9375, 1.96875, 2.0, 240.0, 248.0, 255.9, 256.0,
             416.0, 432.0, 440.0, 448.0, 455.9, 456.0, 463.9, 464.0, 464.1, 479.9, 480.0, 1e9,
             float("inf")]
    g = torch.Generator().manual_seed(0)
    rnd = torch.cat([torch.randn(4000, generator=g) * s for s in (0.01, 1.0, 30.0, 200.0)])
    x = torch.cat([torch.tensor(edges), -torch.tensor(edges), rnd]).to(torch.float32)
    enc = x.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.savez_compressed(OUT / "fp8_e4m3fn.npz", decode=dec, x=x.numpy(), encode=enc)


def quant_rows():
    K = 64
    rows = []
    rows.append(torch.zeros(K))
    rows.append(torch.full((K,), 1e-30))
    rows.append(torch.full((K,), 2.0 ** -130))                   # bf16 subnormal-range input
    rows.append(torch.full((K,), 3.0e38))
    rows.append(torch.full((K,), -7.0))
    r = torch.linspace(-127.0, 127.0, K)                          # exact halves after scaling
    rows.append(r)
    rows.append(r * 0.5 + 0.25)
    rows.append(torch.tensor([127.0, -127.0, 63.5, -63.5] * (K // 4)))
    g = torch.Generator().manual_seed(1)
    for s in (1e-3, 1.0, 1e3):
        rows.append(torch.randn(K, generator=g) * s)
    out = {}
    for name, dt in (("bf16", torch.bfloat16), ("f16", torch.float16)):
        x = torch.stack(rows).clamp(-torch.finfo(dt).max, torch.finfo(dt).max).to(dt)
        xf = x.float()
        amax = xf.abs().amax(dim=1)
        scale = torch.clamp(amax / 127.0, min=1e-30)
        s = scale.to(dt)
        s = torch.where(s == 0, torch.full_like(s, torch.finfo(dt).tiny), s)
        q = torch.clamp(torch.round((xf / s.float()[:, None]).to(dt).float()), -128, 127).to(torch.int8)
        out[f"x_{name}"] = x.view(torch.int16).numpy().view(np.uint16)
        out[f"q_{name}"] = q.numpy()
        out[f"scale_{name}"] = scale.numpy()
    np.savez_compressed(OUT / "quant_rowwise.npz", **out)


def scaled_mm():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(48, 256, generator=g)
    sa = x.abs().amax() / 448
    a = (x / sa).clamp(-448, 448).to(torch.float8_e4m3fn)
    w = 0.02 * torch.randn(40, 256, generator=g)
    sb = w.abs().amax() / 448
    wq = (w / sb).clamp(-448, 448).to(torch.float8_e4m3fn)
    y = torch._scaled_mm(a, wq.t(), scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)
    np.savez_compressed(OUT / "scaled_mm.npz", a=a.view(torch.uint8).numpy(),
                        w=wq.view(torch.uint8).numpy(), sa=sa.numpy(), sb=sb.numpy(),
                        y=y.view(torch.int16).numpy().view(np.uint16))


def digests():
    g = torch.Generator().manual_seed(1)
    M, K, N = 1024, 3072, 3072
    x = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    rs = 0.005 + 0.015 * torch.rand(M, generator=g)
    cs = 0.0005 + 0.0015 * torch.rand(N, generator=g)
    c = torch._int_mm(x, w.t())
    d = (c.float() * (cs[None, :] * rs[:, None])).to(torch.bfloat16)
    v = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    bits = lambda t: t.contiguous().view(torch.int16).numpy()
    out = {
        "c1_seed": 1,
        "c1_int32_sha256": sha(c.numpy()),
        "c1_epilogue_bf16_sha256": sha(bits(d)),
        "silu_sha256": sha(bits(F.silu(v))),
        "gelu_tanh_sha256": sha(bits(F.gelu(v, approximate="tanh"))),
        "situ_h_sha256": sha(bits(25.0 * torch.tanh(v / 25.0))),
        "situ_g_sha256": sha(bits(4.0 * torch.tanh(v / 4.0) * torch.sigmoid(v))),
        "torch": torch.__version__,
    }
    out.update(c4_digests())
    (OUT / "digests.json").write_text(json.dumps(out, indent=1) + "\n")


def c4_inputs():
    """BASELINE C4 inputs from seed 4, on the CPU: X = randn([8192, 3072]).bf16();
    W_gate, W_up = 0.02 * randn([12288, 3072]) each, quantized per output row
    (s_n = amax_n / 127, Wq = rint(W / s_n).clamp(-127, 127)). Shared with
    tests/test_gpu_configs.py, which must draw the same bytes."""
    g = torch.Generator().manual_seed(4)
    x = torch.randn(8192, 3072, generator=g).to(torch.bfloat16)
    ws = []
    for _ in range(2):
        w = 0.02 * torch.randn(12288, 3072, generator=g)
        s = w.abs().amax(dim=1) / 127.0
        q = torch.round(w / s[:, None]).clamp(-127, 127).to(torch.int8)
        ws.append((q, s.float().contiguous()))
    return x, ws


def c4_digests():
    x, ((wg, gs), (wu, us)) = c4_inputs()
    # rowwise quant, the comfy_kitchen formula in torch ops (as quant_rows)
    xf = x.float()
    scale = torch.clamp(xf.abs().amax(dim=1) / 127.0, min=1e-30)
    s = scale.to(torch.bfloat16)
    s = torch.where(s == 0, torch.full_like(s, torch.finfo(torch.bfloat16).tiny), s)
    q = torch.clamp(torch.round((xf / s.float()[:, None]).to(torch.bfloat16).float()),
                    -128, 127).to(torch.int8)
    gate = (torch._int_mm(q, wg.t()).float() * (gs[None, :] * scale[:, None])).to(torch.bfloat16)
    up = (torch._int_mm(q, wu.t()).float() * (us[None, :] * scale[:, None])).to(torch.bfloat16)
    y = F.silu(gate) * up
    return {"c4_seed": 4, "c4_q_sha256": sha(q.numpy()), "c4_scale_sha256": sha(scale.numpy()),
            "c4_pair_bf16_sha256": sha(y.view(torch.int16).numpy())}


if __name__ == "__main__":
    fp8()
    quant_rows()
    scaled_mm()
    digests()
    print("wrote", sorted(p.name for p in OUT.iterdir() if p.suffix in (".npz", ".json")))
