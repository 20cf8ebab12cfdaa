"""The reference's PyTorch CPU path for each BASELINE config, used only as
the timed CPU baseline of bench.py (test infrastructure; never the product).

Each function restates, with torch CPU ops, what the reference pack computes
when its Metal kernels are not used:

  C1  torch._int_mm(X, W.t()) + the chunked eager epilogue
      (reference _patches/int8_linear_kernel_mps.py:203-214)
  C2  kitchen per-tensor dequant W = Wq.to(bf16) * scale.to(bf16)
      (_patches/comfykitchen_fp8.py:86-89) followed by F.linear in bf16
  C3  torch._scaled_mm with per-tensor scales (CPU supports those only)
  C4  two C1 GEMM+epilogues, then F.silu(gate) * up in bf16
"""
import torch
import torch.nn.functional as F


def c1_int8_linear(x_i8, w_i8, row_scale, col_scale):
    c = torch._int_mm(x_i8, w_i8.t())
    return (c.float() * (col_scale[None, :] * row_scale[:, None])).to(torch.bfloat16)


def c2_w8a16_linear(x_bf16, w_fp8, w_scale, bias_bf16):
    w = w_fp8.to(torch.bfloat16) * w_scale.to(torch.bfloat16)
    return F.linear(x_bf16, w, bias_bf16)


def c3_scaled_mm(x_fp8, w_fp8, scale_a, scale_b):
    return torch._scaled_mm(x_fp8, w_fp8.t(), scale_a=scale_a, scale_b=scale_b,
                            out_dtype=torch.bfloat16)


def c4_ffn_pair(q, w_gate, w_up, row_scale, gate_scale, up_scale):
    g = c1_int8_linear(q, w_gate, row_scale, gate_scale)
    u = c1_int8_linear(q, w_up, row_scale, up_scale)
    return F.silu(g) * u
