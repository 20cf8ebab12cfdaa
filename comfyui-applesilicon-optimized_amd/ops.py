"""Tensor-level entry points over libcdna4q.so.

Names, argument meaning and error behaviour follow the reference's native
modules (pybind11 functions taking tensors; a bad argument raises
RuntimeError before any work is enqueued):

    i8_matmul2d_nt, i8_matmul2d_nt_fused, i8_matmul2d_nt_fused_cs,
    i8_matmul2d_nt_fused_cs_half,
    i8_quant_rowwise, i8_merge_rot_quant, i8_swiglu_rot
                                     (_patches/int8_ext/int8_gemm.mm:2626-2715)
    fp8fp8_matmul2d_nt, fp8_matmul2d_nt, fp8_matmul2d
                                     (_patches/fp8_ext/fp8_matmul2d.mm:229-353)
    w8a16_f32, w8a16_bias_bf16, num_variants
                                     (_patches/fp8s_ext/w8a16_gemm.mm:286-329)
    warmup                           (each module's pipeline warm-up)

plus the whole-operation forms the patch layer uses: ``int_mm``
(torch._int_mm), ``scaled_mm`` (torch._scaled_mm), ``fp8_quant_pertensor``,
``fp8_dequant``, ``w8a16_linear``, ``ffn_pair`` and ``moss_bf16_pair`` (the
bf16 FC1/SiTU pair of _patches/moss_bf16_ffn_pair.py:36-48).

Every function enqueues on the current HIP stream of the tensors' device and
returns without synchronizing. Outputs are allocated here with torch; the
library itself never allocates.
"""
import torch
import torch.nn.functional as F

from . import _lib
from ._lib import BF16, F16, F32, SCALE_NONE, SCALE_TENSOR, SCALE_VECTOR, C4QError

_FLOAT_CODE = {torch.bfloat16: BF16, torch.float16: F16, torch.float32: F32}
FP8 = torch.float8_e4m3fn


def _req(cond, msg):
    if not cond:
        raise C4QError(msg)


def _dev(*tensors):
    dev = None
    for t in tensors:
        if t is None:
            continue
        _req(t.device.type == "cuda", f"tensor on {t.device}, expected a ROCm (cuda) device")
        if dev is None:
            dev = t.device
        _req(t.device == dev, f"tensors on different devices ({dev} vs {t.device})")
    return dev


def _ld(t, name):
    """Row stride (elements) of a 2-D tensor whose rows are contiguous."""
    _req(t.dim() == 2, f"{name} must be 2D")
    _req(t.size(1) <= 1 or t.stride(1) == 1, f"{name} rows must be contiguous")
    if t.size(0) <= 1:
        return max(t.size(1), 1)
    _req(t.stride(0) >= t.size(1), f"{name} has overlapping rows")
    return t.stride(0)


def _vec(t, n, dtype, name):
    _req(t.dtype == dtype, f"{name} must be {dtype}")
    _req(t.numel() == n and t.is_contiguous(), f"{name} must be contiguous with {n} elements")
    return t


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


class _on(object):
    """Make `dev` the current device for the duration of a launch."""

    def __init__(self, dev):
        self.dev = dev
        self.ctx = None

    def __enter__(self):
        if self.dev.index is not None and self.dev.index != torch.cuda.current_device():
            self.ctx = torch.cuda.device(self.dev)
            self.ctx.__enter__()

    def __exit__(self, *exc):
        if self.ctx is not None:
            self.ctx.__exit__(*exc)


# ------------------------------------------------------------------ INT8 ---

def _i8_operands(a, b):
    _req(a.dtype == torch.int8 and b.dtype == torch.int8, "a/b must be int8")
    _req(a.dim() == 2 and b.dim() == 2, "a/b must be 2D")
    _req(a.size(1) == b.size(1), "K mismatch: A[M,K], B[N,K]")
    return _dev(a, b), _ld(a, "a"), _ld(b, "b")


def i8_matmul2d_nt(a_i8, b_i8):
    """C[M,N] int32 = A[M,K] int8 @ B[N,K]^T int8, exact."""
    dev, lda, ldb = _i8_operands(a_i8, b_i8)
    M, K = a_i8.shape
    N = b_i8.size(0)
    c = torch.empty((M, N), dtype=torch.int32, device=dev)
    with _on(dev):
        _lib.call("c4q_i8_gemm_nt_i32", a_i8.data_ptr(), lda, b_i8.data_ptr(), ldb,
                  c.data_ptr(), N, M, N, K, _stream(dev))
    return c


def int_mm(a, b):
    """``torch._int_mm(a, b)``: a [M,K] int8 @ b [K,N] int8 -> int32.
    ``b`` is usually ``weight.T`` of an [N,K] weight, whose transpose is the
    NT kernel's operand as-is (reference _patches/int_mm_mps.py:98-103)."""
    _req(a.dim() == 2 and b.dim() == 2 and a.size(1) == b.size(0), "int_mm: a[M,K] @ b[K,N]")
    bt = b.t()
    if bt.size(1) > 1 and bt.stride(1) != 1:
        bt = bt.contiguous()
    if a.size(1) > 1 and a.stride(1) != 1:
        a = a.contiguous()
    return i8_matmul2d_nt(a, bt)


def _bias_bf16(bias, n):
    if bias is None:
        return None
    return _vec(bias.to(torch.bfloat16).contiguous().reshape(-1), n, torch.bfloat16, "bias")


def i8_matmul2d_nt_fused(a_i8, b_i8, row_scale, bias=None):
    """D[M,N] bf16 = bf16(f32(A@B^T) * row_scale[m]) [+ bf16 bias]."""
    dev, lda, ldb = _i8_operands(a_i8, b_i8)
    M, K = a_i8.shape
    N = b_i8.size(0)
    _dev(row_scale, bias)
    _vec(row_scale, M, torch.float32, "row_scale")
    bias = _bias_bf16(bias, N)
    d = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    with _on(dev):
        _lib.call("c4q_i8_gemm_nt_fused", a_i8.data_ptr(), lda, b_i8.data_ptr(), ldb,
                  d.data_ptr(), N, row_scale.data_ptr(),
                  bias.data_ptr() if bias is not None else None, M, N, K, _stream(dev))
    return d


def i8_matmul2d_nt_fused_cs(a_i8, b_i8, row_scale, col_scale, bias=None, split_tail=False,
                            long_schedule=True, moss_schedule=False):
    """D[M,N] bf16 = bf16(f32(A@B^T) * (col_scale[n] * row_scale[m])) [+ bias].
    The reference's schedule switches select tile orders that change no
    output byte; they are accepted and have no effect here."""
    del split_tail, long_schedule, moss_schedule
    dev, lda, ldb = _i8_operands(a_i8, b_i8)
    M, K = a_i8.shape
    N = b_i8.size(0)
    _dev(row_scale, col_scale, bias)
    _vec(row_scale, M, torch.float32, "row_scale")
    _vec(col_scale, N, torch.float32, "col_scale")
    bias = _bias_bf16(bias, N)
    d = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    with _on(dev):
        _lib.call("c4q_i8_gemm_nt_fused_cs", a_i8.data_ptr(), lda, b_i8.data_ptr(), ldb,
                  d.data_ptr(), N, row_scale.data_ptr(), col_scale.data_ptr(),
                  bias.data_ptr() if bias is not None else None, M, N, K, _stream(dev))
    return d


def i8_matmul2d_nt_fused_cs_half(a_i8, b_i8, row_scale, col_scale, bias=None):
    """D[M,N] fp16 = half(f32(A@B^T) * (col_scale[n] * row_scale[m])) [then
    half(D + bias[n])]; bias is converted to fp16 as the reference does
    (_patches/int8_ext/int8_gemm.mm:1965-2010)."""
    _req(a_i8.dim() == 2 and b_i8.dim() == 2, "a/b must be 2D")
    _req(a_i8.size(1) == b_i8.size(1), "K mismatch: A[M,K], B[N,K]")
    dev, lda, ldb = _i8_operands(a_i8, b_i8)
    M, K = a_i8.shape
    N = b_i8.size(0)
    _dev(row_scale, col_scale, bias)
    _vec(row_scale, M, torch.float32, "row_scale")
    _vec(col_scale, N, torch.float32, "col_scale")
    if bias is not None:
        bias = _vec(bias.to(torch.float16).contiguous().reshape(-1), N, torch.float16, "bias")
    d = torch.empty((M, N), dtype=torch.float16, device=dev)
    with _on(dev):
        _lib.call("c4q_i8_gemm_nt_fused_cs_f16", a_i8.data_ptr(), lda, b_i8.data_ptr(), ldb,
                  d.data_ptr(), N, row_scale.data_ptr(), col_scale.data_ptr(),
                  bias.data_ptr() if bias is not None else None, M, N, K, _stream(dev))
    return d


def i8_matmul2d_nt_fused_cs_qkv(a_i8, b_i8, row_scale, col_scale, bias, heads, head_dim,
                                long_schedule=True):
    """H3 QKV projection with the per-channel bf16 epilogue stored straight
    into the attention layout: returns [Q, K, V], each [1, H, M, D] bf16
    (_patches/int8_ext/int8_gemm.mm:2028-2110). long_schedule selects a
    reference tile order that changes no output byte."""
    del long_schedule
    dev, lda, ldb = _i8_operands(a_i8, b_i8)
    _req(a_i8.is_contiguous() and b_i8.is_contiguous(), "a/b must be contiguous 2D tensors")
    M, K = a_i8.shape
    N = b_i8.size(0)
    _req(M > 64, "H3 QKV specialization requires M > 64")
    H, D = int(heads), int(head_dim)
    _req(H > 0 and D > 0 and N == 3 * H * D, "weight width must equal 3*H*D")
    _req(D % 8 == 0, "head_dim must be a multiple of 8")
    _dev(row_scale, col_scale, bias)
    _vec(row_scale, M, torch.float32, "row_scale")
    _vec(col_scale, N, torch.float32, "col_scale")
    bias = _bias_bf16(bias, N)
    outs = [torch.empty((1, H, M, D), dtype=torch.bfloat16, device=dev) for _ in range(3)]
    with _on(dev):
        _lib.call("c4q_i8_gemm_nt_fused_cs_qkv", a_i8.data_ptr(), lda, b_i8.data_ptr(), ldb,
                  outs[0].data_ptr(), outs[1].data_ptr(), outs[2].data_ptr(),
                  row_scale.data_ptr(), col_scale.data_ptr(),
                  bias.data_ptr() if bias is not None else None, M, K, H, D, _stream(dev))
    return outs


def i8_matmul2d_nt_fused_cs_qkv_rms_rope(a_i8, b_i8, row_scale, col_scale, bias, freqs,
                                         q_weight, k_weight, heads, head_dim, eps,
                                         long_schedule=True):
    """H3 QKV projection whose Q and K heads get RMSNorm (fp32 weights
    q_weight / k_weight, eps) and partial split-half RoPE (freqs bf16
    [..., M, R, 2, 2], rotating the first 2R of D = 128 columns) before the
    store; returns [Q, K, V], each [1, H, M, 128] bf16
    (_patches/int8_ext/int8_gemm.mm:2111-2209, kernel :683-861).
    long_schedule selects a reference tile order that changes no output
    byte."""
    del long_schedule
    dev, lda, ldb = _i8_operands(a_i8, b_i8)
    _req(a_i8.is_contiguous() and b_i8.is_contiguous(), "a/b must be contiguous 2D tensors")
    M, K = a_i8.shape
    N = b_i8.size(0)
    _req(M > 64, "H3 QKV specialization requires M > 64")
    H, D = int(heads), int(head_dim)
    _req(H > 0 and D == 128 and N == 3 * H * D,
         "fused QKV norm/RoPE requires D=128 and width=3*H*D")
    _dev(row_scale, col_scale, bias, freqs, q_weight, k_weight)
    _vec(row_scale, M, torch.float32, "row_scale")
    _vec(col_scale, N, torch.float32, "col_scale")
    _req(freqs.dtype == torch.bfloat16 and freqs.is_contiguous() and freqs.dim() >= 3,
         "freqs must be contiguous bf16")
    R = int(freqs.size(-3))
    _req(R > 0 and 2 * R <= D and freqs.numel() == M * R * 4, "freqs shape mismatch")
    for name, w in (("q_weight", q_weight), ("k_weight", k_weight)):
        _req(w.dtype == torch.float32 and w.is_contiguous() and w.numel() == D,
             f"{name} must be {D} contiguous float32 elements")
    # the kernels read the weights 16 bytes and the freqs 4 bytes at a time
    q_weight, k_weight = (w if w.data_ptr() % 16 == 0 else w.clone() for w in (q_weight, k_weight))
    if freqs.data_ptr() % 4:
        freqs = freqs.clone()
    bias = _bias_bf16(bias, N)
    outs = [torch.empty((1, H, M, D), dtype=torch.bfloat16, device=dev) for _ in range(3)]
    with _on(dev):
        _lib.call("c4q_i8_gemm_nt_fused_cs_qkv_rms_rope", a_i8.data_ptr(), lda, b_i8.data_ptr(),
                  ldb, outs[0].data_ptr(), outs[1].data_ptr(), outs[2].data_ptr(),
                  row_scale.data_ptr(), col_scale.data_ptr(),
                  bias.data_ptr() if bias is not None else None, freqs.data_ptr(),
                  q_weight.data_ptr(), k_weight.data_ptr(), M, K, H, R, float(eps), _stream(dev))
    return outs


def i8_matmul2d_nt_fused_cs_qkv_lora_part(a_i8, b_i8, row_scale, col_scale, bias, delta, fr,
                                          norm_weight, heads, head_dim, kind, delta_scale, eps,
                                          long_schedule=True):
    """One partition of the H3 QKV projection with a runtime-LoRA delta:
    b_i8 holds the partition's H*128 weight rows (kind 0 = Q, 1 = K, 2 = V),
    delta the bf16 low-rank output [M, H*128] for it, added after the bias as
    ``bf16(value + bf16(delta * bf16(delta_scale)))``; Q and K then get the
    RMSNorm (fp32 norm_weight) + partial split-half RoPE (fr bf16 [..., M,
    R, 2, 2]) of the fused QKV route. Returns [1, H, M, 128] bf16
    (_patches/int8_ext/int8_gemm.mm:2211-2330, kernels :915-1085).
    long_schedule selects a reference tile order that changes no output
    byte."""
    del long_schedule
    dev, lda, ldb = _i8_operands(a_i8, b_i8)
    _req(a_i8.is_contiguous() and b_i8.is_contiguous(), "a/b must be contiguous 2D tensors")
    M, K = a_i8.shape
    N = b_i8.size(0)
    _req(M > 64, "H3 QKV specialization requires M > 64")
    H, D = int(heads), int(head_dim)
    _req(H > 0 and D == 128 and N == H * D,
         "LoRA QKV partition requires D=128 and width=H*D")
    kind = int(kind)
    _req(0 <= kind <= 2, "kind must be Q=0, K=1 or V=2")
    _dev(row_scale, col_scale, bias, delta, fr, norm_weight)
    _vec(row_scale, M, torch.float32, "row_scale")
    _vec(col_scale, N, torch.float32, "col_scale")
    _req(delta.dtype == torch.bfloat16 and delta.is_contiguous() and delta.dim() == 2,
         "LoRA delta must be contiguous bf16 [M,H*D]")
    _req(tuple(delta.shape) == (M, N), "LoRA delta shape mismatch")
    _req(fr.dtype == torch.bfloat16 and fr.is_contiguous() and fr.dim() >= 3,
         "freqs must be contiguous bf16")
    R = int(fr.size(-3))
    _req(R > 0 and 2 * R <= D and fr.numel() == M * R * 4, "freqs shape mismatch")
    _req(norm_weight.dtype == torch.float32 and norm_weight.is_contiguous()
         and norm_weight.numel() == D, "norm weight must contain D elements")
    # the kernels read delta 8 bytes, the norm weight 16 and the freqs 4 at a time
    if delta.data_ptr() % 8:
        delta = delta.clone()
    if norm_weight.data_ptr() % 16:
        norm_weight = norm_weight.clone()
    if fr.data_ptr() % 4:
        fr = fr.clone()
    bias = _bias_bf16(bias, N)
    out = torch.empty((1, H, M, D), dtype=torch.bfloat16, device=dev)
    with _on(dev):
        _lib.call("c4q_i8_gemm_nt_fused_cs_qkv_lora_part", a_i8.data_ptr(), lda, b_i8.data_ptr(),
                  ldb, out.data_ptr(), row_scale.data_ptr(), col_scale.data_ptr(),
                  bias.data_ptr() if bias is not None else None, delta.data_ptr(), fr.data_ptr(),
                  norm_weight.data_ptr(), M, K, H, R, kind, float(delta_scale), float(eps),
                  _stream(dev))
    return out


# Chunk of FC1 rows of the MLP bridge when the caller asks for "auto": all
# of them. Measured on MI355X at H3's FC1 (K 5376, W 28672), whole-M FC1
# GEMMs win over chunks whose bf16 output would stay in the Infinity Cache:
# 8192 rows take 1344 us at once, 1364 in chunks of 4096, 1536 of 2048, 1512
# of 1024 (5378 rows: 964 / 972 / 1009 / 1006). The scratch then holds the
# whole [M, 2F] FC1 output (470 MB at 8192 rows), small against 288 GB HBM.
MLP_BRIDGE_AUTO_ROWS = 0


def i8_mlp_bridge_prequant(a_i8, fc1_weight, row_scale, fc1_col_scale, fc1_bias=None,
                           long_schedule=True, tile_rows=-1):
    """H3 FC1/SwiGLU/FC2 bridge, front half: (q [M, F] int8, scales [M, 1]
    fp32), FC2's ConvRot-rotated rowwise-quantized activation, from the int8
    FC1 input without storing FC1's [M, 2F] output whole
    (_patches/int8_ext/int8_gemm.mm:2377-2537). tile_rows: -1 auto, 0 all
    rows at once, else at least 128 (rounded down to a multiple of 128).
    long_schedule selects a reference tile order that changes no byte."""
    del long_schedule
    dev, lda, ldw = _i8_operands(a_i8, fc1_weight)
    _req(a_i8.is_contiguous() and fc1_weight.is_contiguous(),
         "activation and FC1 weight must be contiguous 2D tensors")
    M, K = a_i8.shape
    W = fc1_weight.size(0)
    _req(M > 64 and W > 0 and W % 512 == 0, "bridge requires M > 64 and F divisible by 256")
    _req(tile_rows == -1 or tile_rows == 0 or tile_rows >= 128,
         "tile_rows must be -1 (auto), zero, or at least 128")
    _dev(row_scale, fc1_col_scale, fc1_bias)
    _vec(row_scale, M, torch.float32, "row_scale")
    _vec(fc1_col_scale, W, torch.float32, "fc1_col_scale")
    bias = _bias_bf16(fc1_bias, W)
    if tile_rows < 0:
        tile_rows = MLP_BRIDGE_AUTO_ROWS
    rows = M if tile_rows == 0 else min(M, tile_rows)
    rows = rows // 128 * 128 if rows >= 128 else rows
    F = W // 2
    wide = torch.empty((rows, W), dtype=torch.bfloat16, device=dev)
    # rows of F <= 15360 are rotated and quantized in one pass (no rot scratch)
    rot = torch.empty((rows, F) if F * 2 > 30 * 1024 else (0,), dtype=torch.bfloat16, device=dev)
    q = torch.empty((M, F), dtype=torch.int8, device=dev)
    scales = torch.empty((M, 1), dtype=torch.float32, device=dev)
    silu = act_table("silu", dev)
    with _on(dev):
        _lib.call("c4q_i8_mlp_bridge_prequant", a_i8.data_ptr(), lda, fc1_weight.data_ptr(), ldw,
                  row_scale.data_ptr(), fc1_col_scale.data_ptr(),
                  bias.data_ptr() if bias is not None else None, silu.data_ptr(), M, K, W, rows,
                  wide.data_ptr(), rot.data_ptr() if rot.numel() else None, q.data_ptr(),
                  scales.data_ptr(), _stream(dev))
    return q, scales


def i8_mlp_bridge_prequant_noalloc(a_i8, fc1_weight, row_scale, fc1_col_scale, fc1_bias=None):
    """i8_mlp_bridge_prequant with FC1's staging in the library's own
    per-GPU array (64 MiB) instead of torch-allocated scratch: the outputs
    q [M, F] and scales [M, 1] are allocated here, nothing else. Rows run in
    chunks of as many 128-row blocks as the array holds. Calls that overlap
    on one GPU (other streams or threads) race on the array."""
    dev, lda, ldw = _i8_operands(a_i8, fc1_weight)
    _req(a_i8.is_contiguous() and fc1_weight.is_contiguous(),
         "activation and FC1 weight must be contiguous 2D tensors")
    M, K = a_i8.shape
    W = fc1_weight.size(0)
    _req(M > 64 and W > 0 and W % 512 == 0, "bridge requires M > 64 and F divisible by 256")
    _dev(row_scale, fc1_col_scale, fc1_bias)
    _vec(row_scale, M, torch.float32, "row_scale")
    _vec(fc1_col_scale, W, torch.float32, "fc1_col_scale")
    bias = _bias_bf16(fc1_bias, W)
    F = W // 2
    q = torch.empty((M, F), dtype=torch.int8, device=dev)
    scales = torch.empty((M, 1), dtype=torch.float32, device=dev)
    silu = act_table("silu", dev)
    with _on(dev):
        _lib.call("c4q_i8_mlp_bridge_prequant_noalloc", a_i8.data_ptr(), lda,
                  fc1_weight.data_ptr(), ldw, row_scale.data_ptr(), fc1_col_scale.data_ptr(),
                  bias.data_ptr() if bias is not None else None, silu.data_ptr(), M, K, W,
                  q.data_ptr(), scales.data_ptr(), _stream(dev))
    return q, scales


def i8_merge_rot_quant(x, rotate=True):
    """x [B,H,S,D] bf16 (attention layout) -> (q [B*S, H*D] int8,
    scales [B*S, 1] fp32): head merge, ConvRot rotation of every 256-element
    group (rotate=True) and rowwise int8 quant in one pass
    (_patches/int8_ext/int8_gemm.mm:2545-2585)."""
    _req(x.dim() == 4, "x must be [B,H,S,D]")
    _req(x.dtype == torch.bfloat16, "x must be bf16")
    _req(x.is_contiguous(), "x must be contiguous")
    dev = _dev(x)
    B, H, S, D = x.shape
    K = H * D
    _req(0 < D <= 256 and K % 256 == 0, "merged width must tile 256-element convrot groups")
    _req(H >= 1 and K * 2 <= 30 * 1024, "H*D too large for threadgroup memory")
    q = torch.empty((B * S, K), dtype=torch.int8, device=dev)
    scales = torch.empty((B * S, 1), dtype=torch.float32, device=dev)
    with _on(dev):
        _lib.call("c4q_i8_merge_rot_quant", x.data_ptr(), B, H, S, D, 1 if rotate else 0,
                  q.data_ptr(), scales.data_ptr(), _stream(dev))
    return q, scales


def i8_swiglu_rot(x, silu_table=None):
    """x [M, 2F] bf16 contiguous -> [M, F] bf16: SwiGLU (bf16 SiLU of the gate
    half times the up half, in bf16) rotated per 256-element ConvRot group
    (_patches/int8_ext/int8_gemm.mm:2593-2631). silu_table defaults to the
    device's bf16 SiLU table (ops.act_table("silu"))."""
    _req(x.dtype == torch.bfloat16, "x must be bf16")
    _req(x.dim() == 2 and x.is_contiguous(), "x must be contiguous [M,2F]")
    M, W = x.shape
    _req(W % 512 == 0, "F must be a multiple of convrot groupsize 256")
    dev = _dev(x, silu_table)
    t = silu_table if silu_table is not None else act_table("silu", dev)
    _req(t.numel() == 65536 and t.element_size() == 2 and t.is_contiguous(),
         "silu_table must be 65536 contiguous 16-bit entries")
    F = W // 2
    rot = torch.empty((M, F), dtype=torch.bfloat16, device=dev)
    with _on(dev):
        _lib.call("c4q_i8_swiglu_rot", x.data_ptr(), M, F, t.data_ptr(), rot.data_ptr(),
                  _stream(dev))
    return rot


def i8_quant_rowwise(x):
    """x[M,K] bf16/f16 -> (q[M,K] int8, scales[M,1] fp32), bit-exact with
    comfy_kitchen quantize_int8_rowwise."""
    _req(x.dim() == 2, "x must be 2D [M,K]")
    _req(x.dtype in (torch.bfloat16, torch.float16), "x must be bf16 or f16")
    dev = _dev(x)
    ldx = _ld(x, "x")
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.int8, device=dev)
    scales = torch.empty((M, 1), dtype=torch.float32, device=dev)
    with _on(dev):
        _lib.call("c4q_i8_quant_rowwise", x.data_ptr(), _FLOAT_CODE[x.dtype], ldx, q.data_ptr(),
                  max(K, 1), scales.data_ptr(), M, K, _stream(dev))
    return q, scales


def ffn_pair(q, w_gate, w_up, row_scale, gate_scale, up_scale, table_gate=None, table_up=None):
    """Fused gate/up pair, bf16 [M, N_out]:
    bf16(f32(T1[g]) * f32(T2[u])) with g, u the per-channel fused bf16
    projections; a None table is the identity."""
    _req(w_gate.shape == w_up.shape, "gate/up weights differ in shape")
    dev, lda, ldw = _i8_operands(q, w_gate)
    _req(_ld(w_up, "w_up") == ldw, "gate/up weights must share a row stride")
    _dev(w_up, row_scale, gate_scale, up_scale, table_gate, table_up)
    M, K = q.shape
    N = w_gate.size(0)
    _vec(row_scale.reshape(-1), M, torch.float32, "row_scale")
    _vec(gate_scale.reshape(-1), N, torch.float32, "gate_scale")
    _vec(up_scale.reshape(-1), N, torch.float32, "up_scale")
    for t in (table_gate, table_up):
        if t is not None:
            _req(t.numel() == 65536 and t.element_size() == 2 and t.is_contiguous(),
                 "activation tables must be 65536 contiguous 16-bit entries")
    d = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    with _on(dev):
        _lib.call("c4q_i8_ffn_pair", q.data_ptr(), lda, w_gate.data_ptr(), w_up.data_ptr(), ldw,
                  d.data_ptr(), N, row_scale.data_ptr(), gate_scale.data_ptr(),
                  up_scale.data_ptr(),
                  table_gate.data_ptr() if table_gate is not None else None,
                  table_up.data_ptr() if table_up is not None else None, M, N, K, _stream(dev))
    return d


def moss_bf16_pair(x, weight, tables):
    """MOSS bf16 FC1 + SiTU, as the reference's project(x, weight, tables)
    (_patches/moss_bf16_ffn_pair.py:36-48): weight [2F, K] bf16 splits into
    hidden rows [0, F) and gate rows [F, 2F); out[..., F] bf16 =
    bf16(f32(T_h[bf16(x@Wh^T)]) * f32(T_g[bf16(x@Wg^T)])) with fp32
    accumulation; tables = (T_h, T_g), 65,536 bf16 entries each."""
    _req(x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16,
         "x and weight must be bf16")
    _req(weight.dim() == 2 and weight.size(0) % 2 == 0, "weight must be [2F, K]")
    _req(x.size(-1) == weight.size(1), "K mismatch: x[..., K], weight[2F, K]")
    th, tg = tables
    dev = _dev(x, weight, th, tg)
    for t in (th, tg):
        _req(t.numel() == 65536 and t.element_size() == 2 and t.is_contiguous(),
             "activation tables must be 65536 contiguous 16-bit entries")
    lead = x.shape[:-1]
    K = x.size(-1)
    x2 = x.reshape(-1, K)
    M = x2.size(0)
    F = weight.size(0) // 2
    ldw = _ld(weight, "weight")
    wh, wg = weight[:F], weight[F:]
    d = torch.empty((M, F), dtype=torch.bfloat16, device=dev)
    with _on(dev):
        _lib.call("c4q_bf16_ffn_pair", x2.data_ptr(), _ld(x2, "x"), wh.data_ptr(), wg.data_ptr(),
                  ldw, d.data_ptr(), F, th.data_ptr(), tg.data_ptr(), M, F, K, _stream(dev))
    return d.reshape(*lead, F)


# ------------------------------------------------------------------- FP8 ---

def _as_u8(t):
    return t.view(torch.uint8) if t.dtype == FP8 else t


def _scale_mode(s, n, name):
    if s is None:
        return SCALE_NONE, None
    s = s.to(torch.float32).contiguous()
    if s.numel() == 1:
        return SCALE_TENSOR, s
    _req(s.numel() == n, f"{name} must have 1 or {n} elements")
    return SCALE_VECTOR, s


def _f8_gemm(a_u8, lda, w_u8, ldw, M, N, K, dev, out_dtype, scale_a=None, scale_b=None,
             scale_result=None, bias=None):
    _req(out_dtype in _FLOAT_CODE, f"unsupported out_dtype {out_dtype}")
    am, sa = _scale_mode(scale_a, M, "scale_a")
    bm, sb = _scale_mode(scale_b, N, "scale_b")
    sr = None
    if scale_result is not None:
        sr = scale_result.to(torch.float32).contiguous()
        _req(sr.numel() == 1, "scale_result must be a scalar tensor")
    bdt = F32
    if bias is not None:
        _req(bias.dtype in _FLOAT_CODE, "bias must be bf16, f16 or f32")
        bias = bias.contiguous().reshape(-1)
        _req(bias.numel() == N, f"bias must have {N} elements")
        bdt = _FLOAT_CODE[bias.dtype]
    _dev(sa, sb, sr, bias)
    d = torch.empty((M, N), dtype=out_dtype, device=dev)
    with _on(dev):
        _lib.call("c4q_f8_gemm_nt_scaled", a_u8.data_ptr(), lda, w_u8.data_ptr(), ldw,
                  d.data_ptr(), _FLOAT_CODE[out_dtype], N,
                  sa.data_ptr() if sa is not None else None, am,
                  sb.data_ptr() if sb is not None else None, bm,
                  sr.data_ptr() if sr is not None else None,
                  bias.data_ptr() if bias is not None else None, bdt, M, N, K, _stream(dev))
    return d


def fp8fp8_matmul2d_nt(a_u8, w_u8, K=None, N=None):
    """C[M,N] f32 (unscaled) = A[M,K] fp8 @ W[N,K]^T fp8 (e4m3fn bytes)."""
    a_u8, w_u8 = _as_u8(a_u8), _as_u8(w_u8)
    _req(a_u8.dtype == torch.uint8 and w_u8.dtype == torch.uint8, "a/w must be fp8 bytes")
    _req(a_u8.dim() == 2 and w_u8.dim() == 2 and a_u8.size(1) == w_u8.size(1),
         "K mismatch: A[M,K], W[N,K]")
    _req(K is None or K == a_u8.size(1), "K does not match the operands")
    _req(N is None or N == w_u8.size(0), "N does not match the weight")
    dev = _dev(a_u8, w_u8)
    M, K = a_u8.shape
    return _f8_gemm(a_u8, _ld(a_u8, "a"), w_u8, _ld(w_u8, "w"), M, w_u8.size(0), K, dev,
                    torch.float32)


def scaled_mm(input, other, *, out_dtype=None, scale_a=None, scale_b=None, bias=None,
              scale_result=None, use_fast_accum=False):
    """``torch._scaled_mm`` for e4m3fn operands on the fp8 route:
    out = f32(input @ other); *= scale_a; *= scale_b; *= scale_result;
    += f32(bias); -> out_dtype (f32 when None). Per-tensor or vector scales
    (scale_a [M,1] rowwise, scale_b [1,N] columnwise). Accumulation is fp32
    regardless of use_fast_accum."""
    del use_fast_accum
    _req(input.dtype == FP8 and other.dtype == FP8, "scaled_mm: operands must be float8_e4m3fn")
    _req(input.dim() == 2 and other.dim() == 2 and input.size(1) == other.size(0),
         "scaled_mm: input[M,K] @ other[K,N]")
    dev = _dev(input, other)
    a = input if (input.size(1) <= 1 or input.stride(1) == 1) else input.contiguous()
    w = other.t()
    if w.size(1) > 1 and w.stride(1) != 1:
        w = w.contiguous()
    M, K = a.shape
    N = w.size(0)
    return _f8_gemm(a.view(torch.uint8), _ld(a, "input"), w.view(torch.uint8), _ld(w, "other^T"),
                    M, N, K, dev, out_dtype if out_dtype is not None else torch.float32,
                    scale_a, scale_b, scale_result, bias)


def fp8_quant_pertensor(x):
    """Dynamic per-tensor e4m3fn quant: (q same shape as x, scale [] fp32)."""
    _req(x.dtype in (torch.bfloat16, torch.float16), "x must be bf16 or f16")
    dev = _dev(x)
    x = x.contiguous()
    q = torch.empty(x.shape, dtype=FP8, device=dev)
    ws = torch.empty(2, dtype=torch.float32, device=dev)
    with _on(dev):
        _lib.call("c4q_f8_quant_pertensor", x.data_ptr(), _FLOAT_CODE[x.dtype], x.numel(),
                  q.data_ptr(), ws.data_ptr(), ws.data_ptr() + 4, _stream(dev))
    return q, ws[0]


def fp8_dequant(w, scale=None, out_dtype=torch.bfloat16):
    """comfy_kitchen dequantize_per_tensor_fp8: out_dtype(w) * out_dtype(scale),
    one rounding of the product; plain exact decode when scale is None."""
    _req(w.dtype in (FP8, torch.uint8), "w must be float8_e4m3fn")
    _req(out_dtype in _FLOAT_CODE, "out_dtype must be bf16, f16 or f32")
    dev = _dev(w, scale)
    w = w.contiguous()
    if scale is not None:
        scale = scale.to(torch.float32).contiguous()
        _req(scale.numel() == 1, "per-tensor scale must be a scalar")
    out = torch.empty(w.shape, dtype=out_dtype, device=dev)
    with _on(dev):
        _lib.call("c4q_fp8_dequant", w.data_ptr(), w.numel(),
                  scale.data_ptr() if scale is not None else None, out.data_ptr(),
                  _FLOAT_CODE[out_dtype], _stream(dev))
    return out


def w8a16_linear(x, weight, w_scale=None, bias=None, out_dtype=None, act_table=None):
    """W8A16 linear over the last dim of x (bf16/f16): the fp8 [N,K] weight
    is dequantized in registers to x's dtype (kitchen formula when w_scale is
    given), fp32 accumulate, out = out_dtype(acc + f32 bias) rounded once,
    then the optional 65,536-entry bf16 activation table."""
    _req(x.dtype in (torch.bfloat16, torch.float16), "x must be bf16 or f16")
    _req(weight.dtype in (FP8, torch.uint8) and weight.dim() == 2, "weight must be fp8 [N,K]")
    _req(x.size(-1) == weight.size(1), "K mismatch")
    out_dtype = out_dtype or x.dtype
    _req(out_dtype in _FLOAT_CODE, "out_dtype must be bf16, f16 or f32")
    dev = _dev(x, weight, w_scale, bias, act_table)
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.size(-1))
    if x2.size(1) > 1 and x2.stride(1) != 1:
        x2 = x2.contiguous()
    w = weight.view(torch.uint8) if weight.dtype == FP8 else weight
    M, K = x2.shape
    N = w.size(0)
    if w_scale is not None:
        w_scale = w_scale.to(torch.float32).contiguous()
        _req(w_scale.numel() == 1, "w_scale must be a per-tensor scalar")
    bdt = F32
    if bias is not None:
        _req(bias.dtype in _FLOAT_CODE, "bias must be bf16, f16 or f32")
        bias = bias.contiguous().reshape(-1)
        _req(bias.numel() == N, f"bias must have {N} elements")
        bdt = _FLOAT_CODE[bias.dtype]
    if act_table is not None:
        _req(out_dtype == torch.bfloat16, "act_table needs a bf16 output")
        _req(act_table.numel() == 65536 and act_table.element_size() == 2
             and act_table.is_contiguous(), "act_table must be 65536 contiguous 16-bit entries")
    d = torch.empty((M, N), dtype=out_dtype, device=dev)
    with _on(dev):
        _lib.call("c4q_w8a16_gemm_nt", x2.data_ptr(), _FLOAT_CODE[x2.dtype], _ld(x2, "x"),
                  w.data_ptr(), _ld(w, "weight"),
                  w_scale.data_ptr() if w_scale is not None else None,
                  d.data_ptr(), _FLOAT_CODE[out_dtype], N,
                  bias.data_ptr() if bias is not None else None, bdt,
                  act_table.data_ptr() if act_table is not None else None, M, N, K, _stream(dev))
    return d.reshape(*lead, N)


def w8a16_f32(a, w_u8, variant=-1):
    """C[M,N] f32 = A[M,K] (f16/bf16) @ W[N,K]^T fp8. ``variant`` picked the
    reference's Metal tile geometry; tiles are chosen by shape here."""
    del variant
    _req(a.dim() == 2, "a must be 2D")
    return w8a16_linear(a, w_u8, out_dtype=torch.float32)


def w8a16_bias_bf16(a, w_u8, bias=None, variant=-1):
    """D[M,N] bf16 = bf16(A @ W^T + f32 bias[n]) (fused epilogue)."""
    del variant
    _req(a.dim() == 2, "a must be 2D")
    if bias is not None:
        _req(bias.dtype == torch.float32, "bias must be f32")
    return w8a16_linear(a, w_u8, bias=bias, out_dtype=torch.bfloat16)


def fp8_matmul2d_nt(a, w_u8, N=None):
    """C[M,N] f32 = A[M,K] (f16 / bf16) @ W^T, W [N,K] e4m3fn bytes, no
    scale (reference fp8_ext ``fp8_matmul2d_nt``,
    ``_patches/fp8_ext/fp8_matmul2d.mm:312-353``): the W8A16 route with an
    f32 output. The reference requires fp16 activations; bf16 is accepted
    too."""
    _req(a.dim() == 2, "a must be 2D")
    w_u8 = _as_u8(w_u8)
    _req(w_u8.dim() == 2, "w must be 2D [N,K]")
    _req(N is None or int(N) == w_u8.size(0), "N does not match the weight")
    return w8a16_linear(a, w_u8, out_dtype=torch.float32)


def fp8_matmul2d(a, w_u8, N=None):
    """C[M,N] f32 = A[M,K] (f16 / bf16) @ W, W [K,N] e4m3fn bytes (reference
    fp8_ext ``fp8_matmul2d``, ``_patches/fp8_ext/fp8_matmul2d.mm:268-310``).
    The [K,N] weight is transposed to the [N,K] operand order once per call
    (one device copy of the fp8 bytes), then the W8A16 route runs."""
    _req(a.dim() == 2, "a must be 2D")
    w_u8 = _as_u8(w_u8)
    _req(w_u8.dim() == 2 and w_u8.size(0) == a.size(1), "w must be [K,N] with K = a.size(1)")
    _req(N is None or int(N) == w_u8.size(1), "N does not match the weight")
    return w8a16_linear(a, w_u8.t().contiguous(), out_dtype=torch.float32)


# ------------------------------------------------------ activation tables ---

_TABLES = {}


def _all_bf16_cpu():
    return torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)


def _table_on(key, device, build):
    """Table(s) `build()` made once on the CPU, copied once per device."""
    device = torch.device(device)
    t = _TABLES.get((key, device))
    if t is None:
        cpu = _TABLES.get((key, None))
        if cpu is None:
            cpu = build()
            _TABLES[(key, None)] = cpu
        if isinstance(cpu, tuple):
            t = tuple(c.to(device) for c in cpu)
        else:
            t = cpu.to(device)
        _TABLES[(key, device)] = t
    return t


def act_table(name, device):
    """65,536-entry bf16 table of activation `name` ('silu' | 'gelu_tanh'):
    torch's CPU op over every bf16 value -- the unfused "bf16 tensor ->
    F.<act>" chain the fused epilogues reproduce -- built once and copied to
    `device`. (torch's ROCm kernels for these ops round a few entries
    differently from its CPU kernels; the CPU tables are the ones the
    reference's eager chain is pinned to.)"""
    def build():
        v = _all_bf16_cpu()
        if name == "silu":
            r = F.silu(v)
        elif name == "gelu_tanh":
            r = F.gelu(v, approximate="tanh")
        else:
            raise C4QError(f"unknown activation {name!r}")
        return r.contiguous().view(torch.int16)
    if name not in ("silu", "gelu_tanh"):
        raise C4QError(f"unknown activation {name!r}")
    return _table_on(name, device, build)


def situ_tables(device):
    """MOSS SiTU tables T_h = 25 tanh(v/25), T_g = 4 tanh(v/4) sigmoid(v) over
    every bf16 v, each op in bf16 (reference _patches/moss_fast.py:97-99),
    built with torch's CPU ops and copied to `device`."""
    def build():
        v = _all_bf16_cpu()
        th = (25.0 * torch.tanh(v / 25.0)).contiguous().view(torch.int16)
        tg = (4.0 * torch.tanh(v / 4.0) * torch.sigmoid(v)).contiguous().view(torch.int16)
        return (th, tg)
    return _table_on("situ", device, build)


# ------------------------------------------------ module-level utilities ---

def warmup():
    """The reference modules' ``warmup()`` builds their Metal pipelines
    (``_patches/int8_ext/int8_gemm.mm:2691``, ``_patches/fp8_ext/fp8_matmul2d.mm:359``,
    ``_patches/fp8s_ext/w8a16_gemm.mm:325``). Here it loads libcdna4q.so
    (kernels are compiled ahead of time) and returns True."""
    _lib.load()
    return True


def num_variants():
    """Count of the reference's W8A16 Metal tile variants
    (``_patches/fp8s_ext/w8a16_gemm.mm:162-169,324``); the ``variant``
    argument of ``w8a16_f32`` / ``w8a16_bias_bf16`` is accepted and ignored
    here (tiles are planned by shape)."""
    return 4
