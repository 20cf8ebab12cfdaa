"""comfy_kitchen ``int8_linear`` (W8A8) on ROCm through the int8 MFMA kernels.

Mirrors ``_patches/int8_linear_kernel_mps.py`` (and the int8-fast seam of
``_patches/int8_linear_mps.py``):

* ``_int8_linear_kernel`` is the drop-in for comfy_kitchen's eager
  ``int8_linear(x, weight, weight_scale, bias=None, out_dtype=bf16,
  convrot=False, convrot_groupsize=256)`` (``:218-263``): per-row int8
  activation quant, int8 x int8 -> int32 GEMM against the stored [N, K]
  weight, rescale by ``weight_scale * x_scale``, optional bias;
* ``_int8_linear_prequant`` dispatches by scale layout (``:152-215``): a
  per-tensor scale with bf16 output uses the fused per-row epilogue
  (``row_scale = weight_scale * x_scale``), a per-channel scale the fused
  per-channel epilogue (bf16, or fp16 through the half epilogue of
  ``wan_fp16.maybe_prequant``), anything else the raw int32 GEMM followed by
  the reference's eager rescale (chunked ``C.float() * (w_scale * x_scale)``,
  ``.to(out_dtype)``, ``+ bias``) on the GPU;
* ``_quant_cached`` keeps a 1-slot cache of the quantized activation keyed
  by a weak reference to the input tensor (``:97-140``), so the q/k/v (and
  gate/up) projections of a block quantize their shared input once;
* ``_try_int8_kernel_forward`` is the Linear.forward eligibility gate
  (``:779-830``) and ``install`` wraps comfy's ``mixed_precision_ops``
  factory (``:862-894``, with its ``disabled`` filter) and its
  ``linear_input_act`` helper (``:897-977``) when ComfyUI is importable;
* ``int8_forward_dynamic[_per_row]`` are the W8A8 computation that
  ``patches/int8_fast.py`` installs in place of int8-fast's wide-batch
  forwards (``int8_linear_mps.py:54-63``; the reference re-routes them to a
  bf16 dequant + F.linear on MPS, on MI355X the int8 kernel is the fast
  path).

* ``int8_o_proj_prequant`` is the fused o-projection from the attention
  layout (``:436-535``): head merge + ConvRot + rowwise quant in one kernel
  (``ops.i8_merge_rot_quant``), then the fused INT8 GEMM;
* ``_try_int8_swiglu_forward`` is ``linear(swiglu(x))`` (``:708-775``): for a
  ConvRot weight the fused SwiGLU + rotation pass (``ops.i8_swiglu_rot``),
  rowwise quant and the INT8 GEMM; otherwise the bf16 SwiGLU and the
  ordinary W8A8 path.

* ``int8_qkv_prequant`` / ``int8_qkv_rms_rope_prequant`` are the H3 QKV
  projection straight into the attention layout, optionally with the Q/K
  RMSNorm + partial RoPE epilogue (``:266-432``);
* ``int8_mlp_bridge`` is the H3 FC1 -> SwiGLU -> ConvRot -> FC2 chain with
  FC1's output chunked through the bridge (``:538-673``).

ConvRot activations (``int8_linear(..., convrot=True)`` and ConvRot layer
weights) are rotated by the fused rotate + quant pass when they are bf16
with K % 256 == 0 and K <= 15360, group size 256; the reference rotates
with comfy_kitchen's eager Hadamard matmul (same values up to fp32
summation order; comfy_kitchen is not available, so that equivalence is
unpinned). Not supported here (those calls keep the original function):
other ConvRot inputs, non-int8 weights, tensors off the ROCm device.
"""
import inspect
import os
import weakref

import torch

from .. import ops
from .._lib import C4QError
from . import _common

TAG = "[cdna4q/int8_linear]"

_installed = False
_orig_int8_linear = None
_act_cache = None      # (x_weakref, convrot, groupsize, x_8, x_scale)
_RESCALE_CHUNK_BYTES = 256 * 1024 * 1024
_RUNTIME_LORA_ATTR = "_asfp8_runtime_lora"   # attribute a runtime LoRA adapter sets


def _convrot_ok(x, convrot_groupsize):
    """ConvRot activations this build rotates: bf16, group size 256, rows of
    K % 256 == 0 elements that fit the fused pass (K <= 15360)."""
    k = x.shape[-1]
    return (convrot_groupsize == 256 and x.dtype == torch.bfloat16 and k % 256 == 0
            and k * 2 <= 30 * 1024)


def _quant_cached(x, convrot=False, convrot_groupsize=256):
    """Rotate (ConvRot) and rowwise-quantize x (reference ``:97-140``),
    reusing the previous result when the same live tensor object is
    quantized again with the same settings. Disable the reuse with
    ``C4Q_INT8_ACT_CACHE=0``.

    The rotation is the 256-wide normalized Hadamard of every group, done
    by the fused rotate + quant pass with x viewed as [M, K/256, 1, 256]
    heads (its head merge is then the identity). The reference rotates with
    comfy_kitchen's Hadamard matmul (``_rotate_activation``): the same
    values up to the fp32 summation order before the bf16 rounding, the
    order the reference's own fused passes use."""
    global _act_cache
    if convrot and not _convrot_ok(x, convrot_groupsize):
        raise C4QError(f"{TAG} ConvRot rotation needs bf16 rows of K % 256 == 0, K <= 15360 "
                       f"and group size 256 (K={x.shape[-1]}, {x.dtype}, "
                       f"group {convrot_groupsize})")
    c = _act_cache
    if c is not None and c[0]() is x and c[1] == convrot and c[2] == convrot_groupsize:
        return c[3], c[4]
    x2 = x.reshape(-1, x.shape[-1])
    if convrot:
        k = x2.shape[1]
        x_8, x_scale = ops.i8_merge_rot_quant(x2.contiguous().view(x2.shape[0], k // 256, 1, 256))
    else:
        x_8, x_scale = ops.i8_quant_rowwise(x2)
    if os.environ.get("C4Q_INT8_ACT_CACHE", "1") != "0":
        try:
            _act_cache = (weakref.ref(x), convrot, convrot_groupsize, x_8, x_scale)
        except TypeError:      # tensor subclass without weakref support
            _act_cache = None
    return x_8, x_scale


def _int8_linear_prequant(x_8, x_scale, weight, weight_scale, bias, out_dtype, input_shape,
                          split_tail=False):
    """INT8 GEMM + epilogue from an already quantized activation (reference
    ``:152-215``; ``split_tail`` only changes the reference's schedule and is
    accepted for signature parity)."""
    weight_scale = weight_scale.reshape(-1)
    n = weight.shape[0]
    out_shape = (*input_shape[:-1], n)
    if out_dtype == torch.float16 and weight_scale.numel() == n:
        # fp16 output, per-channel scale: the fused half epilogue rounds
        # f32(C) * (w_scale[n] * x_scale[m]) to fp16 and adds the fp16 bias
        # with a second rounding -- the eager chain below, byte for byte
        # (reference ``wan_fp16.maybe_prequant``, ``_patches/wan_fp16.py:17-48``)
        return ops.i8_matmul2d_nt_fused_cs_half(
            x_8, weight, x_scale.reshape(-1).float().contiguous(),
            weight_scale.float().contiguous(), bias).reshape(out_shape)
    if out_dtype == torch.bfloat16 and weight_scale.numel() == 1:
        row_scale = (weight_scale.float() * x_scale.reshape(-1).float()).contiguous()
        bias_arg = bias.to(torch.bfloat16) if bias is not None else None
        return ops.i8_matmul2d_nt_fused(x_8, weight, row_scale, bias_arg).reshape(out_shape)
    if out_dtype == torch.bfloat16 and weight_scale.numel() == n:
        bias_arg = bias.to(torch.bfloat16) if bias is not None else None
        return ops.i8_matmul2d_nt_fused_cs(
            x_8, weight, x_scale.reshape(-1).float().contiguous(),
            weight_scale.float().contiguous(), bias_arg, split_tail).reshape(out_shape)
    # eager rescale of the raw int32 product, as comfy_kitchen does it
    result = ops.i8_matmul2d_nt(x_8, weight)
    m = result.shape[0]
    chunk = max(1, min(m, _RESCALE_CHUNK_BYTES // (n * 4)))
    xs = x_scale.reshape(-1, 1)
    parts = []
    for i in range(0, m, chunk):
        e = min(i + chunk, m)
        parts.append((result[i:e].float() * (weight_scale * xs[i:e])).to(out_dtype))
    result = torch.cat(parts, dim=0)
    if bias is not None:
        result = result + bias.to(device=result.device, dtype=result.dtype)
    return result.reshape(out_shape)


def _int8_linear_kernel(x, weight, weight_scale, bias=None, out_dtype=torch.bfloat16,
                        convrot=False, convrot_groupsize=256):
    """Kernel-backed drop-in for comfy_kitchen's eager ``int8_linear``
    (reference ``:218-263``). Calls it cannot serve go to the original
    function when one is installed, else raise."""
    if ((convrot and not _convrot_ok(x, convrot_groupsize)) or weight.dtype != torch.int8
            or not _common.on_device(x, weight) or x.dtype not in (torch.bfloat16, torch.float16)):
        if _orig_int8_linear is not None:
            return _orig_int8_linear(x, weight, weight_scale, bias, out_dtype, convrot,
                                     convrot_groupsize)
        raise C4QError(f"{TAG} call not supported (convrot={convrot}, weight {weight.dtype}, "
                       f"x {x.dtype} on {x.device})")
    x_8, x_scale = _quant_cached(x, convrot, convrot_groupsize)
    return _int8_linear_prequant(x_8, x_scale, weight, weight_scale, bias, out_dtype, x.shape)


int8_linear = _int8_linear_kernel


def _try_int8_kernel_forward(self, input):
    """Layer output via the kernel W8A8 path, or None to use comfy's forward
    (reference ``:779-830``). Eligible iff the input is a plain tensor on the
    ROCm device, the weight a TensorWiseINT8Layout QuantizedTensor without
    transposition (with ConvRot: an input the rotation pass takes), and the
    layer has no full-precision flag, force-cast or LoRA weight/bias
    functions. A call the kernels reject (C4QError) also returns None."""
    if not _common.on_device(input) or _common.is_quantized_int8(input):
        return None
    w = getattr(self, "weight", None)
    if not _common.is_quantized_int8(w):
        return None
    if getattr(self, "_full_precision_mm", False) or getattr(self, "comfy_force_cast_weights", False):
        return None
    if len(getattr(self, "weight_function", [])) or len(getattr(self, "bias_function", [])):
        return None
    params = w._params
    if getattr(params, "transposed", False):
        return None
    if input.dtype not in (torch.bfloat16, torch.float16):
        return None
    convrot = bool(getattr(params, "convrot", False))
    gs = getattr(params, "convrot_groupsize", 256)
    if convrot and not _convrot_ok(input, gs):
        return None
    try:
        return _int8_linear_kernel(input, w._qdata, params.scale, self.bias, input.dtype,
                                   convrot, gs)
    except C4QError as e:
        # a call the kernels reject keeps comfy's forward (reference :816-830)
        print(f"{TAG} kernel forward fell back ({e})")
        return None


def _plain_int8_layer(layer):
    """The weight/flag part of the reference's eligibility gates."""
    w = getattr(layer, "weight", None)
    if not _common.is_quantized_int8(w):
        return None
    if getattr(layer, "_full_precision_mm", False) or getattr(layer, "comfy_force_cast_weights", False):
        return None
    if len(getattr(layer, "weight_function", [])) or len(getattr(layer, "bias_function", [])):
        return None
    if getattr(w._params, "transposed", False):
        return None
    return w


def _runtime_lora(layer, *methods):
    """The layer's runtime LoRA adapter (the attribute the reference's H3
    Turbo loader sets): (adapter, ok). ok is False when one is attached but
    is not a "fast" adapter with every named method -- the routes then
    decline the layer so the adapter's own forward hook keeps it."""
    adapter = getattr(layer, _RUNTIME_LORA_ATTR, None)
    if adapter is None:
        return None, True
    ok = bool(getattr(adapter, "fast", False)) and all(hasattr(adapter, m) for m in methods)
    return adapter, ok


def _int8_qkv_prequant(layer, x, heads, head_dim, norm_rope):
    """The H3 QKV projection straight into the attention layout (reference
    ``_int8_qkv_prequant``, ``:266-412``): [Q, K, V], each [1, H, S, D]
    bf16, or None when a check fails (the caller then runs the layer and
    splits heads itself). ``norm_rope`` is None (layout only) or
    (freqs, q_weight, k_weight, eps) for the D = 128 RMSNorm + partial RoPE
    epilogue. ConvRot weights quantize x through the rotate + quant pass.
    A fast runtime LoRA adapter is served: with norm/RoPE, one partition
    kernel per Q, K, V adds its bf16 delta before the norm (the adapter's
    ``linear_parts``); without, its ``add_qkv_to`` updates the scattered
    Q, K, V. Switches: ``C4Q_INT8_QKV_SCATTER=0`` /
    ``C4Q_INT8_QKV_NORM_ROPE=0`` (or the reference's ``ASFP8_`` names)."""
    def _on(name):
        return os.environ.get("C4Q_" + name, os.environ.get("ASFP8_" + name, "1")) == "1"

    fused_norm_rope = norm_rope is not None
    if not _on("INT8_QKV_SCATTER") or (fused_norm_rope and not _on("INT8_QKV_NORM_ROPE")):
        return None
    runtime_lora, ok = _runtime_lora(layer, "add_qkv_to")
    lora_norm_rope = fused_norm_rope and runtime_lora is not None
    if not ok or (lora_norm_rope and not hasattr(runtime_lora, "linear_parts")):
        return None
    if (not isinstance(x, torch.Tensor) or x.dim() != 2 or not _common.on_device(x)
            or x.dtype != torch.bfloat16 or not x.is_contiguous()):
        return None
    w = _plain_int8_layer(layer)
    if w is None:
        return None
    params = w._params
    qdata = w._qdata
    if tuple(qdata.shape) != (3 * heads * head_dim, x.shape[1]):
        return None
    weight_scale = params.scale.reshape(-1)
    if weight_scale.numel() != qdata.shape[0]:
        return None
    convrot = bool(getattr(params, "convrot", False))
    groupsize = getattr(params, "convrot_groupsize", 256)
    if convrot and not _convrot_ok(x, groupsize):
        return None
    try:
        x_8, x_scale = _quant_cached(x, convrot, groupsize)
        bias = layer.bias
        bias_arg = bias.to(torch.bfloat16) if bias is not None else None
        rs = x_scale.reshape(-1).float().contiguous()
        cs = weight_scale.float().contiguous()
        if not fused_norm_rope:
            qkv = ops.i8_matmul2d_nt_fused_cs_qkv(x_8, qdata.contiguous(), rs, cs, bias_arg,
                                                  heads, head_dim)
            if runtime_lora is not None:
                qkv = list(runtime_lora.add_qkv_to(*qkv, x, heads, head_dim))
            return qkv
        freqs, q_weight, k_weight, eps = norm_rope
        if (not isinstance(freqs, torch.Tensor) or not isinstance(q_weight, torch.Tensor)
                or not isinstance(k_weight, torch.Tensor)):
            return None
        if runtime_lora is None:
            return ops.i8_matmul2d_nt_fused_cs_qkv_rms_rope(
                x_8, qdata.contiguous(), rs, cs, bias_arg, freqs, q_weight, k_weight, heads,
                head_dim, float(eps))
        # reference :351-379: the low-rank product once, then per partition
        # its delta [M, H D] and the partition kernel
        up, down, lora_scale = runtime_lora.linear_parts(x)
        width = heads * head_dim
        if up.shape[0] != 3 * width or up.shape[1] != down.shape[0] or down.shape[1] != x.shape[1]:
            return None
        low_rank = torch.nn.functional.linear(x, down)
        outputs = []
        for kind in range(3):
            lo, hi = kind * width, (kind + 1) * width
            delta = torch.nn.functional.linear(low_rank, up[lo:hi]).contiguous()
            part_bias = bias_arg[lo:hi].contiguous() if bias_arg is not None else None
            outputs.append(ops.i8_matmul2d_nt_fused_cs_qkv_lora_part(
                x_8, qdata[lo:hi].contiguous(), rs, cs[lo:hi].contiguous(), part_bias, delta,
                freqs, k_weight if kind == 1 else q_weight, heads, head_dim, kind,
                float(lora_scale), float(eps)))
            del delta
        return outputs
    except C4QError as e:
        route = "qkv norm/RoPE epilogue" if fused_norm_rope else "qkv scatter"
        print(f"{TAG} {route} fell back ({e})")
        return None


def int8_qkv_prequant(layer, x, heads, head_dim):
    """H3 QKV projection directly to contiguous [1, H, S, D] Q/K/V
    (reference ``:414-420``)."""
    return _int8_qkv_prequant(layer, x, heads, head_dim, None)


def int8_qkv_rms_rope_prequant(layer, x, freqs, q_weight, k_weight, heads, head_dim, eps):
    """H3 INT8 projection + Q/K RMSNorm / partial-RoPE epilogue (reference
    ``:423-432``)."""
    return _int8_qkv_prequant(layer, x, heads, head_dim, (freqs, q_weight, k_weight, eps))


def int8_o_proj_prequant(layer, out_bhsd):
    """o-projection straight from the attention layout [B, H, S, D]
    (reference ``:436-535``): bf16 [B, S, N], or None when a check fails
    (the caller then merges heads and runs the layer). The rotation is
    always the fused butterfly pass -- the reference's mode "2"; its mode "1"
    for D = 256 rotates with comfy_kitchen's eager Hadamard matmul, which this
    build does not have (same rounding class, different fp32 sum order).
    A fast runtime LoRA adapter's ``add_bhsd_to`` adds its delta to the
    result; a slow one makes the route decline.
    ``C4Q_INT8_OPROJ_FUSE=0`` (or the reference's ``ASFP8_INT8_OPROJ_FUSE=0``)
    turns it off."""
    runtime_lora, ok = _runtime_lora(layer)
    if not ok:
        return None
    mode = os.environ.get("C4Q_INT8_OPROJ_FUSE", os.environ.get("ASFP8_INT8_OPROJ_FUSE", "1"))
    if mode == "0":
        return None
    if (not isinstance(out_bhsd, torch.Tensor) or out_bhsd.dim() != 4
            or not _common.on_device(out_bhsd) or out_bhsd.dtype != torch.bfloat16):
        return None
    w = _plain_int8_layer(layer)
    if w is None:
        return None
    params = w._params
    if not getattr(params, "convrot", False) or getattr(params, "convrot_groupsize", 256) != 256:
        return None
    B, H, S, D = out_bhsd.shape
    qdata = w._qdata
    if D <= 0 or D > 256 or (H * D) % 256 or H * D * 2 > 30 * 1024 or H * D != qdata.shape[1]:
        return None
    x_8, x_scale = ops.i8_merge_rot_quant(out_bhsd.contiguous())
    r = _int8_linear_prequant(x_8, x_scale, qdata.contiguous(), params.scale, layer.bias,
                              torch.bfloat16, (B, S, H * D))
    if runtime_lora is not None:
        # this route bypasses Linear.forward, so the adapter's delta is added
        # here (reference :527-531)
        r = runtime_lora.add_bhsd_to(r, out_bhsd)
    return r


def int8_mlp_bridge(fc1, fc2, x):
    """H3 INT8 FC1 -> SwiGLU -> ConvRot -> FC2 without storing FC1's [M, 2F]
    output whole (reference ``:538-673``): x [M, K] bf16 -> [M, N2] bf16, or
    None when a check fails. FC1 runs through the bridge
    (``ops.i8_mlp_bridge_prequant``), FC2 on its quantized activation.
    Requires per-channel scales on both layers and a ConvRot FC2 (group
    256). With fast runtime LoRA adapters on FC1 and/or FC2 the rows go in
    tiles (``ASFP8_INT8_MLP_LORA_TILE_ROWS``, default 2048): FC1's fused_cs
    output plus its scaled delta, the bf16 SwiGLU, FC2's low-rank input
    from that activation, its rotation + quant; FC2's delta is added to the
    result (reference ``:604-658``). Switches: ``C4Q_INT8_MLP_BRIDGE=0`` (or
    ``ASFP8_INT8_MLP_BRIDGE``, ``ASFP8_INT8_SWIGLU``,
    ``ASFP8_INT8_SWIGLU_ROT`` = 0)."""
    if (os.environ.get("C4Q_INT8_MLP_BRIDGE", os.environ.get("ASFP8_INT8_MLP_BRIDGE", "1")) != "1"
            or os.environ.get("ASFP8_INT8_SWIGLU", "1") != "1"
            or os.environ.get("ASFP8_INT8_SWIGLU_ROT", "1") != "1"):
        return None
    lora1, ok1 = _runtime_lora(fc1, "linear_parts")
    lora2, ok2 = _runtime_lora(fc2, "linear_parts")
    if not (ok1 and ok2):
        return None
    if (not isinstance(x, torch.Tensor) or x.dim() != 2 or not _common.on_device(x)
            or x.dtype != torch.bfloat16 or not x.is_contiguous()):
        return None
    w1, w2 = _plain_int8_layer(fc1), _plain_int8_layer(fc2)
    if w1 is None or w2 is None:
        return None
    p1, p2 = w1._params, w2._params
    if not getattr(p2, "convrot", False) or getattr(p2, "convrot_groupsize", 256) != 256:
        return None
    q1, q2 = w1._qdata, w2._qdata
    if (q1.dim() != 2 or q2.dim() != 2 or q1.shape[0] % 512 or q1.shape[1] != x.shape[1]
            or q2.shape[1] * 2 != q1.shape[0]):
        return None
    s1, s2 = p1.scale.reshape(-1), p2.scale.reshape(-1)
    if s1.numel() != q1.shape[0] or s2.numel() != q2.shape[0]:
        return None
    convrot1 = bool(getattr(p1, "convrot", False))
    gs1 = getattr(p1, "convrot_groupsize", 256)
    if convrot1 and not _convrot_ok(x, gs1):
        return None
    try:
        x_8, x_scale = _quant_cached(x, convrot1, gs1)
        bias1 = fc1.bias.to(torch.bfloat16) if fc1.bias is not None else None
        if lora1 is None and lora2 is None:
            fc2_8, fc2_scale = ops.i8_mlp_bridge_prequant(
                x_8.contiguous(), q1.contiguous(), x_scale.reshape(-1).float().contiguous(),
                s1.float().contiguous(), bias1)
            return _int8_linear_prequant(fc2_8, fc2_scale, q2, s2, fc2.bias, x.dtype, x.shape,
                                         split_tail=True)
        linear = torch.nn.functional.linear
        rows, ffn = x.shape[0], q2.shape[1]
        parts1 = lora1.linear_parts(x) if lora1 is not None else None
        parts2 = lora2.linear_parts(x) if lora2 is not None else None
        if parts1 is not None:
            up1, down1, scale1 = parts1
            if tuple(up1.shape) != (2 * ffn, down1.shape[0]) or down1.shape[1] != x.shape[1]:
                return None
            low1 = linear(x, down1)
        if parts2 is not None:
            up2, down2, scale2 = parts2
            if tuple(up2.shape) != (q2.shape[0], down2.shape[0]) or down2.shape[1] != ffn:
                return None
            low2 = torch.empty((rows, down2.shape[0]), device=x.device, dtype=x.dtype)
        fc2_8 = torch.empty((rows, ffn), device=x.device, dtype=torch.int8)
        fc2_scale = torch.empty((rows, 1), device=x.device, dtype=torch.float32)
        tile_rows = max(128, int(os.environ.get("ASFP8_INT8_MLP_LORA_TILE_ROWS", "2048")))
        tile_rows = tile_rows // 128 * 128
        row_scales = x_scale.reshape(-1).float().contiguous()
        col_scales = s1.float().contiguous()
        q1c = q1.contiguous()
        for lo in range(0, rows, tile_rows):
            hi = min(lo + tile_rows, rows)
            wide = ops.i8_matmul2d_nt_fused_cs(x_8[lo:hi].contiguous(), q1c,
                                               row_scales[lo:hi].contiguous(), col_scales, bias1)
            if parts1 is not None:
                wide.add_(linear(low1[lo:hi], up1), alpha=scale1)
            act = _swiglu_activation(wide)
            del wide
            if parts2 is not None:
                low2[lo:hi].copy_(linear(act, down2))
            act_8, act_scale = _quant_cached(act, True, 256)
            fc2_8[lo:hi].copy_(act_8)
            fc2_scale[lo:hi].copy_(act_scale.reshape(-1, 1))
            del act, act_8, act_scale
        result = _int8_linear_prequant(fc2_8, fc2_scale, q2, s2, fc2.bias, x.dtype, x.shape,
                                       split_tail=True)
        if parts2 is not None:
            result.add_(linear(low2, up2), alpha=scale2)
        return result
    except C4QError as e:
        print(f"{TAG} MLP bridge fell back ({e})")
        return None


def _try_int8_swiglu_forward(linear, x):
    """``linear(swiglu(x))`` (reference ``:708-775``), or None to fall back.
    With a ConvRot weight (group size 256) and a contiguous bf16 input: the
    fused SwiGLU + rotation pass, rowwise quant, the INT8 GEMM; without
    ConvRot: the bf16 SwiGLU (torch ops) and the ordinary kernel path.
    With a fast runtime LoRA adapter the bf16 SwiGLU activation is formed
    once, the INT8 path projects it and the adapter's ``add_to`` adds its
    delta from that activation (a slow adapter makes the route decline, so
    the caller's ``linear(swiglu(x))`` keeps it); a call the kernels reject
    falls back too."""
    if not _common.on_device(x) or _common.is_quantized_int8(x):
        return None
    runtime_lora, ok = _runtime_lora(linear)
    if not ok:
        return None
    w = _plain_int8_layer(linear)
    if w is None:
        return None
    wide = x.shape[-1]
    if wide % 2 or x.dtype not in (torch.bfloat16, torch.float16):
        return None
    half = wide // 2
    params = w._params
    try:
        if runtime_lora is not None:
            act = _swiglu_activation(x)
            base = _int8_linear_kernel(act, w._qdata, params.scale, linear.bias, x.dtype,
                                       bool(getattr(params, "convrot", False)),
                                       getattr(params, "convrot_groupsize", 256))
            return runtime_lora.add_to(base, act)
        if getattr(params, "convrot", False):
            x2 = x.reshape(-1, wide)
            if (getattr(params, "convrot_groupsize", 256) != 256 or x.dtype != torch.bfloat16
                    or not x2.is_contiguous() or half % 256
                    or os.environ.get("C4Q_INT8_SWIGLU_ROT",
                                      os.environ.get("ASFP8_INT8_SWIGLU_ROT", "1")) == "0"):
                return None
            rot = ops.i8_swiglu_rot(x2)
            x_8, x_scale = ops.i8_quant_rowwise(rot)
            return _int8_linear_prequant(x_8, x_scale, w._qdata, params.scale, linear.bias,
                                         x.dtype, (*x.shape[:-1], half), split_tail=True)
        return _int8_linear_kernel(_swiglu_activation(x), w._qdata, params.scale, linear.bias,
                                   x.dtype)
    except C4QError as e:
        print(f"{TAG} SwiGLU forward fell back ({e})")
        return None


# ---------------------------------------------------------- int8-fast seam ---

def _w8a8_dynamic(x, weight, weight_scale, bias, compute_dtype):
    x_8, x_scale = _quant_cached(x)
    return _int8_linear_prequant(x_8, x_scale, weight, weight_scale, bias, compute_dtype, x.shape)


def int8_forward_dynamic(x, weight, weight_scale, bias, compute_dtype):
    """int8-fast's per-tensor W8A8 forward (``x_8, x_s = quant(x)``;
    ``_int_mm(x_8, w.T).float() * (w_scale * x_s)``; ``+ bias``), reference
    seam ``int8_linear_mps.py:54-57``."""
    return _w8a8_dynamic(x, weight, weight_scale, bias, compute_dtype)


def int8_forward_dynamic_per_row(x, weight, weight_scale, bias, compute_dtype):
    """int8-fast's per-output-channel W8A8 forward (reference seam
    ``int8_linear_mps.py:60-63``)."""
    return _w8a8_dynamic(x, weight, weight_scale, bias, compute_dtype)


def _swiglu_activation(x):
    """H3's bf16 SwiGLU, ``silu(x[..., :F]) * x[..., F:]`` in torch ops
    (reference ``_swiglu_activation`` ``:693-705`` without its Metal helper,
    which computes the same bytes)."""
    half = x.shape[-1] // 2
    return torch.nn.functional.silu(x[..., :half]) * x[..., half:]


def _linear_input_act_wrapper(orig_lia):
    """``comfy.ops.linear_input_act(linear, x, input_act)`` with the SwiGLU
    down-projection on the INT8 route (reference ``:897-977``). comfy calls
    this helper for SwiGLU'd down-projections instead of ``Linear.forward``,
    so the factory wrap alone never sees them. Extended calls (extra
    positional or keyword arguments) keep the original helper; a plain
    ``input_act is None`` call on a module runs the module (and with it the
    patched Linear forward); a SwiGLU call the kernel route declines on a
    layer with a runtime LoRA adapter runs ``linear(swiglu(x))`` so the
    adapter hook still fires. Switches: ``C4Q_INT8_SWIGLU`` /
    ``ASFP8_INT8_SWIGLU`` and ``ASFP8_INT8_PLAIN_LIA`` (=0 off)."""
    def linear_input_act(linear, x, input_act, *args, **kwargs):
        if args or kwargs:
            return orig_lia(linear, x, input_act, *args, **kwargs)
        if input_act == "swiglu" and _common.env_on(
                "C4Q_INT8_SWIGLU", os.environ.get("ASFP8_INT8_SWIGLU", "1")):
            res = _try_int8_swiglu_forward(linear, x)
            if res is not None:
                return res
        if (input_act is None and isinstance(linear, torch.nn.Module)
                and os.environ.get("ASFP8_INT8_PLAIN_LIA", "1") == "1"):
            return linear(x)
        if input_act == "swiglu" and getattr(linear, _RUNTIME_LORA_ATTR, None) is not None:
            return linear(_swiglu_activation(x))
        return orig_lia(linear, x, input_act)

    linear_input_act._c4q_wrapped = True
    return linear_input_act


def _wrap_factory(factory):
    """``mixed_precision_ops`` wrapper (reference ``:862-894``): drops
    ``"int8_tensorwise"`` from the ``disabled`` formats (ComfyUI's hardware
    probe does not know this int8 implementation; every other exclusion is
    kept) and patches the generated ``Linear.forward`` to try the kernel
    route first."""
    try:
        sig = inspect.signature(factory)
    except (TypeError, ValueError):
        sig = None

    def wrapped_factory(*a, **k):
        if sig is not None:
            try:
                bound = sig.bind(*a, **k)
            except TypeError:
                bound = None
            if bound is not None:
                disabled = bound.arguments.get("disabled")
                if disabled is not None:
                    bound.arguments["disabled"] = [f for f in disabled if f != "int8_tensorwise"]
                a, k = bound.args, bound.kwargs
        cls = factory(*a, **k)
        linear_cls = getattr(cls, "Linear", None)
        if linear_cls is not None and not getattr(linear_cls, "_c4q_int8_patched", False):
            orig_forward = linear_cls.forward

            def forward(self, input, *args, **kwargs):
                res = _try_int8_kernel_forward(self, input)
                if res is not None:
                    return res
                return orig_forward(self, input, *args, **kwargs)

            linear_cls.forward = forward
            linear_cls._c4q_int8_patched = True
        return cls

    wrapped_factory._c4q_wrapped = True
    return wrapped_factory


def _patch_comfy_ops(comfy_ops):
    """Install the factory and ``linear_input_act`` wraps on a ``comfy.ops``
    module (idempotent)."""
    if not getattr(comfy_ops.mixed_precision_ops, "_c4q_wrapped", False):
        comfy_ops.mixed_precision_ops = _wrap_factory(comfy_ops.mixed_precision_ops)
    lia = getattr(comfy_ops, "linear_input_act", None)
    if lia is not None and not getattr(lia, "_c4q_wrapped", False):
        comfy_ops.linear_input_act = _linear_input_act_wrapper(lia)


def install():
    """Wrap comfy's ``mixed_precision_ops`` factory and ``linear_input_act``
    helper so int8 Linear layers and SwiGLU down-projections route through
    the kernels (reference ``:833-983``). Returns True when installed
    (ComfyUI importable and a ROCm device present)."""
    global _installed, _orig_int8_linear
    if _installed:
        return True
    if not _common.rocm_available():
        return False
    try:
        import comfy.ops as comfy_ops
    except Exception:
        return False
    try:
        from comfy_kitchen.backends.eager.quantization import int8_linear as orig
        _orig_int8_linear = orig
    except Exception:
        _orig_int8_linear = None
    _patch_comfy_ops(comfy_ops)
    _installed = True
    print(f"{TAG} comfy int8 Linear layers and SwiGLU down-projections routed to the int8 "
          "MFMA kernels.")
    return True
