"""CPU oracle for the quantized-linear path. TEST INFRASTRUCTURE ONLY.

This package restates, in numpy (plus torch CPU where the reference's own
CPU/eager path is a torch call), the arithmetic of the reference pack's
quantized linear routes so that the HIP kernels can be checked against it.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the timed CPU
baseline. The product package never imports it; if the HIP library is
missing the product raises instead of falling back to anything here.

Modules
-------
numerics   bf16 / fp16 / fp8-e4m3fn bit-level conversions.
int8       INT8 W8A8 GEMM, fused epilogues, rowwise activation quant,
           comfy_kitchen-style ``int8_linear``.
fp8        FP8 ``_scaled_mm``, per-tensor activation quant, kitchen dequant,
           W8A16 linear.
pair       fused gate/up FFN pair epilogues (Krea2 SiLU*up, MOSS SiTU LUT).
act        bf16 activations (SiLU, GELU-tanh, SiTU tables).
torch_path the reference's PyTorch CPU path for the bench's CPU baseline.

Every function cites the reference file:line whose arithmetic it follows.
What pins each function (library routine, closed form, brute force) is
listed in ``tests/test_oracle.py``.
"""
