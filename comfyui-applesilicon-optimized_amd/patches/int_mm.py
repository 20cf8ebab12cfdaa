"""torch._int_mm on ROCm through the exact int8 MFMA kernel.

Mirrors ``_patches/int_mm_mps.py``: the replacement keeps the
``torch._int_mm(a, b)`` contract (a int8 [M, K], b int8 [K, N] -> int32
[M, N]) and hands b to the NT kernel as the [N, K] operand it usually is
(``b`` is most often ``weight.T`` of a [N, K]-stored weight, so the view is
free; ``int_mm_mps.py:97-103``). Before the first routed call a one-time
adversarial canary (``int_mm_mps.py:54-87``: -128 / 127 corners, ragged K,
shapes (3, 129, 5) and (16, 4096, 32), seed 0) is compared with an int64
product on the CPU.

Differences from the reference, by design: calls that are not int8 x int8
2-D on a ROCm device keep the stock op (there is a native ROCm kernel, so no
fp32 emulation tier exists), and a failed canary or kernel error raises
instead of latching onto a slower path, so a wrong or missing HIP path is
never hidden.
"""
import torch

from .. import ops
from .._lib import C4QError
from . import _common

TAG = "[cdna4q/int_mm]"

_orig = None
_installed = False
_canary_ok = False


def _canary(device):
    """One-time parity gate (reference ``int_mm_mps.py:69-82``)."""
    global _canary_ok
    if _canary_ok:
        return
    g = torch.Generator().manual_seed(0)
    for M, K, N in ((3, 129, 5), (16, 4096, 32)):
        a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
        b = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8)
        a[:, 0] = -128
        b[0, :] = 127
        ref = (a.long() @ b.long()).to(torch.int32)
        out = ops.int_mm(a.to(device), b.to(device))
        if not torch.equal(out.cpu(), ref):
            raise C4QError(f"{TAG} int8 kernel parity canary FAILED at ({M},{K},{N})")
    _canary_ok = True


def _eligible(a, b):
    return (_common.on_device(a, b) and a.dtype == torch.int8 and b.dtype == torch.int8
            and a.dim() == 2 and b.dim() == 2)


def _int_mm_rocm(a, b):
    """Replacement for ``torch._int_mm`` (reference ``int_mm_mps.py:90-110``)."""
    if _eligible(a, b):
        _canary(a.device)
        return ops.int_mm(a, b)
    return _orig(a, b)


def install():
    """Route ``torch._int_mm`` on ROCm tensors through the kernel. Returns True
    when installed (a ROCm device is present and the canary passed)."""
    global _orig, _installed
    if _installed:
        return True
    if not hasattr(torch, "_int_mm") or not _common.rocm_available():
        return False
    _canary(torch.device("cuda", torch.cuda.current_device()))
    _orig = torch._int_mm
    torch._int_mm = _int_mm_rocm
    _installed = True
    print(f"{TAG} torch._int_mm on ROCm routed to the exact int8 MFMA kernel (canary passed).")
    return True


def uninstall():
    global _installed
    if _installed:
        torch._int_mm = _orig
        _installed = False
