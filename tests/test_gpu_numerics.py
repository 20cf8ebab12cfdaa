"""Exhaustive checks of the gfx950 conversion instructions the kernels use,
against the library's integer-only reference roundings, over all 2^32 float
bit patterns (NaN inputs excluded: both sides give a NaN)."""
import ctypes
import pathlib

import pytest
import torch

pytestmark = pytest.mark.gpu

LIB = pathlib.Path(__file__).resolve().parent / "native" / "libc4q_probe.so"


@pytest.fixture(scope="module")
def probe():
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(LIB))
    lib.c4q_probe_cvt_exhaustive.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.c4q_probe_cvt_exhaustive.restype = ctypes.c_int
    lib.c4q_probe_div_bf16_exhaustive.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.c4q_probe_div_bf16_exhaustive.restype = ctypes.c_int
    return lib


@pytest.mark.parametrize("which,name", [(0, "bf16"), (1, "f16")])
def test_hw_round_matches_reference_rne(dev, probe, which, name):
    out = torch.tensor([0, 0xFFFFFFFF], dtype=torch.int64, device=dev)
    rc = probe.c4q_probe_cvt_exhaustive(which, out.data_ptr(),
                                        torch.cuda.current_stream(dev).cuda_stream)
    assert rc == 0
    bad, first = out.cpu().tolist()
    assert bad == 0, f"{name}: {bad} float inputs round differently (first 0x{first & 0xFFFFFFFF:08x})"


def test_reciprocal_quotient_matches_division_for_bf16_operands(dev, probe):
    """The rowwise bf16 quantizers divide by the row's bf16 scale with one
    reciprocal per row and a fused residual step per element; after bf16
    rounding that equals the correctly rounded quotient for every pair of
    bf16 operands (the quantizers' quotients stay below 2^8)."""
    out = torch.tensor([0, 0xFFFFFFFF], dtype=torch.int64, device=dev)
    rc = probe.c4q_probe_div_bf16_exhaustive(out.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
    assert rc == 0
    bad, first = out.cpu().tolist()
    assert bad == 0, f"{bad} pairs differ (first x<<16|s = 0x{first & 0xFFFFFFFF:08x})"
