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
    lib.c4q_probe_e4m3_exhaustive.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.c4q_probe_e4m3_exhaustive.restype = ctypes.c_int
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


@pytest.mark.parametrize("which,name", [(0, "e4m3 pair conversion, every float pattern"),
                                        (1, "bf16 x, bf16 amax quotient"),
                                        (2, "f16 x, f16 amax quotient")])
def test_fp8_pertensor_quantizer_arithmetic(dev, probe, which, name):
    """The per-tensor fp8 activation quantizer's arithmetic: the hardware
    pair conversion equals the integer e4m3 rounding of the clamped value for
    every float (NaN included, both slots), and the reciprocal quotient gives
    the IEEE quotient's e4m3 code for every 16-bit x and every scale the
    quantizer forms from a 16-bit amax >= |x|."""
    out = torch.tensor([0, 0xFFFFFFFF], dtype=torch.int64, device=dev)
    rc = probe.c4q_probe_e4m3_exhaustive(which, out.data_ptr(),
                                         torch.cuda.current_stream(dev).cuda_stream)
    assert rc == 0
    bad, first = out.cpu().tolist()
    assert bad == 0, f"{name}: {bad} mismatches (first 0x{first & 0xFFFFFFFF:08x})"
