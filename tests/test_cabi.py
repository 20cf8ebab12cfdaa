"""C ABI checks that need no GPU: the library loads, exports exactly what
include/cdna4q.h declares, and rejects bad arguments before touching the
device (argument validation is host-only, so these calls enqueue nothing)."""
import ctypes
import pathlib
import re

import pytest

import cdna4q._lib as lib

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _header_functions():
    text = (ROOT / "include" / "cdna4q.h").read_text()
    return sorted(set(re.findall(r"^(?:int|const char\*)\s+(c4q_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    assert _header_functions() == sorted(lib.exported_symbols())


def test_library_loads_and_exports_every_symbol():
    L = lib.load()
    assert L.c4q_abi_version() == lib.ABI_VERSION
    for name in _header_functions():
        assert hasattr(L, name), name


def _status(name, *args):
    L = lib.load()
    return getattr(L, name)(*args), L.c4q_last_error().decode()


def test_negative_shape_rejected():
    st, msg = _status("c4q_i8_gemm_nt_i32", None, 0, None, 0, None, 0, -1, 4, 4, None)
    assert st == -2 and "negative" in msg


def test_short_row_stride_rejected():
    st, msg = _status("c4q_i8_gemm_nt_i32", None, 8, None, 16, None, 4, 4, 4, 16, None)
    assert st == -2 and "stride" in msg


def test_null_pointer_rejected():
    st, msg = _status("c4q_i8_gemm_nt_fused", None, 16, None, 16, None, 16, None, None,
                      4, 4, 16, None)
    assert st == -1 and "null" in msg


def test_bad_dtype_rejected():
    st, msg = _status("c4q_f8_gemm_nt_scaled", None, 16, None, 16, None, 7, 16, None, 0, None,
                      0, None, None, 0, 4, 4, 16, None)
    assert st == -1 and "dtype" in msg
    st, msg = _status("c4q_i8_quant_rowwise", None, 2, 16, None, 16, None, 4, 16, None)
    assert st == -1


def test_act_table_requires_bf16_output():
    st, msg = _status("c4q_w8a16_gemm_nt", None, 0, 16, None, 16, None, None, 2, 16, None, 0,
                      ctypes.c_void_p(16), 4, 4, 16, None)
    assert st == -5


def test_empty_problems_are_noops():
    # M == 0 or N == 0 enqueues nothing and needs no pointers
    assert _status("c4q_i8_gemm_nt_i32", None, 16, None, 16, None, 0, 0, 0, 16, None)[0] == 0
    assert _status("c4q_i8_quant_rowwise", None, 0, 16, None, 16, None, 0, 16, None)[0] == 0
    assert _status("c4q_fp8_dequant", None, 0, None, None, 0, None)[0] == 0


def test_ops_reject_cpu_tensors():
    import torch
    import cdna4q.ops as ops
    with pytest.raises(RuntimeError):
        ops.i8_matmul2d_nt(torch.zeros(4, 16, dtype=torch.int8), torch.zeros(4, 16, dtype=torch.int8))
    with pytest.raises(RuntimeError):
        ops.i8_quant_rowwise(torch.zeros(4, 16))


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(lib, "_lib", None)
    monkeypatch.setattr(lib, "lib_path", lambda: str(tmp_path / "libcdna4q.so"))
    with pytest.raises(lib.C4QError, match="not built"):
        lib.load()
