"""ctypes binding of libcdna4q.so (the C ABI declared in include/cdna4q.h).

The shared library is built in-tree (``make -C <this package dir>``) and
loaded from this directory only. A missing or stale library raises
``C4QError``; nothing here falls back to another implementation.
"""
import ctypes
import os

LIB_NAME = "libcdna4q.so"
ABI_VERSION = 1

# element type codes (C4Q_BF16 / C4Q_F16 / C4Q_F32)
BF16, F16, F32 = 0, 1, 2
# scale layouts (C4Q_SCALE_*)
SCALE_NONE, SCALE_TENSOR, SCALE_VECTOR = 0, 1, 2


class C4QError(RuntimeError):
    """A cdna4q entry point rejected its arguments or failed to launch."""


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int

_SIGNATURES = {
    "c4q_i8_gemm_nt_i32": [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P],
    "c4q_i8_gemm_nt_fused": [_P, _I64, _P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _P],
    "c4q_i8_gemm_nt_fused_cs": [_P, _I64, _P, _I64, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _P],
    "c4q_i8_gemm_nt_fused_cs_f16": [_P, _I64, _P, _I64, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _P],
    "c4q_i8_gemm_nt_fused_cs_qkv": [_P, _I64, _P, _I64, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64,
                                    _I64, _P],
    "c4q_i8_gemm_nt_fused_cs_qkv_rms_rope": [_P, _I64, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P,
                                             _P, _I64, _I64, _I64, _I64, ctypes.c_float, _P],
    "c4q_i8_gemm_nt_fused_cs_qkv_lora_part": [_P, _I64, _P, _I64, _P, _P, _P, _P, _P, _P, _P,
                                              _I64, _I64, _I64, _I64, _I, ctypes.c_float,
                                              ctypes.c_float, _P],
    "c4q_i8_quant_rowwise": [_P, _I, _I64, _P, _I64, _P, _I64, _I64, _P],
    "c4q_i8_swiglu_rot_quant": [_P, _I64, _I64, _P, _P, _P, _P],
    "c4q_i8_mlp_bridge_prequant": [_P, _I64, _P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                   _P, _P, _P, _P, _P],
    "c4q_i8_mlp_bridge_prequant_noalloc": [_P, _I64, _P, _I64, _P, _P, _P, _P, _I64, _I64, _I64,
                                           _P, _P, _P],
    "c4q_i8_merge_rot_quant": [_P, _I64, _I64, _I64, _I64, _I, _P, _P, _P],
    "c4q_i8_swiglu_rot": [_P, _I64, _I64, _P, _P, _P],
    "c4q_f8_gemm_nt_scaled": [_P, _I64, _P, _I64, _P, _I, _I64, _P, _I, _P, _I, _P, _P, _I,
                              _I64, _I64, _I64, _P],
    "c4q_f8_quant_pertensor": [_P, _I, _I64, _P, _P, _P, _P],
    "c4q_fp8_dequant": [_P, _I64, _P, _P, _I, _P],
    "c4q_w8a16_gemm_nt": [_P, _I, _I64, _P, _I64, _P, _P, _I, _I64, _P, _I, _P,
                          _I64, _I64, _I64, _P],
    "c4q_i8_ffn_pair": [_P, _I64, _P, _P, _I64, _P, _I64, _P, _P, _P, _P, _P,
                        _I64, _I64, _I64, _P],
    "c4q_bf16_ffn_pair": [_P, _I64, _P, _P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _P],
}

_lib = None


def lib_path():
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)


def exported_symbols():
    """Names of every entry point the ctypes layer binds (the header's set)."""
    return ["c4q_last_error", "c4q_abi_version"] + sorted(_SIGNATURES)


def load():
    """Load (once) and return the library, with argtypes bound."""
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not os.path.exists(path):
        raise C4QError(f"{path} is not built; run `make -C {os.path.dirname(path)}`")
    lib = ctypes.CDLL(path)
    lib.c4q_last_error.restype = ctypes.c_char_p
    lib.c4q_last_error.argtypes = []
    lib.c4q_abi_version.restype = ctypes.c_int
    lib.c4q_abi_version.argtypes = []
    ver = lib.c4q_abi_version()
    if ver != ABI_VERSION:
        raise C4QError(f"{path}: ABI version {ver}, this binding expects {ABI_VERSION}; rebuild it")
    for name, args in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    _lib = lib
    return lib


def call(name, *args):
    """Invoke entry point `name`; raise C4QError on a non-zero status."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != 0:
        msg = lib.c4q_last_error().decode("utf-8", "replace")
        raise C4QError(f"{name} failed (status {status}): {msg}")
