"""Shared helpers: bit views between torch and numpy, seeded generators,
tolerance checks."""
import numpy as np
import torch


def gen(seed):
    return torch.Generator().manual_seed(seed)


def bits16(t):
    """bf16/f16 tensor -> numpy uint16 bit array (on CPU)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits16(b, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(dtype)


def u8(t):
    """fp8 tensor -> numpy uint8 codes."""
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def bf16_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def assert_bits_equal(got, want, what=""):
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    bad = np.flatnonzero(got.reshape(-1) != want.reshape(-1))
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} of {got.size} elements differ; first at flat "
                             f"{i}: got {got.reshape(-1)[i]!r} want {want.reshape(-1)[i]!r}")


# Floating-point tolerance used for fp32-accumulating GEMMs compared with the
# oracle's exactly-rounded fp32 dot product: the accumulation-order error is
# far below one bf16 ulp, so outputs may differ by at most one final-rounding
# step. Stated bounds:
#   max |out - ref|   <= 2^-7 * max|ref|      (one bf16 ulp at the top binade)
#   ||out - ref||_2   <= 2^-9 * ||ref||_2     (relative L2)
MAXABS_REL = 2.0 ** -7
RELL2 = 2.0 ** -9


def assert_close(out, ref, what="", maxabs_rel=MAXABS_REL, rel_l2=RELL2):
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert out.shape == ref.shape, f"{what}: shape {out.shape} != {ref.shape}"
    assert np.isfinite(out).all(), f"{what}: non-finite output"
    scale = np.abs(ref).max() if ref.size else 0.0
    err = np.abs(out - ref)
    mx = err.max() if err.size else 0.0
    l2 = np.linalg.norm(out - ref) / max(np.linalg.norm(ref), 1e-30)
    assert mx <= maxabs_rel * scale + 1e-30, f"{what}: max-abs {mx:.3e} > {maxabs_rel:.2e}*{scale:.3e}"
    assert l2 <= rel_l2, f"{what}: rel-L2 {l2:.3e} > {rel_l2:.2e}"
    return mx, l2
