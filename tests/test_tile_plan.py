"""Tile plans of the MFMA GEMM launches, run on the host (no GPU).

A GEMM whose last round of big tiles would leave most CUs idle runs its
whole rounds as one launch and the leftover tiles, split into smaller
pieces, as a second launch. tests/native/libc4q_probe.so exposes the
library's own planning and tile-mapping functions (plan_launches, tile_at);
these tests check that the launches of a plan compute every output cell
exactly once, for the BASELINE shapes, ragged edges, FFN pairs and several
CU counts.
"""
import ctypes
import pathlib
import subprocess

import numpy as np
import pytest

NATIVE = pathlib.Path(__file__).resolve().parent / "native"
LIB = NATIVE / "libc4q_probe.so"

TILE_256 = 0
TILE_128_K128 = 4
TILE_64x128_K128 = 5
TILE_64x64_KG4 = 7


@pytest.fixture(scope="module")
def probe():
    if not LIB.exists():
        subprocess.run(["make", "-C", str(NATIVE)], check=True)
    lib = ctypes.CDLL(str(LIB))
    f = lib.c4q_probe_tile_plan
    f.argtypes = [ctypes.c_int64] * 3 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                         ctypes.c_void_p]
    f.restype = ctypes.c_int
    return f


def plan(probe, M, n_rows_b, K, cus):
    cover = np.zeros(-(-M // 64) * -(-n_rows_b // 64), np.int32)
    info = np.zeros(8, np.int64)
    assert probe(M, n_rows_b, K, cus, cover.ctypes.data, cover.size, info.ctypes.data) == 0
    return cover, info


# (M, rows of the B tile space, K): BASELINE C1-C5 linears (FLUX QKV / out /
# MLP up / down, C1 int8, Krea2 pair as 2 * N_out), ragged and tiny shapes
SHAPES = [
    (9216, 9216, 3072), (9216, 3072, 3072), (9216, 12288, 3072), (9216, 3072, 12288),
    (1024, 3072, 3072), (4096, 2 * 12288, 3072), (4352, 4352, 512), (4312, 4280, 512),
    (4352, 2 * 2176, 512), (9280, 9216, 3072), (300, 1000, 64), (1, 16, 16), (65, 129, 32),
    (8192, 12288, 3072), (16384, 5120, 5120), (2000, 70000, 128), (5000, 5000, 16),
]


@pytest.mark.parametrize("cus", [256, 304, 80])
@pytest.mark.parametrize("M,NB,K", SHAPES)
def test_every_cell_computed_once(probe, M, NB, K, cus):
    cover, info = plan(probe, M, NB, K, cus)
    assert info[0] in (1, 2)
    assert cover.min() == 1 and cover.max() == 1, (
        f"{M}x{NB}: cells covered {cover.min()}..{cover.max()} (plan {info.tolist()})")


def test_random_shapes_computed_once(probe):
    rng = np.random.default_rng(0)
    for _ in range(300):
        M = int(rng.integers(1, 12000))
        NB = int(rng.integers(1, 12000))
        K = int(rng.choice([16, 64, 512, 3072, 12288]))
        cus = int(rng.choice([256, 304, 120, 8]))
        cover, info = plan(probe, M, NB, K, cus)
        assert cover.min() == 1 and cover.max() == 1, (M, NB, K, cus, info.tolist())


def test_c2_qkv_runs_whole_rounds_then_split_tail(probe):
    """C2 fused QKV on 256 CUs: 36 x 36 = 1296 tiles of 256x256 are five whole
    rounds (1280 tiles) plus 16; those 16 run as 256 split-K pieces of 64x64,
    one per CU."""
    _, info = plan(probe, 9216, 9216, 3072, 256)
    assert info[0] == 2
    assert (info[1], info[2]) == (TILE_256, 1280)
    assert (info[3], info[4]) == (TILE_64x64_KG4, 16 * 16)
    assert (info[6], info[7]) == (4, 4)


def test_split_k_tile_is_never_the_main_tile(probe):
    """The split-K tile only takes leftover pieces (C1's 1024 x 3072 runs as
    one launch of 64x128 tiles)."""
    _, info = plan(probe, 1024, 3072, 3072, 256)
    assert info[0] == 1 and info[1] == TILE_64x128_K128
    rng = np.random.default_rng(1)
    for _ in range(200):
        M, NB = int(rng.integers(1, 20000)), int(rng.integers(1, 20000))
        _, info = plan(probe, M, NB, 3072, 256)
        assert info[1] != TILE_64x64_KG4, (M, NB, info.tolist())


def test_whole_rounds_need_no_tail(probe):
    """8192 x 12288 is 1536 = 6 x 256 tiles: one launch."""
    _, info = plan(probe, 8192, 12288, 3072, 256)
    assert info[0] == 1 and info[1] == TILE_256 and info[2] == 1536


def test_ragged_out_proj_keeps_one_launch(probe):
    """C2 out-proj (432 tiles): a second round of big tiles is cheaper than
    splitting 176 leftover tiles."""
    _, info = plan(probe, 9216, 3072, 3072, 256)
    assert info[0] == 1 and info[1] == TILE_256


def test_tail_of_128x128_pieces(probe):
    """4608 x 4608: 324 tiles, 68 leftover; as 128x128 pieces (272) they fill
    one round of two workgroups per CU."""
    _, info = plan(probe, 4608, 4608, 1024, 256)
    assert info[0] == 2 and (info[1], info[2]) == (TILE_256, 256)
    assert (info[3], info[4]) == (TILE_128_K128, 68 * 4) and (info[6], info[7]) == (2, 2)


# ------------------------------------------------- head-spanning tile set ---
# HeadTiles (the QKV + RMSNorm/RoPE epilogue): every wave spans one whole
# 128-column head, so every tile's columns start at a multiple of 128. The
# planner picks among ids 0 and 1 (id 2, the 4-wave 256x256 tile, is only
# forced for sweeps).
HEAD_256 = 0       # 256x256, 8 waves of 64x128
HEAD_128 = 1       # 128x128, 2 waves of 64x128


@pytest.fixture(scope="module")
def head_probe():
    if not LIB.exists():
        subprocess.run(["make", "-C", str(NATIVE)], check=True)
    lib = ctypes.CDLL(str(LIB))
    f = lib.c4q_probe_head_tile_plan
    f.argtypes = [ctypes.c_int64] * 3 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                         ctypes.c_void_p]
    f.restype = ctypes.c_int
    return f


# (M, N = 3 * heads * 128, K): H3 (56 heads, hidden 5376) at its three token
# counts, 24 heads (FLUX width), an odd head count, small M
HEAD_SHAPES = [(5378, 21504, 5376), (8192, 21504, 5376), (17000, 21504, 5376),
               (4096, 9216, 3072), (4608, 3 * 7 * 128, 1024), (65, 384, 128), (300, 3 * 5 * 128, 64)]


@pytest.mark.parametrize("cus", [256, 304, 80])
@pytest.mark.parametrize("M,N,K", HEAD_SHAPES)
def test_head_plan_every_cell_once(head_probe, M, N, K, cus):
    cover, info = plan(head_probe, M, N, K, cus)
    assert info[0] in (1, 2)
    assert {info[1], info[3] if info[0] == 2 else HEAD_256} <= {HEAD_256, HEAD_128}
    assert cover.min() == 1 and cover.max() == 1, (M, N, K, cus, info.tolist())


def test_head_plan_random_shapes(head_probe):
    rng = np.random.default_rng(2)
    for _ in range(200):
        M = int(rng.integers(1, 20000))
        N = 384 * int(rng.integers(1, 64))
        K = int(rng.choice([64, 1024, 5376]))
        cus = int(rng.choice([256, 304, 120]))
        cover, info = plan(head_probe, M, N, K, cus)
        assert cover.min() == 1 and cover.max() == 1, (M, N, K, cus, info.tolist())


def test_head_plan_h3_8192(head_probe):
    """H3 at 8192 tokens: 32 x 84 = 2688 tiles of 256x256, ten whole rounds
    on 256 CUs (2560) and 128 leftover tiles as 512 pieces of 128x128, one
    round of two workgroups per CU."""
    _, info = plan(head_probe, 8192, 21504, 5376, 256)
    assert info[0] == 2 and (info[1], info[2]) == (HEAD_256, 2560)
    assert (info[3], info[4]) == (HEAD_128, 512) and (info[6], info[7]) == (2, 2)


# ------------------------------------------------------- W8A16 tile set ---
# W8A16Tiles: the general ids plus 224x256 (one-wave-per-SIMD W8A16 kernel
# with seven 32-row block rows per wave), which the cost model takes where
# 256-row tiles would leave most of a last round idle. Coverage is counted
# in cells of 32 rows x 64 columns.
W8A16_224 = 8


@pytest.fixture(scope="module")
def w8a16_probe():
    if not LIB.exists():
        subprocess.run(["make", "-C", str(NATIVE)], check=True)
    lib = ctypes.CDLL(str(LIB))
    f = lib.c4q_probe_w8a16_tile_plan
    f.argtypes = [ctypes.c_int64] * 3 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                         ctypes.c_void_p]
    f.restype = ctypes.c_int
    return f


def plan32(probe, M, n_rows_b, K, cus):
    cover = np.zeros(-(-M // 32) * -(-n_rows_b // 64), np.int32)
    info = np.zeros(8, np.int64)
    assert probe(M, n_rows_b, K, cus, cover.ctypes.data, cover.size, info.ctypes.data) == 0
    return cover, info


@pytest.mark.parametrize("cus", [256, 304, 80])
@pytest.mark.parametrize("M,NB,K", SHAPES)
def test_w8a16_plan_every_cell_once(w8a16_probe, M, NB, K, cus):
    cover, info = plan32(w8a16_probe, M, NB, K, cus)
    assert info[0] in (1, 2)
    assert cover.min() == 1 and cover.max() == 1, (M, NB, K, cus, info.tolist())


def test_w8a16_plan_random_shapes(w8a16_probe):
    rng = np.random.default_rng(3)
    for _ in range(300):
        M = int(rng.integers(1, 12000))
        NB = int(rng.integers(1, 12000))
        K = int(rng.choice([16, 64, 512, 3072, 12288]))
        cus = int(rng.choice([256, 304, 120, 8]))
        cover, info = plan32(w8a16_probe, M, NB, K, cus)
        assert cover.min() == 1 and cover.max() == 1, (M, NB, K, cus, info.tolist())
        if info[1] == W8A16_224:
            assert info[0] == 1, "the 224-row tile takes no tail launch"


def test_w8a16_out_proj_takes_224_rows(w8a16_probe):
    """C2 / C5 out-projection and C5 MLP-down (9216 x 3072): 432 tiles of
    256x256 are 1.69 rounds on 256 CUs; 42 x 12 = 504 tiles of 224x256 are
    1.97 rounds of 7/8 the work each."""
    for K in (3072, 12288):
        _, info = plan32(w8a16_probe, 9216, 3072, K, 256)
        assert info[0] == 1 and (info[1], info[2]) == (W8A16_224, 42 * 12)


def test_w8a16_qkv_keeps_256_rows(w8a16_probe):
    """C2 QKV (9216 x 9216): five whole rounds of 256x256 plus 256 split-K
    pieces cost less than six rounds of 224x256 (1512 tiles)."""
    _, info = plan32(w8a16_probe, 9216, 9216, 3072, 256)
    assert info[0] == 2 and (info[1], info[2]) == (TILE_256, 1280)
    assert (info[3], info[4]) == (TILE_64x64_KG4, 256)


def test_w8a16_few_tiles_take_split_k(w8a16_probe):
    """Few-tile W8A16 GEMMs (one round of 64x64 split-K pieces covers them)
    run on the split-K tile as the main launch when K >= 1024: M = 128,
    N = 3072 is 96 pieces; with K = 512 the 64x128 tile stays."""
    for M, N in ((65, 3072), (128, 3072), (256, 3072)):
        cover, info = plan32(w8a16_probe, M, N, 3072, 256)
        assert info[0] == 1 and info[1] == TILE_64x64_KG4, (M, N, info.tolist())
        assert cover.min() == 1 and cover.max() == 1
    _, info = plan32(w8a16_probe, 128, 3072, 512, 256)
    assert info[1] != TILE_64x64_KG4
    _, info = plan32(w8a16_probe, 1024, 3072, 3072, 256)     # 768 pieces: three rounds
    assert info[1] != TILE_64x64_KG4


def test_w8a16_one_128_tile_per_cu(w8a16_probe):
    """A 64x128 plan with more tiles than CUs whose 128x128 tiles fit one per
    CU takes the 128x128 tile; 512 x 3072 (192 tiles of 64x128) keeps
    64x128."""
    for M, N in ((1024, 3072), (256, 9216), (128, 18432)):
        cover, info = plan32(w8a16_probe, M, N, 3072, 256)
        assert info[0] == 1 and info[1] == TILE_128_K128, (M, N, info.tolist())
        assert cover.min() == 1 and cover.max() == 1
    _, info = plan32(w8a16_probe, 512, 3072, 3072, 256)
    assert info[1] == TILE_64x128_K128
