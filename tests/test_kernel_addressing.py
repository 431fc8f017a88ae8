"""Host-side address audits of the hand-written kernels (CPU only, no GPU code runs).

Each audit enumerates every global and LDS byte the kernel's launch would touch for a shape and
checks it against the operand sizes and the LDS allocation, using the same index functions the
kernel is compiled from."""
import itertools
import random

import pytest

CFG4_SHAPES = [(4096, 3584), (3584, 3072), (37888, 3584), (3584, 18944), (28672, 4096)]


@pytest.mark.parametrize("N,K", CFG4_SHAPES)
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
def test_h4mv_stream_in_bounds_model_shapes(lib, N, K, M):
    assert lib.fp8kv_h4mv_audit(N, K, M) == 0


def test_h4mv_stream_in_bounds_random_shapes(lib):
    rng = random.Random(0)
    for _ in range(300):
        N = rng.choice([1, 2, 15, 16, 17, 31, 33, 100, 1000, 4097]) + rng.randrange(0, 3)
        K = 512 * rng.randrange(1, 41)
        M = rng.randrange(1, 9)
        assert lib.fp8kv_h4mv_audit(N, K, M) == 0, (N, K, M)


def test_h4mv_register_path_shapes_are_reported(lib):
    for N, K, M in itertools.product([1, 64], [32, 96, 4128], [1, 9, 16]):
        assert lib.fp8kv_h4mv_audit(N, K, M) == 1


@pytest.mark.parametrize("x_mode", [1, 2])
@pytest.mark.parametrize("rt", [1, 2, 4])
def test_h4mv_stream_in_bounds_every_row_tile_count(lib, rt, x_mode):
    """Every row-tile count and activation path the planner can pick (forced through the tuning
    hook), on the model shapes and on random ones, including N not a multiple of 16 rt."""
    rng = random.Random(rt + 10 * x_mode)
    try:
        lib.fp8kv_h4mv_tune(0, 0, rt, x_mode)
        for N, K in CFG4_SHAPES:
            for M in (1, 3, 8):
                assert lib.fp8kv_h4mv_audit(N, K, M) == 0, (N, K, M)
        for _ in range(120):
            N = rng.choice([1, 15, 17, 33, 63, 65, 100, 1000, 4097]) + rng.randrange(0, 3)
            K = 512 * rng.randrange(1, 41)
            M = rng.randrange(1, 9)
            assert lib.fp8kv_h4mv_audit(N, K, M) == 0, (N, K, M)
    finally:
        lib.fp8kv_h4mv_tune(0, 0, 0, 0)


@pytest.mark.parametrize("wgs", [0, 512])
@pytest.mark.parametrize("order", [1, 2])
@pytest.mark.parametrize("depth", [2, 3])
def test_h4mv_kslice_in_bounds(lib, depth, order, wgs):
    """The K-slice kernel forced on every shape it accepts, both tile orders and two workgroup
    targets: model shapes, tile counts per workgroup from 1 to 16, more workgroups than CUs,
    partial last tiles, random shapes; every tile is covered exactly once and every output row
    stored exactly once."""
    rng = random.Random(depth)
    try:
        lib.fp8kv_h4mv_kslice_tune(1, depth, order, wgs)
        lib.fp8kv_h4mv_mx_tune(2, 0, 0)                 # M = 3, 8 on the K-slice kernel too
        shapes = [(N, K) for N, K in CFG4_SHAPES if K <= 4096]
        shapes += [(16, 512), (4112, 1024), (8208, 2048), (65536, 512), (66048, 512)]
        # partial last tiles (N % 16 != 0): the lm_head vocabulary, the smallest N, random N
        shapes += [(128167, 3584), (17, 512), (31, 1024), (4097, 1024), (40003, 3584)]
        # the batched form (more tiles than one round holds) with a partial last tile
        shapes += [(70003, 2048), (70003, 4096), (70000, 4096)]
        for _ in range(60):
            shapes.append((16 * rng.randrange(1, 5000), 512 * rng.randrange(1, 9)))
        for _ in range(30):
            shapes.append((rng.randrange(16, 80000), 512 * rng.randrange(1, 9)))
        for N, K in shapes:
            for M in (1, 3, 8):
                assert lib.fp8kv_h4mv_audit(N, K, M) == 0, (N, K, M)
    finally:
        lib.fp8kv_h4mv_kslice_tune(0, 0, 0, 0)
        lib.fp8kv_h4mv_mx_tune(0, 0, 0)


@pytest.mark.parametrize("wgs", [0, 7, 300])
@pytest.mark.parametrize("depth", [2, 3])
def test_h4mv_m1_in_bounds(lib, depth, wgs):
    """The M = 1 kernel forced on every shape it accepts: model shapes, ragged N (the last tile's
    rows clamped), K from one step up, fewer or more workgroups than CUs (1..16 tiles per
    workgroup, waves without a tile): every tile covered once, the activation row copied and
    converted once, a block's four groups in one quad of lanes."""
    rng = random.Random(depth + wgs)
    try:
        lib.fp8kv_h4mv_m1_tune(1, depth, wgs)
        shapes = list(CFG4_SHAPES) + [(1, 512), (15, 512), (17, 1024), (4097, 2048),
                                      (16 * 4096 + 3, 4096), (250, 1536), (33, 32768), (1000, 32768)]
        for _ in range(30):
            shapes.append((rng.randrange(1, 20000), 512 * rng.randrange(1, 25)))
        for N, K in shapes:
            assert lib.fp8kv_h4mv_audit(N, K, 1) == 0, (N, K)
    finally:
        lib.fp8kv_h4mv_m1_tune(0, 0, 0)


@pytest.mark.parametrize("wgs", [0, 7, 300])
@pytest.mark.parametrize("depth", [2, 3])
def test_h4mv_mx_in_bounds(lib, depth, wgs):
    """The M = 2 .. 8 hi / lo kernel forced on every shape it accepts, at two, four and eight
    activation rows (M = 2, 3, 4, 5, 8): model shapes, ragged N, K from one step up, 1..16 tiles
    per workgroup and waves without a tile.  Every tile covered once, every LDS byte of the rows
    copied once, each 32-byte unit converted by one thread with its block partner in the
    neighbouring lane, every fragment and scale read inside its row."""
    import ctypes
    rng = random.Random(depth + wgs + 1)
    out = (ctypes.c_int * 6)()
    try:
        lib.fp8kv_h4mv_mx_tune(1, depth, wgs)
        shapes = list(CFG4_SHAPES) + [(1, 512), (15, 512), (17, 1024), (4097, 2048), (250, 1536),
                                      (100, 8192), (16 * 4096 + 3, 4096)]
        for _ in range(30):
            shapes.append((rng.randrange(1, 20000), 512 * rng.randrange(1, 17)))
        used = 0
        for N, K in shapes:
            for M in (2, 3, 4, 5, 8):
                assert lib.fp8kv_h4mv_audit(N, K, M) == 0, (N, K, M)
                assert lib.fp8kv_h4mv_plan(N, K, M, out) == 0
                used += out[0] == 4
        assert used > len(shapes)
    finally:
        lib.fp8kv_h4mv_mx_tune(0, 0, 0)


def test_h4mv_plan_picks_the_measured_kernels(lib):
    """The default plans: M = 1 kernel for cfg1, gate/up and the lm_head vocabulary at M = 1, the hi / lo kernel at
    M = 2 .. 8 (one round of workgroups; conversion chunks of two steps for workgroups of more
    than four waves), the K-slice kernel for the lm_head vocabulary, the streaming kernel for the
    short-N configs[4] linears."""
    import ctypes
    out = (ctypes.c_int * 6)()

    def kernel(N, K, M):
        assert lib.fp8kv_h4mv_plan(N, K, M, out) == 0
        return out[0]
    for N, K in ((28672, 4096), (37888, 3584)):
        assert kernel(N, K, 1) == 3
        assert [kernel(N, K, M) for M in (2, 3, 4, 5, 8)] == [4, 4, 4, 4, 4]
    assert kernel(28672, 4096, 4) == 4 and out[5] == 4 and out[1] == 448 and out[2] == 4
    assert kernel(28672, 4096, 8) == 4 and out[5] == 8 and out[1] == 256 and out[2] == 7
    assert [kernel(128167, 3584, M) for M in (3, 8)] == [5, 5]
    # M = 1 at the lm_head vocabulary: more tiles than one round holds at any wave count the LDS
    # allows, so 4-wave workgroups over several rounds
    assert kernel(128167, 3584, 1) == 3 and out[1] == 2003 and out[2] == 4 and out[3] == 2
    assert lib.fp8kv_h4mv_audit(128167, 3584, 1) == 0
    # ... and the same form of the hi / lo kernel at M = 2 (two rows in LDS)
    assert kernel(128167, 3584, 2) == 4 and out[1] == 2003 and out[2] == 4 and out[5] == 2
    assert lib.fp8kv_h4mv_audit(128167, 3584, 2) == 0
    for N, K in ((4096, 3584), (3584, 3072), (3584, 18944)):
        assert [kernel(N, K, M) for M in (1, 4, 8)] == [1, 1, 1]
    assert kernel(64, 96, 2) == 0
    assert lib.fp8kv_h4mv_plan(64, 96, 17, out) != 0
