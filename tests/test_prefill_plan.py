"""Host-side prefill launch planner (CPU only, no GPU code runs): which kernel, block pairing and
grid the entry points launch for a shape, including the plans the GPU parity cases rely on."""
import ctypes

import pytest

SPLIT_GQA = [6, 12, 4, 8, 16]          # GQA of key-split shape s (tuning index 8 + s, 13 + s paired)
FIELDS = ("split", "shape", "nb", "paired", "ntb", "grid_x", "grid_z", "threads")


def plan(lib, hq, hkv, num_seqs, max_query_len, ctx_hint):
    out = (ctypes.c_int * 8)()
    st = lib.fp8kv_prefill_plan(hq, hkv, num_seqs, max_query_len, ctx_hint, ctypes.addressof(out))
    assert st == 0, st
    return dict(zip(FIELDS, list(out)))


def check_cover(p, hkv, num_seqs, n16):
    """Every token block of every (sequence, kv head) has a workgroup, and the grid matches."""
    per_wg = 2 if p["paired"] else p["nb"]
    assert p["ntb"] * per_wg >= n16
    assert p["grid_x"] == p["ntb"] * hkv and p["grid_z"] == num_seqs
    if hkv <= 8 and 8 % hkv == 0:
        assert p["ntb"] % (8 // hkv) == 0            # XCD-aware grid: whole rounds of ranks


@pytest.fixture
def tuned(lib):
    yield lib
    lib.fp8kv_prefill_tune(-1)


@pytest.mark.parametrize("gqa", SPLIT_GQA)
def test_split_paired_above_one_round(lib, gqa):
    """600 new tokens after 1000 cached at 8 kv heads: 38 blocks x 8 heads exceed 256 workgroups,
    so the key-split kernel pairs blocks (19 ranks per head)."""
    p = plan(lib, 8 * gqa, 8, 1, 600, 1600)
    assert (p["split"], p["shape"], p["paired"], p["ntb"]) == (1, SPLIT_GQA.index(gqa), 1, 19)
    assert p["threads"] == 512
    check_cover(p, 8, 1, 38)


def test_split_paired_varlen(lib):
    """Varlen [1100, 1030, 300] at GQA 6 / 4 kv heads: 69 blocks, paired into 35 ranks, rounded
    up to whole XCD rounds of 2."""
    p = plan(lib, 24, 4, 3, 1100, 1100)
    assert (p["split"], p["shape"], p["paired"], p["ntb"], p["grid_x"], p["grid_z"]) == \
        (1, 0, 1, 36, 144, 3)
    check_cover(p, 4, 3, 69)


def test_split_single_blocks_within_one_round(lib):
    """512 tokens at 8 kv heads (32 x 8 = 256 workgroups) keeps one block per workgroup; one more
    block tips it into pairs."""
    p = plan(lib, 48, 8, 1, 512, 1600)
    assert (p["split"], p["paired"], p["ntb"]) == (1, 0, 32)
    p = plan(lib, 48, 8, 1, 513, 1600)
    assert (p["split"], p["paired"], p["ntb"]) == (1, 1, 17)


def test_configs3_plan(lib):
    """2048 new tokens after 2048 cached, 24/4 heads: paired key-split kernel."""
    p = plan(lib, 24, 4, 1, 2048, 4096)
    assert (p["split"], p["shape"], p["paired"], p["ntb"]) == (1, 0, 1, 64)
    check_cover(p, 4, 1, 128)


@pytest.mark.parametrize("split", range(len(SPLIT_GQA)))
def test_forced_split_shapes(tuned, split):
    """The tuning hook's split indices: 8 + s plans single blocks for the small parity cases,
    13 + s pairs them, the middle block alone when the count is odd."""
    gqa = SPLIT_GQA[split]
    for qlen, q0 in [(161, 45), (200, 0), (250, 7)]:
        n16 = (qlen + 15) // 16
        tuned.fp8kv_prefill_tune(8 + split)
        p = plan(tuned, 4 * gqa, 4, 1, qlen, q0 + qlen)
        assert (p["split"], p["shape"], p["paired"], p["ntb"]) == (1, split, 0, n16 + n16 % 2)
        tuned.fp8kv_prefill_tune(13 + split)
        p = plan(tuned, 4 * gqa, 4, 1, qlen, q0 + qlen)
        assert (p["split"], p["shape"], p["paired"]) == (1, split, 1)
        assert p["ntb"] == ((n16 + 1) // 2 + 1) // 2 * 2
        check_cover(p, 4, 1, n16)


def test_forced_split_shape_other_gqa_uses_per_wave_kernel(tuned):
    """A forced split shape applies only at its own GQA; other GQAs keep the per-wave kernel."""
    tuned.fp8kv_prefill_tune(13)                     # split shape 0 (GQA 6), paired
    p = plan(tuned, 32, 4, 1, 200, 200)              # GQA 8
    assert p["split"] == 0


@pytest.mark.parametrize("hq,hkv,qlen,ctx", [(24, 4, 200, 200), (24, 4, 128, 128),
                                             (4, 4, 300, 5000), (28, 4, 197, 258)])
def test_per_wave_plans(lib, hq, hkv, qlen, ctx):
    """Short contexts and GQAs without a split shape (1, 7) take the per-wave kernel; every block
    is covered."""
    p = plan(lib, hq, hkv, 1, qlen, ctx)
    assert p["split"] == 0
    check_cover(p, hkv, 1, (qlen + 15) // 16)


def test_empty_and_invalid(lib):
    assert plan(lib, 24, 4, 1, 0, 0)["grid_x"] == 0
    out = (ctypes.c_int * 8)()
    assert lib.fp8kv_prefill_plan(24, 5, 1, 10, 10, ctypes.addressof(out)) == 2
    assert lib.fp8kv_prefill_plan(24, 4, 0, 10, 10, ctypes.addressof(out)) == 1
    assert lib.fp8kv_prefill_plan(24, 4, 1, 10, 10, None) == 1
