"""GPU parity of the paged fp8 causal prefill attention against the CPU oracle.

Bar (BASELINE): bf16 output vs the oracle within rtol = atol = 1e-2 elementwise; the reference's
own bar (max-abs < 0.05, vllm-fp8kv/prefill_test.py:49) is also checked on its data regime.
Cases follow vllm-fp8kv/prefill_test.py:95-98 (first chunk, continuation, small tail, scales
0.5 / 2.0) at the BASELINE head geometry (24/4) and at the reference's own (32/8), plus configs[3]
(2048 new tokens over 2048 cached), varlen batches and every GQA the kernel plans for.
"""
import pytest
import torch

from fp8kv_amd import _lib, ops, workloads
from oracle import attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
RTOL = ATOL = 1e-2


def _run_single(c, q0, qlen, ks=None, vs=None, out=None):
    d = workloads.to_device(c, DEV)
    ks = c["k_scale"] if ks is None else ks
    vs = c["v_scale"] if vs is None else vs
    if out is None:
        out = torch.zeros_like(d["q"])
    ops.prefill_attention(d["q"], d["k_cache"], d["v_cache"], out, d["block_table"],
                          torch.tensor([ks], device=DEV), torch.tensor([vs], device=DEV),
                          c["sm_scale"], q0, qlen)
    torch.cuda.synchronize()
    return out.cpu()


def _oracle_single(c, q0, qlen, ks=None, vs=None, dtype=torch.float64):
    ks = c["k_scale"] if ks is None else ks
    vs = c["v_scale"] if vs is None else vs
    return attention.prefill_attention(c["q"], c["k_cache"], c["v_cache"], c["block_table"][0],
                                       ks, vs, c["sm_scale"], q0, qlen, dtype=dtype)


def _check_single(qlen, q0, HQ=24, HKV=4, seed=0, ks=None, vs=None, layout="standalone",
                  kv_gen="amax", PBLK=16, dtype=torch.float64):
    c = workloads.prefill_case([qlen], [q0], HQ=HQ, HKV=HKV, PBLK=PBLK, seed=seed, layout=layout,
                               kv_gen=kv_gen)
    got = _run_single(c, q0, qlen, ks, vs)[:qlen].to(torch.float64)
    ref = _oracle_single(c, q0, qlen, ks, vs, dtype).to(torch.float64)
    torch.testing.assert_close(got, ref, rtol=RTOL, atol=ATOL)
    return (got - ref).abs().max().item(), c


# --- vllm-fp8kv/prefill_test.py:95-98, on the reference's data regime (N(0,1)*2 cast to e4m3) ------

@pytest.mark.parametrize("hq,hkv", [(24, 4), (32, 8)])
@pytest.mark.parametrize("qlen,q0,ks,vs", [
    (2048, 0, 1.0, 1.0),        # first chunk
    (850, 2048, 1.0, 1.0),      # continuation, ctx 2898
    (256, 3840, 1.0, 1.0),      # small tail
    (512, 0, 0.5, 2.0),         # scales
])
def test_reference_cases(hq, hkv, qlen, q0, ks, vs):
    err, _ = _check_single(qlen, q0, HQ=hq, HKV=hkv, seed=qlen + q0, ks=ks, vs=vs, kv_gen="ref",
                           dtype=torch.float32 if qlen * (qlen + q0) > 3_000_000 else torch.float64)
    assert err < 0.05


def test_config3_2048_over_2048_cached():
    """2048 query tokens after 2048 cached ones, 24/4 heads, engine cache layout."""
    err, _ = _check_single(2048, 2048, seed=3, layout="engine", dtype=torch.float32)
    print(f"cfg3 max-abs {err:.2e}")


def test_first_row_is_v0():
    """q0 = 0: query 0 sees key 0 only, so its output is v_scale * V_0 (rounded to bf16)."""
    c = workloads.prefill_case([40], [0], seed=4)
    got = _run_single(c, 0, 40, 1.0, 1.5)
    blk = int(c["block_table"][0, 0])
    for h in range(24):
        v0 = (c["v_cache"][blk, 0, h // 6].to(torch.float64) * 1.5).to(torch.bfloat16)
        assert torch.equal(got[0, h], v0)


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 4), (16, 4), (20, 4), (32, 4), (64, 4), (28, 4)])
def test_gqa_plans(hq, hkv):
    """GQA 1, 2, 4, 5, 8, 16, 7: every (token blocks, row-sets per wave) plan of the kernel."""
    _check_single(197, 61, HQ=hq, HKV=hkv, seed=hq)


@pytest.mark.parametrize("qlen,q0", [(1, 0), (1, 5000), (15, 0), (16, 16), (17, 3), (31, 1),
                                     (33, 32), (64, 0), (100, 31), (129, 4095)])
def test_edge_lengths(qlen, q0):
    _check_single(qlen, q0, seed=qlen * 7 + q0)


def test_block_size_32_engine_layout():
    _check_single(300, 77, PBLK=32, layout="engine", seed=8)


def test_rows_beyond_qlen_untouched_and_deterministic():
    c = workloads.prefill_case([120], [33], seed=9)
    d = workloads.to_device(c, DEV)
    T = d["q"].shape[0]
    big = torch.full((T + 8, 24, 128), 5.0, dtype=torch.bfloat16, device=DEV)
    out = big[:T]
    ks = torch.tensor([c["k_scale"]], device=DEV)
    vs = torch.tensor([c["v_scale"]], device=DEV)
    ops.prefill_attention(d["q"], d["k_cache"], d["v_cache"], out, d["block_table"], ks, vs,
                          c["sm_scale"], 33, 100)                  # only the first 100 rows
    a = big.clone()
    ops.prefill_attention(d["q"], d["k_cache"], d["v_cache"], out, d["block_table"], ks, vs,
                          c["sm_scale"], 33, 100)
    torch.cuda.synchronize()
    assert torch.equal(a, big)
    assert torch.all(big[100:] == 5.0)
    ref = _oracle_single(c, 33, 100)
    torch.testing.assert_close(big[:100].cpu().to(torch.float64), ref, rtol=RTOL, atol=ATOL)


# --- varlen -------------------------------------------------------------------------------------

def _check_varlen(qlens, q0s, seed, HQ=24, HKV=4, layout="standalone", dtype=torch.float64,
                  kv_gen="amax", PBLK=16):
    c = workloads.prefill_case(qlens, q0s, HQ=HQ, HKV=HKV, seed=seed, layout=layout, kv_gen=kv_gen,
                               PBLK=PBLK)
    d = workloads.to_device(c, DEV)
    out = torch.full_like(d["q"], 7.0)
    ops.prefill_attention_varlen(d["q"], d["k_cache"], d["v_cache"], out, d["cu_seqlens_q"],
                                 d["seq_lens"], d["block_table"],
                                 torch.tensor([c["k_scale"]], device=DEV),
                                 torch.tensor([c["v_scale"]], device=DEV), c["sm_scale"])
    torch.cuda.synchronize()
    ref = attention.varlen_prefill_attention(c["q"], c["k_cache"], c["v_cache"], c["cu_seqlens_q"],
                                             c["seq_lens"], c["block_table"], c["k_scale"],
                                             c["v_scale"], c["sm_scale"], dtype=dtype)
    torch.testing.assert_close(out.cpu().to(torch.float64), ref.to(torch.float64), rtol=RTOL, atol=ATOL)


def test_config3_varlen_4x512():
    """configs[3] varlen variant: 4 sequences of 512 new tokens (q0 = 0 each)."""
    _check_varlen([512] * 4, [0] * 4, seed=10, layout="engine")


def test_varlen_mixed_offsets():
    _check_varlen([5, 100, 33, 512, 1], [0, 7, 1000, 3, 250], seed=11)


@pytest.mark.parametrize("shape", [7, 8])
def test_varlen_equals_single_runs(shape):
    """The varlen bookkeeping is exact: with the kernel fixed (per-wave shape 7, key-split shape
    8 + 0 at GQA 6), each sequence of a varlen call is bit-equal to a single-sequence call.  (By
    default the two entry points may pick different kernels: the single call knows its context,
    the varlen host side only max_query_len.)"""
    qlens, q0s = [70, 130, 16], [10, 0, 300]
    c = workloads.prefill_case(qlens, q0s, seed=12)
    d = workloads.to_device(c, DEV)
    ks = torch.tensor([c["k_scale"]], device=DEV)
    vs = torch.tensor([c["v_scale"]], device=DEV)
    lib = _lib.load()
    try:
        lib.fp8kv_prefill_tune(shape)
        out = torch.zeros_like(d["q"])
        ops.prefill_attention_varlen(d["q"], d["k_cache"], d["v_cache"], out, d["cu_seqlens_q"],
                                     d["seq_lens"], d["block_table"], ks, vs, c["sm_scale"])
        cu = c["cu_seqlens_q"].tolist()
        for s in range(3):
            single = torch.zeros_like(d["q"][cu[s]:cu[s + 1]])
            ops.prefill_attention(d["q"][cu[s]:cu[s + 1]], d["k_cache"], d["v_cache"], single,
                                  d["block_table"][s:s + 1], ks, vs, c["sm_scale"], q0s[s], qlens[s])
            torch.cuda.synchronize()
            assert torch.equal(single, out[cu[s]:cu[s + 1]])
    finally:
        lib.fp8kv_prefill_tune(-1)


def test_rejects_bad_arguments():
    c = workloads.prefill_case([16], [0], seed=13)
    d = workloads.to_device(c, DEV)
    out = torch.zeros_like(d["q"])
    lib = _lib.load()
    st = lib.fp8kv_prefill_attn(d["q"].data_ptr(), d["q"].stride(0), d["k_cache"].data_ptr(),
                                d["v_cache"].data_ptr(), *d["k_cache"].stride()[:3],
                                *d["v_cache"].stride()[:3], out.data_ptr(), out.stride(0),
                                d["block_table"].data_ptr(), d["block_table"].stride(0), None, None,
                                0.1, 24, 4, 128, 16, 0, 16, None)
    assert st == 1                                     # null scales
    st = lib.fp8kv_prefill_attn(d["q"].data_ptr(), d["q"].stride(0), d["k_cache"].data_ptr(),
                                d["v_cache"].data_ptr(), *d["k_cache"].stride()[:3],
                                *d["v_cache"].stride()[:3], out.data_ptr(), out.stride(0),
                                d["block_table"].data_ptr(), d["block_table"].stride(0),
                                d["q"].data_ptr(), d["q"].data_ptr(), 0.1, 24, 5, 128, 16, 0, 16, None)
    assert st == 2                                     # HQ % HKV != 0


SHAPE_CAP = [12, 12, 16, 16, 8, 4, 12, 16]      # waves x row-sets of each launch shape
SPLIT_GQA = [6, 12, 4, 8, 16]                   # GQA of each key-split shape (tuning index 8 + s)
SPLIT_PAIRED = 8 + len(SPLIT_GQA)               # tuning index 13 + s: shape s, paired token blocks


@pytest.mark.parametrize("shape", [0, 1, 2, 3, 4, 5, 6, 7])
def test_every_launch_shape(shape):
    """Each (waves, row-sets, ring depth) shape the tuning hook can select meets the same bar,
    single-sequence and varlen, wherever it can hold the GQA."""
    lib = _lib.load()
    try:
        lib.fp8kv_prefill_tune(shape)
        for hq in (4, 8, 24, 64):
            cap = SHAPE_CAP[shape]
            if hq // 4 > cap:
                continue
            _check_single(161, 45, HQ=hq, HKV=4, seed=shape * 100 + hq)
            _check_single(200, 0, HQ=hq, HKV=4, seed=shape * 100 + hq + 1)     # odd block count
        cap = SHAPE_CAP[shape]
        _check_varlen([40, 97], [3, 200], seed=shape + 50, HQ=4 * min(6, cap), HKV=4)
    finally:
        lib.fp8kv_prefill_tune(-1)


@pytest.mark.parametrize("PBLK", [64, 128])
def test_large_cache_blocks(PBLK):
    """Cache blocks larger than a 32-key tile: the copies' in-block slot offset is then a different
    multiple of 32 for each tile of a block (key-split kernel at GQA 6 and 4, per-wave kernel
    below 1024 keys)."""
    _check_single(700, 600, HQ=24, HKV=4, seed=PBLK, PBLK=PBLK, layout="engine")
    _check_single(1100, 300, HQ=16, HKV=4, seed=PBLK + 1, PBLK=PBLK, layout="engine")
    _check_single(300, 77, HQ=24, HKV=4, seed=PBLK + 2, PBLK=PBLK, layout="engine")


@pytest.mark.parametrize("paired", [False, True])
@pytest.mark.parametrize("split", range(len(SPLIT_GQA)))
def test_every_split_shape(split, paired):
    """Each key-split shape (row-sets per wave x head groups, keys split over the rest of the 8
    waves) at its GQA: a tail block, varlen, block size 32, and odd (11, 13, 33; varlen 3, 7, 19)
    and even (16) token-block counts.  These grids fit one round of 256 workgroups, so the
    default plan gives every workgroup one 16-token block; ``paired`` forces the two-phase plan
    (blocks r and n16 - 1 - r in one workgroup, the middle block alone when n16 is odd) that
    larger grids take."""
    lib = _lib.load()
    gqa = SPLIT_GQA[split]
    try:
        lib.fp8kv_prefill_tune((SPLIT_PAIRED if paired else 8) + split)
        _check_single(161, 45, HQ=4 * gqa, HKV=4, seed=split * 10)
        _check_single(200, 0, HQ=4 * gqa, HKV=4, seed=split * 10 + 1)
        _check_single(250, 7, HQ=4 * gqa, HKV=4, seed=split * 10 + 3)
        _check_single(513, 1000, HQ=2 * gqa, HKV=2, seed=split * 10 + 2, PBLK=32, layout="engine")
        _check_varlen([40, 97, 300], [3, 200, 0], seed=split + 60, HQ=4 * gqa, HKV=4)
    finally:
        lib.fp8kv_prefill_tune(-1)


def _plan(lib, hq, hkv, num_seqs, max_query_len, ctx_hint):
    import ctypes
    out = (ctypes.c_int * 8)()
    assert lib.fp8kv_prefill_plan(hq, hkv, num_seqs, max_query_len, ctx_hint, ctypes.addressof(out)) == 0
    return dict(zip(("split", "shape", "nb", "paired", "ntb", "grid_x", "grid_z", "threads"), list(out)))


@pytest.mark.parametrize("case", ["configs3_paired", "1k_over_1k_single", "forced_paired_gqa6",
                                  "forced_paired_gqa4", "varlen_paired"])
def test_split_kernel_repeats_bitwise(case):
    """The key-split kernel is deterministic: its partial states merge in LDS in a fixed order and
    every copy is waited for by count, so repeated calls on the same inputs give the same bits.
    Ten calls each on the configs[3] plan (256 workgroups of two paired token blocks), the
    single-block plan (1024 over 1024), the paired plan forced onto a smaller grid at GQA 6 and
    4, and the paired varlen plan; the first call is also checked against the oracle."""
    lib = _lib.load()
    tune = -1
    if case == "configs3_paired":
        qlens, q0s, hq, layout = [2048], [2048], 24, "engine"
    elif case == "1k_over_1k_single":
        qlens, q0s, hq, layout = [1024], [1024], 24, "engine"
    elif case == "forced_paired_gqa6":
        qlens, q0s, hq, layout, tune = [600], [700], 24, "standalone", SPLIT_PAIRED + 0
    elif case == "forced_paired_gqa4":
        qlens, q0s, hq, layout, tune = [600], [700], 16, "standalone", SPLIT_PAIRED + 2
    else:
        qlens, q0s, hq, layout = [1100, 1030, 300], [0, 40, 900], 24, "engine"
    c = workloads.prefill_case(qlens, q0s, HQ=hq, HKV=4, seed=len(case) + 400, layout=layout)
    d = workloads.to_device(c, DEV)
    ks = torch.tensor([c["k_scale"]], device=DEV)
    vs = torch.tensor([c["v_scale"]], device=DEV)
    varlen = len(qlens) > 1
    try:
        lib.fp8kv_prefill_tune(tune)
        if varlen:
            p = _plan(lib, hq, 4, len(qlens), max(qlens), max(qlens))
        else:
            p = _plan(lib, hq, 4, 1, qlens[0], q0s[0] + qlens[0])
        assert p["split"] == 1, p                       # the key-split kernel serves every case
        assert p["paired"] == (case != "1k_over_1k_single"), p
        outs = []
        for _ in range(10):
            out = torch.zeros_like(d["q"])
            if varlen:
                ops.prefill_attention_varlen(d["q"], d["k_cache"], d["v_cache"], out, d["cu_seqlens_q"],
                                             d["seq_lens"], d["block_table"], ks, vs, c["sm_scale"])
            else:
                ops.prefill_attention(d["q"], d["k_cache"], d["v_cache"], out, d["block_table"], ks, vs,
                                      c["sm_scale"], q0s[0], qlens[0])
            outs.append(out)
        torch.cuda.synchronize()
    finally:
        lib.fp8kv_prefill_tune(-1)
    for i, o in enumerate(outs[1:], 1):
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16)), f"call {i} differs"
    if varlen:
        ref = attention.varlen_prefill_attention(c["q"], c["k_cache"], c["v_cache"], c["cu_seqlens_q"],
                                                 c["seq_lens"], c["block_table"], c["k_scale"],
                                                 c["v_scale"], c["sm_scale"], dtype=torch.float32)
        got = outs[0].cpu()
    else:
        ref = _oracle_single(c, q0s[0], qlens[0], dtype=torch.float32)
        got = outs[0].cpu()[:qlens[0]]
    torch.testing.assert_close(got.to(torch.float64), ref.to(torch.float64), rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("gqa", SPLIT_GQA)
def test_split_paired_default_plan(gqa):
    """Grids above one round of 256 workgroups take paired token blocks on the default plan:
    600 new tokens after 1000 cached at 8 kv heads (38 blocks x 8 heads = 304 workgroups)."""
    _check_single(600, 1000, HQ=8 * gqa, HKV=8, seed=gqa + 70, layout="engine")


def test_split_paired_varlen_default_plan():
    """Varlen on the paired plan: 69, 65 and 19 token blocks (odd), 4 kv heads, GQA 6."""
    _check_varlen([1100, 1030, 300], [0, 40, 900], seed=81, HQ=24, HKV=4, layout="engine")


@pytest.mark.parametrize("layout", ["standalone", "engine"])
def test_cascade_shared_prefix_batch(layout):
    """A cascade batch as vLLM describes it (the hook sends it to the varlen kernel): three
    requests share the first 40 cache blocks (640 tokens) of their block tables, each with its own
    suffix and new tokens; the varlen kernel over the full tables equals the oracle."""
    c = workloads.prefill_case([300, 130, 257], [500, 700, 900], seed=33, layout=layout)
    bt = c["block_table"]
    bt[1:, :40] = bt[0, :40]                      # the shared prefix: same blocks, same K/V bytes
    c["block_table"] = bt
    d = workloads.to_device(c, DEV)
    out = torch.full_like(d["q"], 7.0)
    ops.prefill_attention_varlen(d["q"], d["k_cache"], d["v_cache"], out, d["cu_seqlens_q"], d["seq_lens"],
                                 d["block_table"], torch.tensor([c["k_scale"]], device=DEV),
                                 torch.tensor([c["v_scale"]], device=DEV), c["sm_scale"])
    torch.cuda.synchronize()
    ref = attention.varlen_prefill_attention(c["q"], c["k_cache"], c["v_cache"], c["cu_seqlens_q"],
                                             c["seq_lens"], c["block_table"], c["k_scale"], c["v_scale"],
                                             c["sm_scale"])
    torch.testing.assert_close(out.cpu().to(torch.float64), ref.to(torch.float64), rtol=RTOL, atol=ATOL)


# ---- bf16 caches (the reference's K_FP8 = False branch, vllm-fp8kv/fp8kv_prefill.py:57-60,77-82,
# 117,143): fp8kv_prefill_attn_bf16 / _varlen_bf16, values used as stored, scales ignored.

@pytest.mark.parametrize("hq,hkv", [(24, 4), (32, 8)])
@pytest.mark.parametrize("qlen,q0", [(2048, 0), (850, 2048), (256, 3840), (512, 0)])
def test_bf16_kv_reference_cases(hq, hkv, qlen, q0):
    """The reference's four prefill cases (prefill_test.py:95-98) over bf16 caches; the scales
    passed (0.5, 2.0) must play no part."""
    c = workloads.prefill_case([qlen], [q0], HQ=hq, HKV=hkv, seed=qlen + q0 + 5, kv_gen="bf16")
    got = _run_single(c, q0, qlen, ks=0.5, vs=2.0)[:qlen].to(torch.float64)
    ref = _oracle_single(c, q0, qlen, 1.0, 1.0).to(torch.float64)
    torch.testing.assert_close(got, ref, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("gqa", [1, 2, 3, 4, 6, 7, 8, 12, 16])
def test_bf16_kv_every_gqa(gqa):
    """Up to 8 query heads per workgroup, two head groups above 8; a tail block and odd lengths."""
    _check_single(161, 45, HQ=4 * gqa, HKV=4, seed=gqa + 90, kv_gen="bf16")
    _check_single(33, 0, HQ=2 * gqa, HKV=2, seed=gqa + 91, kv_gen="bf16", layout="engine")


@pytest.mark.parametrize("gqa", [3, 6, 16])
def test_bf16_kv_one_head_per_wave(gqa):
    """The one-head-per-wave kernel (the MHA default) forced at GQA > 1."""
    lib = _lib.load()
    try:
        lib.fp8kv_prefill_bf16_tune(1)
        _check_single(161, 45, HQ=4 * gqa, HKV=4, seed=gqa + 97, kv_gen="bf16")
    finally:
        lib.fp8kv_prefill_bf16_tune(0)


@pytest.mark.parametrize("qlen,q0", [(1, 0), (1, 700), (16, 0), (17, 15), (300, 1)])
def test_bf16_kv_edge_lengths(qlen, q0):
    _check_single(qlen, q0, seed=qlen * 7 + q0, kv_gen="bf16")


@pytest.mark.parametrize("PBLK", [32, 64, 128])
def test_bf16_kv_block_sizes(PBLK):
    _check_single(700, 600, seed=PBLK + 3, PBLK=PBLK, layout="engine", kv_gen="bf16")


def test_bf16_kv_varlen():
    _check_varlen([5, 100, 33, 512, 1], [0, 7, 1000, 3, 250], seed=93, kv_gen="bf16")
    _check_varlen([512] * 4, [0] * 4, seed=94, layout="engine", kv_gen="bf16", PBLK=32)


def test_bf16_kv_config3_full_size():
    """configs[3] over bf16 caches: 2048 new tokens after 2048 cached, 24/4 heads."""
    _check_single(2048, 2048, seed=95, layout="engine", kv_gen="bf16")


def test_bf16_kv_through_the_reference_run():
    """fp8kv_prefill.run (the reference's signature) takes bf16 caches as the reference does."""
    import fp8kv_prefill
    c = workloads.prefill_case([200], [100], seed=96, kv_gen="bf16")
    d = workloads.to_device(c, DEV)
    out = torch.full_like(d["q"], 7.0)
    fp8kv_prefill.run(d["q"], d["k_cache"], d["v_cache"], out, d["block_table"], 0.3, 5.0,
                      c["sm_scale"], 100, 200)
    torch.cuda.synchronize()
    ref = _oracle_single(c, 100, 200).to(torch.float64)
    torch.testing.assert_close(out.cpu().to(torch.float64), ref, rtol=RTOL, atol=ATOL)
