"""C-ABI checks that need no GPU: the library loads, exports what include/*.h declares, and rejects
bad arguments before launching anything."""
import ctypes
import glob
import os
import re
import subprocess

import pytest

from conftest import REPO


def _declared_functions():
    names = []
    for hdr in glob.glob(os.path.join(REPO, "include", "*.h")):
        text = open(hdr).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b([A-Za-z_]\w*)\s*\([^;{]*\)\s*;", text, re.M):
            names.append(m.group(1))
    return names


def test_header_declares_reference_symbol():
    names = _declared_functions()
    assert "h4mv_launch" in names and "h4mv_launch_status" in names


def test_library_exports_every_declared_symbol(lib):
    from fp8kv_amd import _lib
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.lib_path()], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for name in _declared_functions():
        assert name in exported, name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
        getattr(lib, name)


def test_status_strings(lib):
    assert lib.fp8kv_status_string(0) == b"ok"
    assert lib.fp8kv_status_string(5).startswith(b"scratch")
    assert lib.fp8kv_status_string(99) == b"unknown status"


# Pointer values below are never dereferenced: every call is rejected before any launch.
A = 0x10000


@pytest.mark.parametrize("args,code", [
    ((0, A, A, A, 64, 64, 1), 1),          # null W
    ((A, A, A, A, 0, 64, 1), 1),           # N = 0
    ((A, A, A, A, 64, 64, 0), 1),          # M = 0
    ((A, A, A, A, 64, 64, 17), 2),         # M > 16
    ((A, A, A, A, 64, 48, 1), 2),          # K % 32 != 0
    ((A + 1, A, A, A, 64, 64, 1), 3),      # W not 16-byte aligned
    ((A, A, A + 8, A, 64, 64, 1), 3),      # X not 16-byte aligned
])
def test_h4mv_rejects_before_launch(lib, args, code):
    assert lib.h4mv_launch_status(*args, None) == code
    lib.h4mv_launch(*args, None)
    assert lib.fp8kv_last_status() == code


def test_loader_fails_loudly_without_library(monkeypatch, tmp_path):
    from fp8kv_amd import _lib
    monkeypatch.setenv("FP8KV_AMD_LIB", str(tmp_path / "missing.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(FileNotFoundError):
        _lib.load()


def _decode_args(**kw):
    a = dict(q=A, qs=24 * 128, k=A, v=A, sk0=16 * 4 * 128, sk1=4 * 128, sk2=128, sv0=16 * 4 * 128,
             sv1=4 * 128, sv2=128, out=A, os=24 * 128, qsl=A, sl=A, bt=A, bts=64, ks=A, vs=A,
             sm=0.088, ns=8, hq=24, hkv=4, hd=128, pblk=16, nsplit=1, scr=None, scrb=0, stream=None)
    a.update(kw)
    return list(a.values())


@pytest.mark.parametrize("kw,code", [
    (dict(q=0), 1), (dict(ns=0), 1), (dict(nsplit=0), 1), (dict(nsplit=257), 1),
    (dict(hd=64), 2), (dict(hq=25), 2), (dict(hq=68, hkv=4), 2), (dict(pblk=8), 2), (dict(pblk=48), 2),
    (dict(k=A + 8), 3), (dict(sk1=4 * 128 + 8), 3), (dict(sv2=4), 3), (dict(qs=24 * 128 + 4), 3),
    (dict(nsplit=8), 5), (dict(nsplit=8, scr=A, scrb=100), 5),
])
def test_decode_rejects_before_launch(lib, kw, code):
    assert lib.fp8kv_decode_attn(*_decode_args(**kw)) == code


@pytest.mark.parametrize("kw,code", [
    (dict(q=0), 1), (dict(hd=64), 2), (dict(hq=25), 2), (dict(pblk=8), 2),
    (dict(k=A + 8), 3), (dict(v=A + 8), 3),                  # bf16 V rows are 16-byte loads
    (dict(sk1=4 * 128 + 4), 3), (dict(sv2=4), 3),            # strides in elements, multiples of 8
    (dict(sk1=1 << 26), 2),                                  # slot stride above 2^25 elements
    (dict(ks=None, vs=None, nsplit=8), 5),                   # no scales needed: reaches the scratch check
])
def test_decode_bf16_rejects_before_launch(lib, kw, code):
    assert lib.fp8kv_decode_attn_bf16(*_decode_args(**kw)) == code


def test_decode_e4m3_needs_scales(lib):
    assert lib.fp8kv_decode_attn(*_decode_args(ks=None)) == 1


def test_decode_scratch_sizing(lib):
    assert lib.fp8kv_decode_scratch_bytes(8, 24, 4, 128, 1) == 0
    b = lib.fp8kv_decode_scratch_bytes(8, 24, 4, 128, 8)
    assert b == 65536 * 4 + 8 * 4 * 8 * 6 * 130 * 4
    assert lib.fp8kv_decode_scratch_bytes(8, 24, 4, 64, 8) == 0


def test_decode_split_planner(lib):
    assert lib.fp8kv_decode_num_splits(8, 4, 4096) == 8       # b8@4k: one workgroup per CU
    assert lib.fp8kv_decode_num_splits(8, 4, 0) == 1
    for ns, hkv, ctx in [(1, 1, 100000), (64, 8, 8192), (1, 4, 17), (300, 8, 4096)]:
        n = lib.fp8kv_decode_num_splits(ns, hkv, ctx)
        assert 1 <= n <= 256


# fp8kv_cache_write: every call below is rejected before any HIP call (fake pointers).
CW_OK = [A, 512, A, 512, A, A, 8192, 512, 128, 8192, 512, 128, A, A, A, 4, 4, 128, 16, None]


@pytest.mark.parametrize("idx,val,code", [
    (17, 120, 2),              # head_size % 16 != 0
    (18, 24, 2),               # block size not a power of two
    (6, 8200, 3),              # K block stride not a multiple of 16
    (9, 8196, 3),              # V block stride not a multiple of 8
    (0, A + 8, 3),             # key not 16-byte aligned
    (1, 100, 3),               # key row stride not a multiple of 8
    (1, 256, 1),               # key row stride shorter than a token row
    (12, None, 1),             # no slot mapping
    (15, -1, 1),               # negative token count
    (16, 0, 1),                # no kv heads
])
def test_cache_write_rejects_before_launch(lib, idx, val, code):
    args = list(CW_OK)
    args[idx] = val
    assert lib.fp8kv_cache_write(*args) == code


def test_cache_write_zero_tokens_is_a_no_op(lib):
    args = list(CW_OK)
    args[15] = 0
    assert lib.fp8kv_cache_write(*args) == 0


# fp8kv_prefill_attn on the engine layout [NB, HKV, PBLK, 2D]: qlen = 0 returns before any launch.
PF_OK = [A, 24 * 128, A, A + 128, 16384, 256, 4096, 16384, 256, 4096, A, 24 * 128, A, 64, A, A,
         0.088, 24, 4, 128, 16, 0, 0, None]


@pytest.mark.parametrize("changes,code", [
    ({0: None}, 1), ({12: None}, 1), ({18: 0}, 1), ({21: -1}, 1), ({22: -1}, 1),
    ({19: 64}, 2), ({17: 25}, 2), ({17: 68}, 2), ({20: 8}, 2), ({20: 48}, 2),
    ({2: A + 8}, 3), ({3: A + 4}, 3), ({5: 264}, 3), ({8: 260}, 3), ({1: 24 * 128 + 4}, 3),
    ({5: -256}, 2),                                  # negative slot stride
    ({5: 1 << 28, 20: 32}, 2),                       # in-block offsets beyond 32 bits
    ({8: 1 << 28, 20: 32}, 2),
])
def test_prefill_rejects_before_launch(lib, changes, code):
    args = list(PF_OK)
    for k, v in changes.items():
        args[k] = v
    assert lib.fp8kv_prefill_attn(*args) == code


# fp8kv_prefill_attn_varlen, same cache geometry: max_query_len = 0 returns before any launch.
PFV_OK = [A, 24 * 128, A, A + 128, 16384, 256, 4096, 16384, 256, 4096, A, 24 * 128, A, A, A, 64, A,
          A, 0.088, 2, 24, 4, 128, 16, 0, None]


@pytest.mark.parametrize("changes,code", [
    ({12: None}, 1), ({13: None}, 1), ({19: 0}, 1), ({24: -1}, 1), ({19: 65536}, 2),
    ({5: -256}, 2), ({5: 1 << 28, 23: 32}, 2), ({8: 1 << 28, 23: 32}, 2), ({2: A + 8}, 3),
])
def test_prefill_varlen_rejects_before_launch(lib, changes, code):
    args = list(PFV_OK)
    for k, v in changes.items():
        args[k] = v
    assert lib.fp8kv_prefill_attn_varlen(*args) == code


def test_prefill_varlen_zero_query_is_a_no_op(lib):
    assert lib.fp8kv_prefill_attn_varlen(*PFV_OK) == 0


# The bf16 entry points on the engine layout [NB, HKV, PBLK, 2D] of bf16 (strides in elements, the V
# view 128 elements = 256 bytes in); qlen = 0 / max_query_len = 0 return before any launch.
PFB_OK = [A, 24 * 128, A, A + 256, 16384, 256, 4096, 16384, 256, 4096, A, 24 * 128, A, 64, None, None,
          0.088, 24, 4, 128, 16, 0, 0, None]


@pytest.mark.parametrize("changes,code", [
    ({0: None}, 1), ({12: None}, 1), ({21: -1}, 1), ({19: 64}, 2), ({17: 25}, 2), ({20: 8}, 2),
    ({2: A + 8}, 3), ({3: A + 8}, 3), ({5: 260}, 3), ({8: 260}, 3), ({1: 24 * 128 + 4}, 3),
    ({5: 1 << 26}, 2), ({5: -256}, 2),
])
def test_prefill_bf16_rejects_before_launch(lib, changes, code):
    args = list(PFB_OK)
    for k, v in changes.items():
        args[k] = v
    assert lib.fp8kv_prefill_attn_bf16(*args) == code


def test_prefill_bf16_takes_no_scales(lib):
    assert lib.fp8kv_prefill_attn_bf16(*PFB_OK) == 0


def test_prefill_varlen_bf16_rejects_before_launch(lib):
    base = PFB_OK[:12] + [A, A] + PFB_OK[12:14] + [None, None, 0.088, 2, 24, 4, 128, 16, 0, None]
    assert lib.fp8kv_prefill_attn_varlen_bf16(*base) == 0
    for idx, val, code in [(12, None, 1), (19, 0, 1), (24, -1, 1), (19, 65536, 2), (3, A + 8, 3)]:
        args = list(base)
        args[idx] = val
        assert lib.fp8kv_prefill_attn_varlen_bf16(*args) == code, (idx, val)


def test_prefill_accepts_largest_32_bit_block_offsets(lib):
    args = list(PF_OK)
    args[5] = args[8] = 1 << 27                      # 15 * 2^27 + 128 < 2^32 at block size 16
    assert lib.fp8kv_prefill_attn(*args) == 0


@pytest.mark.parametrize("args,code", [
    ((0, A, 64, 64, None), 1),            # null input
    ((A, A, 0, 64, None), 1),             # N = 0
    ((A, A, 64, 48, None), 2),            # K % 32 != 0
])
def test_repack_scales_rejects_before_launch(lib, args, code):
    assert lib.h4mv_repack_scales(*args) == code


# Layer epilogues: every call below is rejected (or is a no-op) before any HIP call.
RN_OK = [A, 4096, A, 4096, A, A, 4096, 8, 4096, 1e-6, 0, None]


@pytest.mark.parametrize("idx,val,code", [
    (0, None, 1),              # no x
    (8, 4100, 2),              # hidden size not a multiple of 8
    (8, 16392, 2),             # hidden size above 16384
    (10, 2, 1),                # unknown mode
    (9, -1.0, 1),              # negative eps
    (1, 100, 1),               # row stride shorter than a row
    (1, 4100, 3),              # row stride not a multiple of 8
    (4, A + 8, 3),             # weight not 16-byte aligned
])
def test_rmsnorm_rejects_before_launch(lib, idx, val, code):
    args = list(RN_OK)
    args[idx] = val
    assert lib.fp8kv_fused_add_rmsnorm(*args) == code


def test_rmsnorm_zero_tokens_is_a_no_op(lib):
    args = list(RN_OK)
    args[7] = 0
    assert lib.fp8kv_fused_add_rmsnorm(*args) == 0


@pytest.mark.parametrize("args,code", [
    ((None, 64, A, 32, 4, 32, 0, None), 1),       # null input
    ((A, 64, A, 32, 4, 36, 0, None), 2),         # d % 8 != 0
    ((A, 48, A, 32, 4, 32, 0, None), 1),         # input row shorter than 2 d
    ((A, 64, A, 32, 4, 32, 3, None), 1),         # unknown mode
    ((A + 2, 64, A, 32, 4, 32, 0, None), 3),     # misaligned input
])
def test_silu_mul_rejects_before_launch(lib, args, code):
    assert lib.fp8kv_silu_mul(*args) == code


@pytest.mark.parametrize("args,code", [
    ((A, A, A, A, 8, 1024, 1, 0, None), 1),      # N < 16
    ((A, A, A, A, 64, 1024, 9, 0, None), 2),     # M > 8
    ((A, A, A, A, 64, 1000, 1, 0, None), 2),     # K % 512 != 0
    ((A, A, A, A, 72, 1024, 1, 0, None), 2),     # N % 16 != 0
    ((A, A, A, A + 4, 64, 1024, 1, 0, None), 3), # out not 8-byte aligned
    ((A, A, A, A, 64, 1024, 1, 5, None), 1),     # unknown mode
])
def test_h4mv_silu_mul_rejects_before_launch(lib, args, code):
    assert lib.h4mv_silu_mul(*args) == code


@pytest.mark.parametrize("args,code", [
    ((A, A, A, A, 72, 1024, None), 2),           # N % 16 != 0
    ((A, A, A, None, 64, 1024, None), 1),        # no scale output
    ((A + 8, A, A, A, 64, 1024, None), 3),       # misaligned codes
])
def test_interleave_rejects_before_launch(lib, args, code):
    assert lib.h4mv_interleave_gate_up(*args) == code


@pytest.mark.parametrize("args,code", [
    ((A, 64, A, A, 4, 48, None), 2),              # K % 32 != 0
    ((A, 16, A, A, 4, 64, None), 1),              # row stride shorter than K
    ((A + 8, 64, A, A, 4, 64, None), 3),          # X not 16-byte aligned
    ((None, 64, A, A, 4, 64, None), 1),           # no X
])
def test_quant_act_rejects_before_launch(lib, args, code):
    assert lib.h4a8_quant_act(*args) == code


@pytest.mark.parametrize("args,code", [
    ((A, A, A, A, A, 64, 192, 16, None), 2),      # K % 128 != 0
    ((A, A, A, A, A, 66, 256, 16, None), 2),      # N % 4 != 0
    ((A, A, A, A, A + 2, 64, 256, 16, None), 3),  # out misaligned
    ((A, A, None, A, A, 64, 256, 16, None), 1),   # no activations
])
def test_h4a8_gemm_rejects_before_launch(lib, args, code):
    assert lib.h4a8_gemm(*args) == code


def test_h4a8_zero_rows_are_a_no_op(lib):
    assert lib.h4a8_gemm(A, A, A, A, A, 64, 256, 0, None) == 0
    assert lib.h4a8_quant_act(A, 64, A, A, 0, 64, None) == 0
