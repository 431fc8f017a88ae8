"""The build's scratch guard (fp8kv_amd/build.py): no kernel of the library may use scratch memory.

The LDS-ring kernels (matvec, decode chunk loads, prefill rings) wait for their own asynchronous
copies with hand-counted ``s_waitcnt vmcnt(N)``.  A register spill adds scratch loads and stores on
the same counter, so the build fails when hipcc's resource remarks report any scratch, VGPR spill
or dynamic stack.  CPU only: hipcc cross-compiles for gfx950 without a GPU.
"""
import os
import shutil
import subprocess

import pytest

from fp8kv_amd import build

HIPCC = None
try:
    HIPCC = build.hipcc()
except FileNotFoundError:
    pass

needs_hipcc = pytest.mark.skipif(HIPCC is None, reason="hipcc not installed")

REMARKS = """\
k.hip:3:1: remark: Function Name: _Z4goodPf [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark:     TotalSGPRs: 22 [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark:     VGPRs: 10 [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark:     Dynamic Stack: False [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark:     SGPRs Spill: 12 [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
k.hip:9:1: remark: Function Name: _Z5spillPf [-Rpass-analysis=kernel-resource-usage]
k.hip:9:1: remark:     ScratchSize [bytes/lane]: 88 [-Rpass-analysis=kernel-resource-usage]
k.hip:9:1: remark:     Dynamic Stack: False [-Rpass-analysis=kernel-resource-usage]
k.hip:9:1: remark:     VGPRs Spill: 22 [-Rpass-analysis=kernel-resource-usage]
"""


def test_parse_and_flag_spills():
    recs = build.parse_resource_usage(REMARKS)
    assert [r["name"] for r in recs] == ["_Z4goodPf", "_Z5spillPf"]
    assert recs[0]["ScratchSize [bytes/lane]"] == "0" and recs[0]["SGPRs Spill"] == "12"
    bad = build.resource_violations(recs)
    # SGPR spills live in VGPR lanes and are allowed; the scratch user is flagged
    assert len(bad) == 1 and bad[0].startswith("_Z5spillPf") and "88" in bad[0]


def test_dynamic_stack_is_flagged():
    recs = [{"name": "k", "ScratchSize [bytes/lane]": "0", "VGPRs Spill": "0", "Dynamic Stack": "True"}]
    assert build.resource_violations(recs)


@needs_hipcc
def test_guard_catches_a_kernel_with_scratch(tmp_path):
    """A dynamically indexed private array lives in scratch: the remarks must show it and the
    guard must reject it."""
    src = tmp_path / "probe.hip"
    src.write_text(
        "#include <hip/hip_runtime.h>\n"
        "__global__ void __launch_bounds__(256) probe(float* p, int i) {\n"
        "  float a[64];\n"
        "  for (int j = 0; j < 64; ++j) a[j] = p[j * 256 + threadIdx.x];\n"
        "  p[threadIdx.x] = a[(i + threadIdx.x) & 63];\n"
        "}\n")
    res = subprocess.run([HIPCC, *build.HIPCC_FLAGS, build.RESOURCE_FLAG, "-c", str(src), "-o",
                          str(tmp_path / "probe.o")], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    recs = build.parse_resource_usage(res.stderr)
    assert [r["name"] for r in recs] == ["_Z5probePfi"]
    assert build.resource_violations(recs)


@needs_hipcc
def test_library_kernels_use_no_scratch(tmp_path):
    """The whole library, built with the guard: build() raises if any kernel spills."""
    out = tmp_path / "libfp8kv_amd.so"
    assert build.build(out=str(out), measure_out=str(tmp_path / "libfp8kv_measure.so")) == str(out)
    assert out.exists() and out.stat().st_size > 0
