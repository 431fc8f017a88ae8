"""Build libfp8kv_amd.so (all HIP kernels + the C ABI) for gfx950 with hipcc, in-tree.

Usage: ``python -m fp8kv_amd.build`` (with gfx1201-tuning-log_amd/ on sys.path) or
``fp8kv_amd.build.build()``.  The library lands next to the package directory, which is where
``fp8kv_amd._lib`` looks for it (override with FP8KV_AMD_LIB).
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
import tempfile

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))   # gfx1201-tuning-log_amd/
REPO_ROOT = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
INCLUDE = os.path.join(REPO_ROOT, "include")
LIB_NAME = "libfp8kv_amd.so"
LIB_PATH = os.path.join(PKG_ROOT, LIB_NAME)

SOURCES = ["h4mv.hip", "h4mv_repack.hip", "decode_attn.hip", "prefill_attn.hip", "prefill_bf16kv.hip",
           "cache_write.hip", "epilogues.hip", "w4a8_gemm.hip", "lm_head.hip"]
# The benchmark's read-only reference launch (fp8kv_stream_read) is a measurement aid, not part of
# the path: it is built into a library of its own that only bench.py loads.
MEASURE_LIB_NAME = "libfp8kv_measure.so"
MEASURE_LIB_PATH = os.path.join(PKG_ROOT, MEASURE_LIB_NAME)
MEASURE_SOURCES = ["stream_read.hip"]

# Packed-fp32 VALU forms are disabled for every HIP file built here (the compiler would otherwise
# emit v_pk_{add,mul,fma}_f32 from ordinary float code).
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]

# Per-file code-generation options.  The block-scaled MFMA accumulates in place only in its VGPR
# form; left to choose, the compiler keeps the GEMM accumulators in VGPRs and copies them into
# AGPRs around every MFMA.  The GEMM is also scheduled with the iterative ILP strategy (measured
# at the configs[4] linears, M = 2048: gate/up 298-299 -> 274-275 us on MXFP8 activations and
# 283-284 -> 264 us per-token, the four linears together -4%; the attention and matvec kernels
# were slower or unchanged with it).  Kernel-argument preloading (gfx950: the first 16 SGPRs of the leading
# scalar arguments are loaded before the wave starts) removes one dependent round trip from the
# start of the matvec and decode kernels (measured: matvec cfg1 M = 1 11.35 -> 11.12 us, M = 8
# 12.85 -> 12.40 us).  Arguments passed as a struct are not preloaded.
FILE_FLAGS = {
    "w4a8_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-amdgpu-sched-strategy=iterative-ilp"],
    "h4mv.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
    "decode_attn.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
    "prefill_bf16kv.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
    # the read-only reference launch is preloaded like the kernels it is compared with: the
    # dispatch-stamped events leave the preload out of the kernel's window
    "stream_read.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise FileNotFoundError("hipcc not found (set HIPCC)")


# Every device compile reports each kernel's resources (registers, scratch, LDS) as remarks.
RESOURCE_FLAG = "-Rpass-analysis=kernel-resource-usage"
_REMARK = re.compile(r"remark:\s+(Function Name|[A-Za-z][A-Za-z ]*?(?: \[[^\]]*\])?):\s*(\S+)\s+\[-Rpass-analysis")


def parse_resource_usage(text: str) -> list[dict]:
    """Kernel records from hipcc's ``-Rpass-analysis=kernel-resource-usage`` remarks: one dict per
    kernel with its mangled name under "name" and every reported field (``ScratchSize [bytes/lane]``,
    ``VGPRs Spill``, ``Dynamic Stack``, ...) as a string."""
    recs: list[dict] = []
    for key, val in _REMARK.findall(text):
        if key == "Function Name":
            recs.append({"name": val})
        elif recs:
            recs[-1][key.strip()] = val
    return recs


def resource_violations(recs: list[dict]) -> list[str]:
    """Kernels that touch private (scratch) memory.  The LDS-ring kernels wait for their own
    asynchronous copies with hand-counted ``s_waitcnt vmcnt(N)``, and a scratch spill or reload is
    one more vector-memory operation on the same counter, so no kernel in the library may spill
    VGPRs, need scratch or a dynamic stack.  (SGPR spills go to VGPR lanes, not to memory; an SGPR
    spill that did reach memory shows up as scratch.)"""
    bad = []
    for r in recs:
        scratch = int(r.get("ScratchSize [bytes/lane]", "0"))
        vspill = int(r.get("VGPRs Spill", "0"))
        dyn = r.get("Dynamic Stack", "False") != "False"
        if scratch or vspill or dyn:
            bad.append(f"{r['name']}: scratch {scratch} B/lane, {vspill} VGPRs spilled, dynamic stack {dyn}")
    return bad


def _run(cmd: list[str], verbose: bool) -> str:
    if verbose:
        print(" ".join(cmd), file=sys.stderr)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-6000:]}")
    return res.stderr


def build(out: str = LIB_PATH, verbose: bool = False, jobs: int | None = None,
          measure_out: str | None = MEASURE_LIB_PATH) -> str:
    """Compile every source in SOURCES (one object each, in parallel) and link them into one
    shared library; atomic replace of ``out``.  Fails, leaving ``out`` untouched, when any kernel
    uses scratch memory (``resource_violations``).  Also builds the benchmark's measurement
    library at ``measure_out`` (None: skipped)."""
    path = _build_lib(SOURCES, out, verbose, jobs)
    if measure_out is not None:
        _build_lib(MEASURE_SOURCES, measure_out, verbose, jobs)
    return path


def _build_lib(sources: list[str], out: str, verbose: bool, jobs: int | None) -> str:
    from concurrent.futures import ThreadPoolExecutor
    cc = hipcc()
    with tempfile.TemporaryDirectory(prefix=".fp8kv_amd_build_", dir=os.path.dirname(out)) as tmpdir:
        objs = []
        cmds = []
        for src in sources:
            obj = os.path.join(tmpdir, os.path.splitext(src)[0] + ".o")
            objs.append(obj)
            cmds.append([cc, *HIPCC_FLAGS, *FILE_FLAGS.get(src, []), RESOURCE_FLAG, f"-I{INCLUDE}",
                         f"-I{CSRC}", "-c", os.path.join(CSRC, src), "-o", obj])
        workers = jobs or min(len(cmds), max(1, min(8, os.cpu_count() or 1)))
        recs: list[dict] = []
        with ThreadPoolExecutor(max_workers=workers) as ex:
            for f in [ex.submit(_run, c, verbose) for c in cmds]:
                recs += parse_resource_usage(f.result())
        bad = resource_violations(recs)
        if bad:
            raise RuntimeError("kernels using scratch memory (not allowed):\n  " + "\n  ".join(bad))
        if not recs:
            raise RuntimeError("hipcc reported no kernel resource usage; the scratch check did not run")
        tmp = os.path.join(tmpdir, os.path.basename(out))
        _run([cc, *HIPCC_FLAGS, "-shared", *objs, "-o", tmp], verbose)
        os.chmod(tmp, 0o755)
        os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
