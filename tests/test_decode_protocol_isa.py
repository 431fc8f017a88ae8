"""The decode split-merge protocol in the compiled gfx950 code (CPU only: hipcc cross-compiles).

Each split writes its (o, m, l) record with device-coherent (`sc1`) stores, waits for them with
`s_waitcnt vmcnt(0)`, and only then takes its ticket with an agent-scope atomic add; the workgroup
that draws the last ticket reads the records with device-coherent loads issued after the atomic's
result has arrived.  The argument for that order is about instructions, not about the C++ source,
so this test checks the instructions every decode kernel variant compiles to, and checks that the
checker itself rejects planted breaks of each rule.
"""
import os
import re
import subprocess

import pytest

from fp8kv_amd import build

HIPCC = None
try:
    HIPCC = build.hipcc()
except FileNotFoundError:
    pass

pytestmark = pytest.mark.skipif(HIPCC is None, reason="hipcc not installed")


def _kernels(asm: str):
    """{symbol: [instruction lines]} for every decode kernel in the assembly."""
    out = {}
    for m in re.finditer(r"^(_ZN5fp8kv13decode_detail\d+decode_\w*kernel\w*):", asm, re.M):
        name = m.group(1)
        end = asm.index(".Lfunc_end", m.end())
        body = [ln.strip() for ln in asm[m.end():end].splitlines()]
        out[name] = [ln for ln in body if ln and not ln.startswith((";", "."))]
    return out


def protocol_errors(lines):
    """Rule violations in one kernel's instruction list (empty when the protocol holds)."""
    errs = []
    at = [i for i, ln in enumerate(lines) if ln.startswith("global_atomic_add")]
    if not at:
        return ["no ticket atomic"]
    a = at[0]
    waits = [i for i in range(a) if lines[i].startswith("s_waitcnt") and "vmcnt(0)" in lines[i]]
    if not waits:
        return ["no vmcnt(0) before the ticket"]
    w = waits[-1]
    bars = [i for i in range(w) if lines[i].startswith("s_barrier")]
    start = bars[-1] if bars else 0
    stores = [i for i in range(start, w) if lines[i].startswith("global_store")]
    if not stores:
        errs.append("no record stores before the ticket's wait")
    errs += [f"record store without sc1: {lines[i]}" for i in stores if not re.search(r"\bsc1\b", lines[i])]
    errs += [f"store between the wait and the ticket: {lines[i]}" for i in range(w + 1, a)
             if lines[i].startswith("global_store")]
    rw = [i for i in range(a + 1, len(lines)) if lines[i].startswith("s_waitcnt") and "vmcnt(0)" in lines[i]]
    if not rw:
        return errs + ["the ticket's value is never waited for"]
    loads = [i for i in range(a + 1, len(lines)) if lines[i].startswith("global_load")]
    errs += [f"merge load before the ticket's value arrived: {lines[i]}" for i in loads if i < rw[0]]
    errs += [f"merge load without sc1: {lines[i]}" for i in loads if not re.search(r"\bsc1\b", lines[i])]
    if not loads:
        errs.append("no merge loads after the ticket")
    return errs


@pytest.fixture(scope="module")
def decode_asm(tmp_path_factory):
    out = tmp_path_factory.mktemp("isa") / "decode_attn.s"
    src = os.path.join(build.CSRC, "decode_attn.hip")
    cmd = [HIPCC, *build.HIPCC_FLAGS, *build.FILE_FLAGS.get("decode_attn.hip", []), f"-I{build.INCLUDE}",
           f"-I{build.CSRC}", "--cuda-device-only", "-S", src, "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text()


def test_every_decode_kernel_keeps_the_protocol(decode_asm):
    kernels = _kernels(decode_asm)
    # seven e4m3 launch variants and the bf16-cache kernel
    assert len(kernels) >= 8, sorted(kernels)
    for name, lines in kernels.items():
        assert protocol_errors(lines) == [], name


def test_checker_rejects_planted_breaks(decode_asm):
    name, lines = next(iter(_kernels(decode_asm).items()))
    assert protocol_errors(lines) == []
    a = next(i for i, ln in enumerate(lines) if ln.startswith("global_atomic_add"))
    w = max(i for i in range(a) if lines[i].startswith("s_waitcnt") and "vmcnt(0)" in lines[i])
    st = max(i for i in range(w) if lines[i].startswith("global_store"))
    ld = next(i for i in range(a + 1, len(lines)) if lines[i].startswith("global_load"))

    no_sc1_store = list(lines)
    no_sc1_store[st] = re.sub(r"\s*\bsc1\b", "", lines[st])
    assert any("record store without sc1" in e for e in protocol_errors(no_sc1_store))

    no_wait = [ln for i, ln in enumerate(lines) if i != w]
    assert protocol_errors(no_wait) != []

    late_store = list(lines)
    late_store.insert(a, lines[st])
    assert any("between the wait and the ticket" in e for e in protocol_errors(late_store))

    no_sc1_load = list(lines)
    no_sc1_load[ld] = re.sub(r"\s*\bsc1\b", "", lines[ld])
    assert any("merge load without sc1" in e for e in protocol_errors(no_sc1_load))

    early_load = list(lines)
    early_load.insert(a + 1, lines[ld])
    assert any("before the ticket's value arrived" in e for e in protocol_errors(early_load))
