"""CPU oracle for the fp8-KV attention + MXFP4 matvec hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (the gfx1201-tuning-log_amd/ package, its
C ABI or its vLLM hooks) imports this package.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker.

Each function restates the reference's algorithm on the CPU in fp32/fp64 torch or numpy and
cites the reference file:line it follows.  How each function is pinned (checked against
something other than itself) is listed in its module docstring; every function here has at
least one such check in ``tests/test_oracle.py``.
"""
from . import formats, matvec, attention, kv_cache, epilogues, w4a8, lm_head  # noqa: F401
