"""MI355X (gfx950) kernels of the fp8-KV attention + MXFP4 matvec hot path.

Layout of this directory (put it on PYTHONPATH, where the reference used /opt/fp8kv):
  csrc/                 HIP kernels for gfx950 and the C ABI (declared in include/fp8kv_amd.h)
  libfp8kv_amd.so       the built library (fp8kv_amd.build)
  fp8kv_amd/            host package: build, ctypes loader, torch wrappers, synthetic workloads
  fp8kv_v3.py, fp8kv_prefill.py, fp8kv_override.py, fp8kv_hipw4.py, sitecustomize.py
                        the reference's module names and hook surface
"""
from . import _lib, build  # noqa: F401

__all__ = ["_lib", "build"]
