"""Build oracle/_ref/ (the reference's h4mv.cu compiled for gfx950) when /root/reference exists.

TEST INFRASTRUCTURE ONLY.  Runs ``make -C oracle`` (recipe: oracle/Makefile).  On machines without
the reference sources (the GPU box) the prebuilt oracle/_ref/libh4mv_ref.so is used as shipped.
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
REF_ROOT = os.environ.get("FP8KV_REFERENCE", "/root/reference")
REF_LIB = os.path.join(HERE, "_ref", "libh4mv_ref.so")


def build() -> str | None:
    if not os.path.exists(os.path.join(REF_ROOT, "h4mv", "h4mv.cu")):
        return REF_LIB if os.path.exists(REF_LIB) else None
    subprocess.run(["make", "-s", "-C", HERE, f"REF={REF_ROOT}"], check=True)
    return REF_LIB


if __name__ == "__main__":
    print(build())
