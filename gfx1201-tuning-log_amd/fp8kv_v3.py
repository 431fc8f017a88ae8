"""Paged fp8-KV decode attention entry point under the reference's module name.

Mirrors vllm-fp8kv/fp8kv_v3.py:116-139 ``run(q, k_cache, v_cache, out, qsl, slens, bt, kscale,
vscale, sm_scale, TILE=32, warps=4, stages=3, nsplit=8, scratch=None)``: same arguments, same
meaning, writes ``out[qsl[s]]`` for every sequence s (one query token each).  The work runs in
the gfx950 HIP kernel of libfp8kv_amd.so (``fp8kv_decode_attn``); there is no Triton and no CPU
path.  ``TILE``, ``warps`` and ``stages`` were Triton launch parameters and are accepted and
ignored (the HIP kernel's tiling is fixed).  ``nsplit`` is the number of context splits per
(sequence, kv head) as in the reference (any value in 1..256 gives the same result up to
rounding; ``None`` lets the library plan it from the longest context).  ``scratch`` is a
zero-initialised uint8 device buffer of at least ``fp8kv_amd.ops.decode_scratch_bytes`` bytes, or
None for a per-device cached one (the reference's (o, m, l) float tuple is also accepted and
replaced by the cached buffer, since the partial layout differs).  bf16 caches take the
reference's K_FP8 = False branch (fp8kv_v3.py:135): ``fp8kv_decode_attn_bf16``, scales ignored.
"""
from __future__ import annotations

import os
import sys

_PKG = os.path.dirname(os.path.abspath(__file__))
if _PKG not in sys.path:
    sys.path.insert(0, _PKG)

from fp8kv_amd import ops  # noqa: E402


def run(q, k_cache, v_cache, out, qsl, slens, bt, kscale, vscale, sm_scale,
        TILE=32, warps=4, stages=3, nsplit=8, scratch=None):
    del TILE, warps, stages
    if isinstance(scratch, (tuple, list)):
        scratch = None
    max_seq_len = None
    if nsplit is None:
        max_seq_len = int(slens.max().item()) if slens.numel() else 0
    return ops.decode_attention(q, k_cache, v_cache, out, qsl, slens, bt, kscale, vscale, sm_scale,
                                num_splits=nsplit, max_seq_len=max_seq_len, scratch=scratch)
