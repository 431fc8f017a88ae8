"""Route fp8 per-tensor KV decode attention through the gfx950 decode kernel (vLLM hook).

Drop-in for vllm-fp8kv/fp8kv_override.py: importing this module replaces
``vllm.v1.attention.backends.triton_attn.TritonAttentionImpl.forward`` (fp8kv_override.py:109)
with a forward that, when the decode gate holds (fp8kv_override.py:50-64: fp8 per-tensor KV,
max_query_len == 1, head_size 128, no sliding window / sinks / alibi / soft cap / td), views the
engine's KV tensor as separate K and V fp8 caches (fp8kv_override.py:82-85) and runs
``fp8kv_decode_attn`` of libfp8kv_amd.so on the current stream; otherwise the original forward
runs.  As in the reference, decode-path errors propagate (fp8kv_override.py:102-106).

Differences, all on the host side:
  * the split count is planned from ``attn_metadata.max_seq_len`` (reference: fixed 8); while a
    graph is captured it is planned from the batch shape alone, so the captured count suits every
    context the graph replays;
  * the scratch buffer is the library's (zeroed once, reused); it is never allocated while the
    stream is being captured into a graph - a call that would need a bigger one during capture
    falls back to the original forward instead;
  * the reference's Triton ``_cast_kv_tile`` replacement for vLLM's stock fallback kernel
    (fp8kv_override.py:15-24) is not reproduced: it speeds up a path this hook does not take.

Environment: FP8KV_FORCE_TRITON (force vLLM's backend selector to the Triton backend, as in
fp8kv_override.py:122-129); FP8KV_OVERRIDE_COUNTERS=0 silences the 15-second counter line.
"""
from __future__ import annotations

import os
import sys
import threading

_PKG = os.path.dirname(os.path.abspath(__file__))
if _PKG not in sys.path:
    sys.path.insert(0, _PKG)

TAG = "[fp8kv-override]"
# Context length the split planner is given while a graph is being captured: long enough that the
# plan depends only on the batch shape (sequences x kv heads).
CAPTURE_PLAN_SEQ_LEN = 1 << 30
COUNTERS = {"impl_forward": 0, "fallback": 0}
_STATE = {"installed": False, "orig": None, "diag_done": False, "engaged": False}


def _log(msg: str) -> None:
    sys.stderr.write(f"{TAG} {msg}\n")


def decode_gate(impl, attn_metadata, fp8_per_tensor) -> bool:
    """The reference's decode gate (fp8kv_override.py:50-64); missing attributes mean no."""
    try:
        return bool(
            attn_metadata is not None
            and impl._kv_quant_mode == fp8_per_tensor
            and attn_metadata.max_query_len == 1
            and impl.head_size == 128
            and impl.num_kv_heads > 0
            and not impl.use_td
            and impl.sliding_window[0] < 0
            and impl.sinks is None
            and impl.alibi_slopes is None
            and impl.logits_soft_cap == 0
        )
    except AttributeError:
        return False


def engine_cache_views(kv_cache, head_size: int, fp8_dtype):
    """K and V fp8 views of the engine's [NB, HKV, PBLK, 2*D] cache (fp8kv_override.py:82-85)."""
    kc = kv_cache.transpose(1, 2)
    key_cache, value_cache = kc.split(head_size, dim=-1)
    return key_cache.view(fp8_dtype), value_cache.view(fp8_dtype)


def make_forward(orig, fp8_per_tensor, ops, is_capturing):
    """Build the replacement forward around ``orig`` (the forward it wraps).

    ``ops`` provides decode_num_splits / decode_scratch_bytes / decode_scratch / decode_attention
    (fp8kv_amd.ops); ``is_capturing()`` reports graph capture on the current stream.
    """

    def _forward(self, layer, query, key, value, kv_cache, attn_metadata, output,
                 output_scale=None, output_block_scale=None):
        fast_ok = decode_gate(self, attn_metadata, fp8_per_tensor)
        if not _STATE["diag_done"]:
            _STATE["diag_done"] = True
            try:
                _log(f"diag: mode={self._kv_quant_mode!r} maxq={attn_metadata.max_query_len} "
                     f"hs={self.head_size} sw={self.sliding_window} td={self.use_td} "
                     f"sinks={self.sinks is None} alibi={self.alibi_slopes is None} "
                     f"cap={self.logits_soft_cap} fast_ok={fast_ok}")
            except Exception as e:  # diagnostics never break the forward
                _log(f"diag-fail {e}")
        if not fast_ok:
            return orig(self, layer, query, key, value, kv_cache, attn_metadata,
                        output, output_scale, output_block_scale)

        n = attn_metadata.num_actual_tokens
        hs = self.head_size
        key_cache, value_cache = engine_cache_views(kv_cache, hs, self.fp8_dtype)
        NS = attn_metadata.query_start_loc.shape[0] - 1
        HKV = self.num_kv_heads
        HQ = query.shape[1]
        capturing = is_capturing()
        # Under capture the split count is baked into the graph and replayed for every later
        # batch of this size, whatever its contexts: plan it from the batch shape alone (the
        # planner's longest-context cap lifted), not from the capture's dummy max_seq_len.
        plan_len = CAPTURE_PLAN_SEQ_LEN if capturing else int(attn_metadata.max_seq_len)
        nsplit = ops.decode_num_splits(NS, HKV, plan_len)
        need = ops.decode_scratch_bytes(NS, HQ, HKV, nsplit, hs)
        scratch = ops.decode_scratch(need, query.device, allow_alloc=not capturing)
        if need > 0 and scratch is None:
            COUNTERS["fallback"] += 1
            _log(f"scratch of {need} bytes not allocated before graph capture; stock path")
            return orig(self, layer, query, key, value, kv_cache, attn_metadata,
                        output, output_scale, output_block_scale)
        COUNTERS["impl_forward"] += 1
        if not _STATE["engaged"]:
            _STATE["engaged"] = True
            _log(f"ENGAGED: NS={NS} HKV={HKV} hs={hs} GQA={HQ // HKV} nsplit={nsplit}")
        ops.decode_attention(query[:n], key_cache, value_cache, output[:n],
                             attn_metadata.query_start_loc, attn_metadata.seq_lens,
                             attn_metadata.block_table, layer._k_scale, layer._v_scale, self.scale,
                             num_splits=nsplit, scratch=scratch)
        return output

    _forward.__fp8kv_wraps__ = orig
    return _forward


def _reporter():
    import time
    last = None
    while True:
        time.sleep(15)
        snap = dict(COUNTERS)
        if snap != last:
            _log(f"counters: {snap}")
            last = snap


def _install() -> bool:
    try:
        import torch
        from vllm.v1.attention.backends.triton_attn import TritonAttentionImpl
        from vllm.v1.kv_cache_interface import KVQuantMode
        from fp8kv_amd import _lib, ops
        _lib.load()
    except Exception as e:
        _log(f"install skipped: {e}")
        return False

    orig = TritonAttentionImpl.forward
    TritonAttentionImpl.forward = make_forward(orig, KVQuantMode.FP8_PER_TENSOR, ops,
                                               torch.cuda.is_current_stream_capturing)
    _STATE.update(installed=True, orig=orig)

    if os.environ.get("FP8KV_OVERRIDE_COUNTERS", "1") != "0":
        threading.Thread(target=_reporter, daemon=True).start()

    try:
        from vllm.model_executor.layers.attention.attention import Attention as _Attn
        _orig_pw = _Attn.process_weights_after_loading

        def _pw(self, act_dtype):
            _log(f"layer impl = {self.impl.__class__.__name__} "
                 f"(VLLM_ATTENTION_BACKEND={os.environ.get('VLLM_ATTENTION_BACKEND')})")
            return _orig_pw(self, act_dtype)
        _Attn.process_weights_after_loading = _pw
    except Exception as e:
        _log(f"pw-probe fail {e}")

    if os.environ.get("FP8KV_FORCE_TRITON"):
        try:
            import vllm.v1.attention.selector as _sel
            from vllm.v1.attention.backends.triton_attn import TritonAttentionBackend as _TB
            _sel.get_attn_backend = lambda *a, **kw: _TB
            _log("selector forced to TritonAttentionBackend")
        except Exception as e:
            _log(f"force-triton fail {e}")

    _log("installed")
    return True


_install()
