"""fp8-KV causal prefill attention on gfx950, and its vLLM hook, under the reference's module name.

Drop-in for vllm-fp8kv/fp8kv_prefill.py:
  * ``run(q, k_cache, v_cache, out, bt, kscale, vscale, sm_scale, q0, qlen, BM=64, BN=32,
    warps=2, stages=2)`` (fp8kv_prefill.py:124-144): one sequence whose context is block-table row
    0, query i is token q0 + i; the work runs in ``fp8kv_prefill_attn`` of libfp8kv_amd.so.  BM,
    BN, warps and stages were Triton tiling knobs and are accepted and ignored.
  * with FP8KV_PREFILL=1, importing the module wraps ``TritonAttentionImpl.forward`` (whatever it
    is at import time - the decode override when imported after it, fp8kv_prefill.py:153) with the
    prefill gate of fp8kv_prefill.py:158-181: fp8 per-tensor KV, max_query_len >= 64, head_size
    128, no sliding window / sinks / alibi / soft cap / td / cascade.  q0 = max_seq_len -
    num_actual_tokens (fp8kv_prefill.py:179).  Errors are logged and the wrapped forward runs
    (fp8kv_prefill.py:193-196).

Extension: the reference takes exactly one sequence (fp8kv_prefill.py:163); batches of several
sequences go to ``fp8kv_prefill_attn_varlen`` here (each sequence's q0 is seq_lens[s] - qlen_s on
the device).  FP8KV_PREFILL_VARLEN=0 restores the single-sequence gate; FP8KV_PREFILL_MIN_Q
(default 64) is the max_query_len threshold.  Cascade batches (requests sharing a prefix), which
the reference leaves to stock vLLM (fp8kv_prefill.py:168), also go to the varlen kernel: vLLM's
cascade metadata keeps every sequence's full block table and length next to the shared-prefix
fields, and attention over each full context is exactly what the prefix / suffix decomposition
computes.  FP8KV_PREFILL_CASCADE=0 (or FP8KV_PREFILL_VARLEN=0) leaves them to stock.
"""
from __future__ import annotations

import os
import sys

_PKG = os.path.dirname(os.path.abspath(__file__))
if _PKG not in sys.path:
    sys.path.insert(0, _PKG)

TAG = "[fp8kv-prefill]"
_STATE = {"installed": False, "next": None, "engaged": False}


def _log(msg: str) -> None:
    sys.stderr.write(f"{TAG} {msg}\n")


def run(q, k_cache, v_cache, out, bt, kscale, vscale, sm_scale, q0, qlen,
        BM=64, BN=32, warps=2, stages=2):
    del BM, BN, warps, stages
    from fp8kv_amd import ops
    return ops.prefill_attention(q, k_cache, v_cache, out, bt, kscale, vscale, sm_scale, q0, qlen)


def prefill_gate(impl, attn_metadata, fp8_per_tensor, min_q: int = 64, varlen: bool = True,
                 cascade: bool = True) -> bool:
    """The reference's prefill gate (fp8kv_prefill.py:158-172), optionally without the
    single-sequence condition and, on the varlen path, without the no-cascade condition; missing
    attributes mean no."""
    try:
        nseq_ok = (attn_metadata.query_start_loc.shape[0] >= 2 if varlen
                   else attn_metadata.query_start_loc.shape[0] == 2)
        cascade_ok = not getattr(attn_metadata, "use_cascade", False) or (cascade and varlen)
        return bool(
            attn_metadata is not None
            and impl._kv_quant_mode == fp8_per_tensor
            and attn_metadata.max_query_len >= min_q
            and nseq_ok
            and impl.head_size == 128
            and impl.num_kv_heads > 0
            and not impl.use_td
            and impl.sliding_window[0] < 0
            and impl.sinks is None
            and impl.alibi_slopes is None
            and impl.logits_soft_cap == 0
            and cascade_ok
        )
    except AttributeError:
        return False


def make_forward(nxt, fp8_per_tensor, ops, min_q: int = 64, varlen: bool = True, cascade: bool = True):
    """Build the prefill forward wrapping ``nxt`` (the forward in place before this hook)."""
    from fp8kv_override import engine_cache_views

    def _forward(self, layer, query, key, value, kv_cache, attn_metadata, output,
                 output_scale=None, output_block_scale=None):
        if prefill_gate(self, attn_metadata, fp8_per_tensor, min_q, varlen, cascade):
            try:
                n = int(attn_metadata.num_actual_tokens)
                hs = self.head_size
                key_cache, value_cache = engine_cache_views(kv_cache, hs, self.fp8_dtype)
                nseq = attn_metadata.query_start_loc.shape[0] - 1
                done = False
                use_cascade = bool(getattr(attn_metadata, "use_cascade", False))
                if nseq == 1 and not use_cascade:
                    q0 = int(attn_metadata.max_seq_len) - n       # no num_computed_tokens in this vLLM
                    if 0 <= q0 and n >= min_q:
                        ops.prefill_attention(query[:n], key_cache, value_cache, output[:n],
                                              attn_metadata.block_table, layer._k_scale,
                                              layer._v_scale, self.scale, q0, n)
                        done = True
                        desc = f"qlen={n} q0={q0}"
                else:
                    ops.prefill_attention_varlen(query[:n], key_cache, value_cache, output[:n],
                                                 attn_metadata.query_start_loc,
                                                 attn_metadata.seq_lens, attn_metadata.block_table,
                                                 layer._k_scale, layer._v_scale, self.scale,
                                                 max_query_len=int(attn_metadata.max_query_len))
                    done = True
                    desc = f"varlen nseq={nseq} tokens={n}" + (" cascade" if use_cascade else "")
                if done:
                    if not _STATE["engaged"]:
                        _STATE["engaged"] = True
                        _log(f"ENGAGED {desc}")
                    return output
            except Exception as e:
                _log(f"fast path failed ({e!r}), falling back")
        return nxt(self, layer, query, key, value, kv_cache, attn_metadata,
                   output, output_scale, output_block_scale)

    _forward.__fp8kv_wraps__ = nxt
    return _forward


def _install() -> bool:
    if os.environ.get("FP8KV_PREFILL", "0") != "1":
        return False
    try:
        from vllm.v1.attention.backends.triton_attn import TritonAttentionImpl
        from vllm.v1.kv_cache_interface import KVQuantMode
        from fp8kv_amd import _lib, ops
        _lib.load()
    except Exception as e:
        _log(f"install skipped: {e}")
        return False
    nxt = TritonAttentionImpl.forward
    TritonAttentionImpl.forward = make_forward(
        nxt, KVQuantMode.FP8_PER_TENSOR, ops,
        min_q=int(os.environ.get("FP8KV_PREFILL_MIN_Q", "64")),
        varlen=os.environ.get("FP8KV_PREFILL_VARLEN", "1") != "0",
        cascade=os.environ.get("FP8KV_PREFILL_CASCADE", "1") != "0")
    _STATE.update(installed=True, next=nxt)
    _log("installed")
    return True


_install()
