"""The vLLM hook layer (decode override, prefill override, MXFP4 linear hook, sitecustomize chain)
driven on the CPU through fake ``vllm`` / ``radiance_mxfp4`` module trees.

No kernel runs here: the HIP entry points are replaced by recorders, so these tests pin the
gates, argument mapping, fallbacks and patch chain of vllm-fp8kv/fp8kv_override.py,
vllm-fp8kv/fp8kv_prefill.py, h4mv/fp8kv_hipw4.py and vllm-fp8kv/sitecustomize.py.
"""
import enum
import importlib
import math
import sys
import types

import pytest
import torch


# ------------------------------------------------------------------------------ fake vLLM tree

class KVQuantMode(enum.Enum):
    NONE = 0
    FP8_PER_TENSOR = 1


def _fake_vllm(monkeypatch):
    calls = []

    class TritonAttentionImpl:
        def forward(self, layer, query, key, value, kv_cache, attn_metadata, output,
                    output_scale=None, output_block_scale=None):
            calls.append("stock")
            output.fill_(-1.0)
            return output

    class TritonAttentionBackend:
        pass

    class Attention:
        def process_weights_after_loading(self, act_dtype):
            return "pw"

    def mod(name, **attrs):
        m = types.ModuleType(name)
        m.__dict__.update(attrs)
        return m

    tree = {
        "vllm": mod("vllm"), "vllm.v1": mod("vllm.v1"), "vllm.v1.attention": mod("vllm.v1.attention"),
        "vllm.v1.attention.backends": mod("vllm.v1.attention.backends"),
        "vllm.v1.attention.backends.triton_attn": mod(
            "vllm.v1.attention.backends.triton_attn", TritonAttentionImpl=TritonAttentionImpl,
            TritonAttentionBackend=TritonAttentionBackend),
        "vllm.v1.kv_cache_interface": mod("vllm.v1.kv_cache_interface", KVQuantMode=KVQuantMode),
        "vllm.v1.attention.selector": mod("vllm.v1.attention.selector", get_attn_backend=lambda *a, **k: None),
        "vllm.model_executor": mod("vllm.model_executor"),
        "vllm.model_executor.layers": mod("vllm.model_executor.layers"),
        "vllm.model_executor.layers.attention": mod("vllm.model_executor.layers.attention"),
        "vllm.model_executor.layers.attention.attention": mod(
            "vllm.model_executor.layers.attention.attention", Attention=Attention),
    }
    for k, v in tree.items():
        monkeypatch.setitem(sys.modules, k, v)
    return TritonAttentionImpl, calls


class Recorder:
    """Stands in for the fp8kv_amd.ops kernel wrappers (no kernel runs on the CPU)."""

    def __init__(self, fail=False):
        self.calls = []
        self.fail = fail

    def __call__(self, name):
        def f(*a, **kw):
            self.calls.append((name, a, kw))
            if self.fail:
                raise RuntimeError("kernel failed")
            out = a[3]
            out.fill_(7.0)
            return out
        return f


def _impl(cls, **over):
    impl = cls()
    impl._kv_quant_mode = KVQuantMode.FP8_PER_TENSOR
    impl.head_size = 128
    impl.num_kv_heads = 4
    impl.num_queries_per_kv = 6
    impl.use_td = False
    impl.sliding_window = (-1, -1)
    impl.sinks = None
    impl.alibi_slopes = None
    impl.logits_soft_cap = 0
    impl.fp8_dtype = torch.float8_e4m3fn
    impl.scale = 1 / math.sqrt(128)
    for k, v in over.items():
        setattr(impl, k, v)
    return impl


def _batch(ns=3, max_q=1, nb=40, ctx=(100, 37, 250), qlens=None):
    qlens = qlens or [max_q] * ns
    T = sum(qlens)
    cu = torch.tensor([0] + list(torch.tensor(qlens).cumsum(0).tolist()), dtype=torch.int32)
    md = types.SimpleNamespace(
        max_query_len=max(qlens), num_actual_tokens=T, query_start_loc=cu,
        seq_lens=torch.tensor(list(ctx)[:ns], dtype=torch.int32),
        block_table=torch.arange(ns * 16, dtype=torch.int32).view(ns, 16),
        max_seq_len=max(list(ctx)[:ns]), use_cascade=False)
    layer = types.SimpleNamespace(_k_scale=torch.tensor([0.5]), _v_scale=torch.tensor([2.0]))
    kv = torch.zeros(nb, 4, 16, 256, dtype=torch.uint8)
    q = torch.zeros(T + 2, 24, 128, dtype=torch.bfloat16)
    out = torch.zeros(T + 2, 24, 128, dtype=torch.bfloat16)
    return md, layer, kv, q, out


def _fresh(monkeypatch, name):
    monkeypatch.delitem(sys.modules, name, raising=False)
    return importlib.import_module(name)


@pytest.fixture
def no_capture(monkeypatch):
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)


# ------------------------------------------------------------------------------ decode override

def test_engine_cache_views_match_reference_transpose_split():
    import fp8kv_override as ov
    kv = torch.arange(6 * 4 * 16 * 256, dtype=torch.int64).remainder(251).to(torch.uint8).view(6, 4, 16, 256)
    k, v = ov.engine_cache_views(kv, 128, torch.float8_e4m3fn)
    assert k.shape == (6, 16, 4, 128) and v.shape == (6, 16, 4, 128)
    assert k.stride() == (4 * 16 * 256, 256, 16 * 256, 1)
    assert k.data_ptr() == kv.data_ptr() and v.data_ptr() == kv.data_ptr() + 128
    assert torch.equal(k.view(torch.uint8)[2, 5, 3], kv[2, 3, 5, :128])
    assert torch.equal(v.view(torch.uint8)[2, 5, 3], kv[2, 3, 5, 128:])


@pytest.mark.parametrize("over,md_over", [
    ({}, {"max_query_len": 2}),
    ({"_kv_quant_mode": KVQuantMode.NONE}, {}),
    ({"head_size": 64}, {}),
    ({"use_td": True}, {}),
    ({"sliding_window": (128, 0)}, {}),
    ({"sinks": torch.zeros(1)}, {}),
    ({"alibi_slopes": torch.zeros(1)}, {}),
    ({"logits_soft_cap": 30.0}, {}),
])
def test_decode_gate_rejections_fall_through(monkeypatch, no_capture, over, md_over):
    cls, calls = _fake_vllm(monkeypatch)
    rec = Recorder()
    from fp8kv_amd import ops
    monkeypatch.setattr(ops, "decode_attention", rec("decode"))
    _fresh(monkeypatch, "fp8kv_override")
    md, layer, kv, q, out = _batch()
    for k, v in md_over.items():
        setattr(md, k, v)
    cls.forward(_impl(cls, **over), layer, q, None, None, kv, md, out)
    assert calls == ["stock"] and rec.calls == []


def test_decode_gate_missing_attribute_falls_through(monkeypatch, no_capture):
    cls, calls = _fake_vllm(monkeypatch)
    _fresh(monkeypatch, "fp8kv_override")
    impl = _impl(cls)
    del impl.sinks
    md, layer, kv, q, out = _batch()
    cls.forward(impl, layer, q, None, None, kv, md, out)
    assert calls == ["stock"]


def test_decode_fast_path_argument_mapping(monkeypatch, no_capture):
    cls, calls = _fake_vllm(monkeypatch)
    rec = Recorder()
    from fp8kv_amd import ops
    monkeypatch.setattr(ops, "decode_attention", rec("decode"))
    ov = _fresh(monkeypatch, "fp8kv_override")
    md, layer, kv, q, out = _batch()
    impl = _impl(cls)
    res = cls.forward(impl, layer, q, None, None, kv, md, out)
    assert calls == [] and res is out
    (name, a, kw), = rec.calls
    qq, kc, vc, oo, qsl, sl, bt, ks, vs, sm = a
    assert qq.shape[0] == 3 and oo.shape[0] == 3 and qq.data_ptr() == q.data_ptr()
    assert kc.shape == (40, 16, 4, 128) and kc.dtype == torch.float8_e4m3fn
    assert vc.data_ptr() == kv.data_ptr() + 128
    assert qsl is md.query_start_loc and sl is md.seq_lens and bt is md.block_table
    assert ks is layer._k_scale and vs is layer._v_scale and sm == impl.scale
    assert kw["num_splits"] == ops.decode_num_splits(3, 4, 250)
    assert torch.all(out[:3] == 7.0) and torch.all(out[3:] == 0)
    assert ov.COUNTERS["impl_forward"] >= 1


def test_decode_no_scratch_during_capture_falls_back(monkeypatch):
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    cls, calls = _fake_vllm(monkeypatch)
    rec = Recorder()
    from fp8kv_amd import ops
    monkeypatch.setattr(ops, "decode_attention", rec("decode"))
    monkeypatch.setattr(ops, "_scratch_cache", {})
    _fresh(monkeypatch, "fp8kv_override")
    md, layer, kv, q, out = _batch(ctx=(4000, 4000, 4000))
    cls.forward(_impl(cls), layer, q, None, None, kv, md, out)
    assert calls == ["stock"] and rec.calls == []


def test_decode_capture_plans_from_batch_shape(monkeypatch):
    """While capturing, the split count (baked into the graph) ignores the capture's max_seq_len:
    it is the plan for the batch shape with no context cap, the same for short and long dummies."""
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    cls, calls = _fake_vllm(monkeypatch)
    rec = Recorder()
    from fp8kv_amd import ops
    monkeypatch.setattr(ops, "decode_attention", rec("decode"))
    monkeypatch.setattr(ops, "_scratch_cache", {("cpu", 0): torch.zeros(ops.DECODE_SCRATCH_MIN_BYTES,
                                                                          dtype=torch.uint8)})
    ov = _fresh(monkeypatch, "fp8kv_override")
    for ctx in ((1, 1, 1), (250, 250, 250)):
        md, layer, kv, q, out = _batch(ctx=ctx)
        cls.forward(_impl(cls), layer, q, None, None, kv, md, out)
    assert calls == [] and len(rec.calls) == 2
    want = ops.decode_num_splits(3, 4, ov.CAPTURE_PLAN_SEQ_LEN)
    assert want > 1 and [kw["num_splits"] for _, _, kw in rec.calls] == [want, want]
    assert ops.decode_num_splits(3, 4, 1) == 1                 # what the dummy context would give


def test_decode_scratch_never_frees_a_replaced_buffer(monkeypatch):
    """A larger request replaces the cached scratch but keeps the old buffer alive (graphs captured
    with it replay into it)."""
    from fp8kv_amd import ops
    monkeypatch.setattr(ops, "_scratch_cache", {})
    monkeypatch.setattr(ops, "_scratch_retired", [])
    a = ops.decode_scratch(1000, "cpu")
    assert a.numel() == ops.DECODE_SCRATCH_MIN_BYTES and int(a.sum()) == 0
    assert ops.decode_scratch(5000, "cpu") is a
    b = ops.decode_scratch(ops.DECODE_SCRATCH_MIN_BYTES + 1, "cpu")
    assert b is not a and b.numel() >= ops.DECODE_SCRATCH_MIN_BYTES + 1
    assert ops._scratch_retired == [a]
    assert ops.decode_scratch(10, "cpu", allow_alloc=False) is b


def test_decode_errors_propagate(monkeypatch, no_capture):
    """fp8kv_override.py:102-106 does not catch kernel errors; neither does this hook."""
    cls, calls = _fake_vllm(monkeypatch)
    from fp8kv_amd import ops
    monkeypatch.setattr(ops, "decode_attention", Recorder(fail=True)("decode"))
    _fresh(monkeypatch, "fp8kv_override")
    md, layer, kv, q, out = _batch()
    with pytest.raises(RuntimeError):
        cls.forward(_impl(cls), layer, q, None, None, kv, md, out)


def test_install_skipped_without_vllm(monkeypatch, capsys):
    monkeypatch.setitem(sys.modules, "vllm", None)
    ov = _fresh(monkeypatch, "fp8kv_override")
    assert not ov._STATE["installed"]
    assert "install skipped" in capsys.readouterr().err


def test_force_triton_selector(monkeypatch, no_capture):
    cls, _ = _fake_vllm(monkeypatch)
    monkeypatch.setenv("FP8KV_FORCE_TRITON", "1")
    _fresh(monkeypatch, "fp8kv_override")
    sel = sys.modules["vllm.v1.attention.selector"]
    assert sel.get_attn_backend() is sys.modules["vllm.v1.attention.backends.triton_attn"].TritonAttentionBackend


# ------------------------------------------------------------------------------ prefill override

def test_prefill_not_installed_without_env(monkeypatch):
    cls, _ = _fake_vllm(monkeypatch)
    monkeypatch.delenv("FP8KV_PREFILL", raising=False)
    before = cls.forward
    pf = _fresh(monkeypatch, "fp8kv_prefill")
    assert not pf._STATE["installed"] and cls.forward is before


def _chain(monkeypatch, varlen="1"):
    cls, calls = _fake_vllm(monkeypatch)
    stock = cls.forward
    rec = Recorder()
    from fp8kv_amd import ops
    monkeypatch.setattr(ops, "decode_attention", rec("decode"))
    monkeypatch.setattr(ops, "prefill_attention", rec("prefill"))
    monkeypatch.setattr(ops, "prefill_attention_varlen", rec("varlen"))
    monkeypatch.setenv("FP8KV_PREFILL", "1")
    monkeypatch.setenv("FP8KV_PREFILL_VARLEN", varlen)
    ov = _fresh(monkeypatch, "fp8kv_override")
    pf = _fresh(monkeypatch, "fp8kv_prefill")
    return cls, calls, rec, stock, ov, pf


def test_patch_chain_order(monkeypatch, no_capture):
    """prefill wraps the decode override, which wraps stock (vllm-fp8kv/fp8kv_prefill.py:153)."""
    cls, calls, rec, stock, ov, pf = _chain(monkeypatch)
    assert cls.forward.__fp8kv_wraps__.__fp8kv_wraps__ is stock


def test_prefill_single_sequence_q0(monkeypatch, no_capture):
    cls, calls, rec, *_ = _chain(monkeypatch)
    md, layer, kv, q, out = _batch(ns=1, qlens=[100], ctx=(300,))
    cls.forward(_impl(cls), layer, q, None, None, kv, md, out)
    (name, a, kw), = rec.calls
    assert name == "prefill"
    q_, kc, vc, o_, bt, ks, vs, sm, q0, qlen = a
    assert (q0, qlen) == (200, 100) and q_.shape[0] == 100 and bt is md.block_table


def test_prefill_routes_decode_and_short_chunks(monkeypatch, no_capture):
    cls, calls, rec, *_ = _chain(monkeypatch)
    md, layer, kv, q, out = _batch()                                   # decode batch
    cls.forward(_impl(cls), layer, q, None, None, kv, md, out)
    assert [c[0] for c in rec.calls] == ["decode"]
    md, layer, kv, q, out = _batch(ns=1, qlens=[63], ctx=(63,))        # below the 64-token gate
    cls.forward(_impl(cls), layer, q, None, None, kv, md, out)
    assert calls == ["stock"]


def test_prefill_multi_sequence_varlen(monkeypatch, no_capture):
    cls, calls, rec, *_ = _chain(monkeypatch)
    md, layer, kv, q, out = _batch(ns=3, qlens=[70, 5, 64], ctx=(70, 105, 300))
    cls.forward(_impl(cls), layer, q, None, None, kv, md, out)
    (name, a, kw), = rec.calls
    assert name == "varlen" and kw["max_query_len"] == 70
    assert a[4] is md.query_start_loc and a[5] is md.seq_lens and a[6] is md.block_table


def test_prefill_multi_sequence_reference_gate(monkeypatch, no_capture):
    """FP8KV_PREFILL_VARLEN=0: exactly one sequence, like fp8kv_prefill.py:163."""
    cls, calls, rec, *_ = _chain(monkeypatch, varlen="0")
    md, layer, kv, q, out = _batch(ns=2, qlens=[70, 80], ctx=(70, 100))
    cls.forward(_impl(cls), layer, q, None, None, kv, md, out)
    assert calls == ["stock"] and rec.calls == []


def test_prefill_negative_q0_falls_through(monkeypatch, no_capture):
    cls, calls, rec, *_ = _chain(monkeypatch)
    md, layer, kv, q, out = _batch(ns=1, qlens=[100], ctx=(90,))     # max_seq_len < tokens
    cls.forward(_impl(cls), layer, q, None, None, kv, md, out)
    assert calls == ["stock"] and rec.calls == []


def test_prefill_cascade_batch_runs_varlen_on_full_contexts(monkeypatch, no_capture):
    """A cascade batch (shared prefix) goes to the varlen kernel with the full per-sequence
    metadata, whatever its sequence count."""
    cls, calls, rec, *_ = _chain(monkeypatch)
    md, layer, kv, q, out = _batch(ns=3, qlens=[70, 80, 64], ctx=(600, 610, 700))
    md.use_cascade = True
    cls.forward(_impl(cls), layer, q, None, None, kv, md, out)
    md1, layer, kv, q, out = _batch(ns=1, qlens=[100], ctx=(300,))
    md1.use_cascade = True
    cls.forward(_impl(cls), layer, q, None, None, kv, md1, out)
    assert calls == [] and [c[0] for c in rec.calls] == ["varlen", "varlen"]
    a = rec.calls[0][1]
    assert a[4] is md.query_start_loc and a[5] is md.seq_lens and a[6] is md.block_table


@pytest.mark.parametrize("env", [{"FP8KV_PREFILL_CASCADE": "0"}, {"FP8KV_PREFILL_VARLEN": "0"}])
def test_prefill_cascade_left_to_stock_when_disabled(monkeypatch, no_capture, env):
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    cls, calls, rec, *_ = _chain(monkeypatch, varlen=env.get("FP8KV_PREFILL_VARLEN", "1"))
    md, layer, kv, q, out = _batch(ns=2, qlens=[70, 80], ctx=(600, 610))
    md.use_cascade = True
    cls.forward(_impl(cls), layer, q, None, None, kv, md, out)
    assert calls == ["stock"] and rec.calls == []


def test_prefill_exception_falls_back(monkeypatch, no_capture, capsys):
    cls, calls, rec, *_ = _chain(monkeypatch)
    from fp8kv_amd import ops
    monkeypatch.setattr(ops, "prefill_attention", Recorder(fail=True)("prefill"))
    md, layer, kv, q, out = _batch(ns=1, qlens=[100], ctx=(300,))
    res = cls.forward(_impl(cls), layer, q, None, None, kv, md, out)
    assert calls == ["stock"] and torch.all(res[:100] == -1.0)
    assert "falling back" in capsys.readouterr().err


def test_reference_run_signatures(monkeypatch):
    """fp8kv_v3.run / fp8kv_prefill.run take the reference's arguments (extra knobs ignored)."""
    import fp8kv_prefill
    import fp8kv_v3
    from fp8kv_amd import ops
    rec = Recorder()
    monkeypatch.setattr(ops, "decode_attention", rec("decode"))
    monkeypatch.setattr(ops, "prefill_attention", rec("prefill"))
    out = torch.zeros(2, 24, 128)
    fp8kv_v3.run(None, None, None, out, None, torch.tensor([5]), None, 1.0, 1.0, 0.1,
                 TILE=64, warps=8, stages=2, nsplit=4, scratch=(1, 2, 3))
    fp8kv_prefill.run(None, None, None, out, None, 1.0, 1.0, 0.1, 3, 9, BM=16, BN=64, warps=4, stages=3)
    (n1, a1, k1), (n2, a2, k2) = rec.calls
    assert n1 == "decode" and k1["num_splits"] == 4 and k1["scratch"] is None
    assert n2 == "prefill" and a2[-2:] == (3, 9)


# ------------------------------------------------------------------------------ linear hook

class FakeLaunch:
    def __init__(self):
        self.calls = []

    def __call__(self, *a):
        self.calls.append(a)


def _hipw4(monkeypatch):
    return _fresh(monkeypatch, "fp8kv_hipw4")


def _lin(M=2, N=64, K=256, dtype=torch.bfloat16):
    x = torch.zeros(M, K, dtype=dtype)
    w = torch.zeros(N, K // 2, dtype=torch.uint8)
    s = torch.zeros(K // 32, N, dtype=torch.uint8)
    return x, w, s


def test_hipw4_not_installed_without_env(monkeypatch):
    monkeypatch.delenv("FP8KV_HIPW4", raising=False)
    h = _hipw4(monkeypatch)
    assert not h._STATE["installed"]


def test_hipw4_launcher_binding_matches_reference():
    import ctypes
    import fp8kv_hipw4 as h
    fn = h.load_launcher()
    assert fn.argtypes == [ctypes.c_void_p] * 4 + [ctypes.c_int] * 3 + [ctypes.c_void_p]
    assert fn.restype is None


@pytest.mark.parametrize("case", ["m0", "m_big", "fp32", "noncontig", "k_odd", "n_small", "scale_rows",
                                  "misaligned", "3d"])
def test_hipw4_gate_rejections(monkeypatch, case):
    h = _hipw4(monkeypatch)
    x, w, s = _lin()
    if case == "m0":
        x = x[:0]
    elif case == "m_big":
        x = torch.zeros(5, 256, dtype=torch.bfloat16)
    elif case == "fp32":
        x = x.float()
    elif case == "noncontig":
        x = torch.zeros(256, 2, dtype=torch.bfloat16).t()
    elif case == "k_odd":
        x, w, s = torch.zeros(2, 48, dtype=torch.bfloat16), torch.zeros(64, 24, dtype=torch.uint8), s[:1]
    elif case == "n_small":
        w = w[:4]
    elif case == "scale_rows":
        s = s[:3]
    elif case == "misaligned":
        w = torch.zeros(64 * 128 + 1, dtype=torch.uint8)[1:].view(64, 128)
    elif case == "3d":
        x = x[None]
    assert not h.fast_path_ok(x, w, s, 4, torch)


def test_hipw4_fast_path_and_repack_cache(monkeypatch):
    h = _hipw4(monkeypatch)
    launch = FakeLaunch()
    repack = h.ScaleRepack(lambda: False, transpose=lambda t: t.t().contiguous())
    body_calls = []
    patched = h.make_patched(lambda *a: body_calls.append(a) or "body", launch, repack, 4, torch,
                             lambda: 1234)
    x, w, s = _lin(M=3, N=64, K=256)
    s.copy_(torch.arange(s.numel()).view(s.shape).to(torch.uint8))
    out = patched(x, w, s, None)
    assert out.shape == (3, 64) and out.dtype == torch.bfloat16 and body_calls == []
    Wp, Sp, Xp, Op, N, K, M, stream = launch.calls[0]
    assert (Wp, Xp, Op, N, K, M, stream.value) == (w.data_ptr(), x.data_ptr(), out.data_ptr(), 64, 256, 3, 1234)
    st = repack.cache[(s.data_ptr(), tuple(s.shape))]
    assert Sp == st.data_ptr() and torch.equal(st, s.t()) and st.is_contiguous()
    patched(x, w, s, None)
    assert len(repack.cache) == 1 and launch.calls[1][1] == Sp            # cached, not repacked


def test_hipw4_capture_refuses_repack_and_falls_back(monkeypatch):
    h = _hipw4(monkeypatch)
    launch = FakeLaunch()
    patched = h.make_patched(lambda *a: "body", launch, h.ScaleRepack(lambda: True, transpose=lambda t: t.t().contiguous()), 4, torch, lambda: 0)
    x, w, s = _lin()
    assert patched(x, w, s, None) == "body" and launch.calls == []


def test_hipw4_exception_falls_back(monkeypatch):
    h = _hipw4(monkeypatch)

    def boom(*a):
        raise RuntimeError("launch failed")
    patched = h.make_patched(lambda *a: "body", boom,
                             h.ScaleRepack(lambda: False, transpose=lambda t: t.t().contiguous()),
                             4, torch, lambda: 0)
    x, w, s = _lin()
    assert patched(x, w, s, None) == "body"


def test_hipw4_rejected_launch_falls_back(monkeypatch):
    """The void h4mv_launch only records a rejection; the hook reads that status and runs the
    stolen body instead of returning its unwritten output tensor."""
    h = _hipw4(monkeypatch)
    launch = FakeLaunch()
    status = {"rc": 2}
    body_calls = []
    patched = h.make_patched(lambda *a: body_calls.append(a) or "body", launch,
                             h.ScaleRepack(lambda: False, transpose=lambda t: t.t().contiguous()),
                             4, torch, lambda: 0, last_status=lambda: status["rc"])
    x, w, s = _lin(M=3, N=64, K=256)
    assert patched(x, w, s, None) == "body" and len(launch.calls) == 1 and len(body_calls) == 1
    status["rc"] = 0
    out = patched(x, w, s, None)
    assert torch.is_tensor(out) and out.shape == (3, 64) and len(body_calls) == 1


@pytest.mark.parametrize("env,expect", [("4", 4), ("16", 16), ("17", 16), ("64", 16), ("0", 1), ("-3", 1)])
def test_hipw4_max_m_is_clamped(monkeypatch, capsys, env, expect):
    h = _hipw4(monkeypatch)
    assert h.clamp_max_m(env) == expect
    assert ("clamped" in capsys.readouterr().err) == (int(env) != expect)


def test_hipw4_batches_above_kernel_limit_never_launch(monkeypatch):
    """Even with a configured limit above the kernel's 16 rows, M = 17 runs the stolen body."""
    h = _hipw4(monkeypatch)
    launch = FakeLaunch()
    patched = h.make_patched(lambda *a: "body", launch,
                             h.ScaleRepack(lambda: False, transpose=lambda t: t.t().contiguous()),
                             64, torch, lambda: 0, last_status=lambda: 0)
    x, w, s = _lin(M=17, N=64, K=256)
    assert patched(x, w, s, None) == "body" and launch.calls == []
    x, w, s = _lin(M=16, N=64, K=256)
    assert torch.is_tensor(patched(x, w, s, None)) and len(launch.calls) == 1


def test_hipw4_status_binding():
    import ctypes
    import fp8kv_hipw4 as h
    fn = h.load_status()
    assert fn.argtypes == [] and fn.restype is ctypes.c_int and isinstance(fn(), int)


def test_hipw4_repack_cache_limit(monkeypatch):
    h = _hipw4(monkeypatch)
    rp = h.ScaleRepack(lambda: False, limit=3, transpose=lambda t: t.t().contiguous())
    keep = [torch.zeros(2, 8, dtype=torch.uint8) for _ in range(6)]
    for t in keep:
        rp(t)
    assert len(rp.cache) <= 4


def test_hipw4_steal_prefers_cuda_backend_fn():
    import fp8kv_hipw4 as h
    cuda_fn, init_fn = object(), object()
    rm = types.SimpleNamespace(mxfp4_linear=types.SimpleNamespace(_backend_fns={"cuda": cuda_fn}, _init_fn=init_fn))
    assert h.steal_body(rm) is cuda_fn
    rm.mxfp4_linear._backend_fns = {}
    assert h.steal_body(rm) is init_fn


def test_hipw4_poll_wperm_stands_down(monkeypatch, capsys):
    h = _hipw4(monkeypatch)
    monkeypatch.setitem(sys.modules, "radiance_mxfp4", types.SimpleNamespace(WPERM=True))
    registered = []
    monkeypatch.setattr(h, "register", lambda p, t: registered.append(p))
    h._poll(FakeLaunch(), 4, tries=2, delay=0)
    assert registered == [] and "standing down" in capsys.readouterr().err


def test_hipw4_poll_registers_patched_op(monkeypatch):
    h = _hipw4(monkeypatch)
    body = lambda *a: "body"  # noqa: E731
    rm = types.SimpleNamespace(WPERM=False, mxfp4_linear=types.SimpleNamespace(_backend_fns={"cuda": body}, _init_fn=None))
    monkeypatch.setitem(sys.modules, "radiance_mxfp4", rm)
    registered = []
    monkeypatch.setattr(h, "register", lambda p, t: registered.append(p))
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    h._poll(FakeLaunch(), 4, tries=2, delay=0)
    assert registered and h._STATE["body"] is body
    x, w, s = _lin(M=8)                               # M > MAXM: the stolen body runs
    assert registered[0](x, w, s, None) == "body"


def test_hipw4_poll_gives_up_without_radiance(monkeypatch, capsys):
    h = _hipw4(monkeypatch)
    monkeypatch.setitem(sys.modules, "radiance_mxfp4", None)
    h._poll(FakeLaunch(), 4, tries=2, delay=0)
    assert "never appeared" in capsys.readouterr().err


def test_sitecustomize_chain_without_vllm(monkeypatch):
    """Importing sitecustomize in a process without vLLM leaves everything untouched."""
    monkeypatch.setitem(sys.modules, "vllm", None)
    monkeypatch.delenv("FP8KV_PREFILL", raising=False)
    monkeypatch.delenv("FP8KV_HIPW4", raising=False)
    for m in ("sitecustomize", "fp8kv_override", "fp8kv_prefill", "fp8kv_hipw4"):
        monkeypatch.delitem(sys.modules, m, raising=False)
    import os
    from conftest import PKG_DIR
    spec = importlib.util.spec_from_file_location("fp8kv_sitecustomize", os.path.join(PKG_DIR, "sitecustomize.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    assert not sys.modules["fp8kv_override"]._STATE["installed"]
    assert not sys.modules["fp8kv_prefill"]._STATE["installed"]
    assert not sys.modules["fp8kv_hipw4"]._STATE["installed"]


def test_hipw4_gemm_path_for_large_batches(monkeypatch):
    """With the opt-in GEMM callable, M above the matvec limit goes to it (scales repacked once);
    without it the stolen body runs as in the reference."""
    h = _hipw4(monkeypatch)
    launch = FakeLaunch()
    repack = h.ScaleRepack(lambda: False, transpose=lambda t: t.t().contiguous())
    calls = []

    def gemm(x, w, st, out, stream):
        calls.append((x.data_ptr(), w.data_ptr(), st.data_ptr(), out.data_ptr(), tuple(out.shape), stream.value))

    patched = h.make_patched(lambda *a: "body", launch, repack, 4, torch, lambda: 77, gemm=gemm)
    x, w, s = _lin(M=40, N=64, K=256)
    out = patched(x, w, s, None)
    assert out.shape == (40, 64) and launch.calls == [] and len(calls) == 1
    xp, wp, sp, op, shape, stream = calls[0]
    assert (xp, wp, op, shape, stream) == (x.data_ptr(), w.data_ptr(), out.data_ptr(), (40, 64), 77)
    assert sp == repack.cache[(s.data_ptr(), tuple(s.shape))].data_ptr()
    x2, _, _ = _lin(M=2, N=64, K=256)
    patched(x2, w, s, None)
    assert len(launch.calls) == 1 and len(calls) == 1            # small M still takes the matvec
    plain = h.make_patched(lambda *a: "body", launch, repack, 4, torch, lambda: 0)
    assert plain(x, w, s, None) == "body"


@pytest.mark.parametrize("case", ["k_not_128", "n_odd", "small_m", "fp32"])
def test_hipw4_gemm_gate_rejections(monkeypatch, case):
    h = _hipw4(monkeypatch)
    x, w, s = _lin(M=40, N=64, K=256)
    if case == "k_not_128":
        x, w, s = torch.zeros(40, 96, dtype=torch.bfloat16), torch.zeros(64, 48, dtype=torch.uint8), s[:3]
    elif case == "n_odd":
        w = torch.zeros(66, 128, dtype=torch.uint8)
    elif case == "small_m":
        x = x[:4]
    elif case == "fp32":
        x = x.float()
    assert not h.gemm_path_ok(x, w, s, 4, torch)


def test_topk_workspace_never_frees_a_replaced_buffer(monkeypatch):
    """lm_head_topk's cached workspace: a larger request replaces it but keeps the old buffer
    alive (a captured graph replays into it), and no buffer is allocated when allocation is off."""
    from fp8kv_amd import ops
    monkeypatch.setattr(ops, "_topk_ws", {})
    monkeypatch.setattr(ops, "_topk_ws_retired", [])
    assert ops.topk_workspace(1000, "cpu", allow_alloc=False) is None
    a = ops.topk_workspace(1000, "cpu")
    assert a.numel() == 1000
    assert ops.topk_workspace(600, "cpu") is a
    assert ops.topk_workspace(5000, "cpu", allow_alloc=False) is None
    b = ops.topk_workspace(1500, "cpu")
    assert b is not a and b.numel() >= 2000
    assert ops._topk_ws_retired == [a]
    assert ops.topk_workspace(1800, "cpu", allow_alloc=False) is b
