"""One configs[4] decode layer (hidden 3584, 24/4 heads of 128, intermediate 18944, batch 8) run
through the library, stage by stage against the CPU oracle, and end to end against an oracle chain.

GPU chain: add+RMSNorm -> qkv matvec (N 4096, K 3584) -> fp8 KV-cache write of the new token ->
decode attention -> o matvec (N 3584, K 3072) -> add+RMSNorm -> fused gate/up matvec + SiLU-and-mul
(N 37888, K 3584) -> down matvec (N 3584, K 18944), all at M = 8 (the shapes of configs[4]).
Rotary embeddings, biases and the sampler are not part of the path and are left out.

Stage bars (each stage's oracle is fed the GPU's own input to that stage): matvecs within half a
bf16 ulp + 1e-4 max|ref| of the fp64 oracle (the matvec bar); the cache write bit-exact; decode
within rtol = atol = 1e-2; RMSNorm within one bf16 step (99% exact); the fused SiLU-and-mul
rel-to-max < 1e-2 of the oracle's fp64 matvec followed by SiLU-and-mul.  End to end, the GPU's
down output against an oracle chain that rounds every stage to bf16 like the engine does:
rel-to-max < 2e-2 (bf16 rounding differences carried through seven stages).
"""
import math

import numpy as np
import pytest
import torch

from fp8kv_amd import ops, workloads
from oracle import attention, epilogues as ep, kv_cache, matvec

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
H, HQ, HKV, D, I, M = 3584, 24, 4, 128, 18944, 8
EPS = 1e-6
MV_EXCESS = 1e-4


def _w(N, K, seed):
    c = workloads.w4_case(N=N, K=K, M=1, seed=seed)
    return c["W"], c["St"]


def _bf(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16)


def _steps_apart(a: torch.Tensor, b: np.ndarray) -> np.ndarray:
    ia = a.cpu().view(torch.int16).numpy().astype(np.int64)
    ib = _bf(b).view(torch.int16).numpy().astype(np.int64)
    return np.abs(ia - ib)


def test_configs4_layer_chain():
    g = torch.Generator().manual_seed(404)
    x = torch.randn(M, H, generator=g).to(torch.bfloat16)
    residual = (torch.randn(M, H, generator=g) * 2).to(torch.bfloat16)
    wn1 = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    wn2 = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    Wqkv, Sqkv = _w(HQ * D + 2 * HKV * D, H, 1)
    Wo, So = _w(H, HQ * D, 2)
    Wgu, Sgu = _w(2 * I, H, 3)
    Wd, Sd = _w(H, I, 4)
    ctx = [512, 1000, 64, 2047, 300, 777, 1, 1536]          # new token included
    c = workloads.decode_case(ctx, HQ=HQ, HKV=HKV, D=D, seed=405)
    ks, vs, sm = c["k_scale"], c["v_scale"], c["sm_scale"]
    bt = c["block_table"]
    slots = torch.tensor([int(bt[s, (n - 1) // 16]) * 16 + (n - 1) % 16 for s, n in enumerate(ctx)],
                         dtype=torch.int64)

    # ---- GPU chain ----------------------------------------------------------------------------
    d = workloads.to_device(c, DEV)
    xg, rg = x.to(DEV), residual.to(DEV)
    h1 = ops.fused_add_rmsnorm(xg, rg, wn1.to(DEV), EPS)
    res1 = rg.clone()
    qkv = ops.h4mv(h1, Wqkv.to(DEV), Sqkv.to(DEV))
    q = qkv[:, :HQ * D].view(M, HQ, D)
    k = qkv[:, HQ * D:HQ * D + HKV * D].view(M, HKV, D)
    v = qkv[:, HQ * D + HKV * D:].view(M, HKV, D)
    kc0, vc0 = d["k_cache"].clone(), d["v_cache"].clone()
    ksd = torch.tensor([ks], device=DEV)
    vsd = torch.tensor([vs], device=DEV)
    ops.cache_write(k.contiguous(), v.contiguous(), d["k_cache"], d["v_cache"], slots.to(DEV), ksd, vsd)
    attn = torch.empty(M, HQ, D, dtype=torch.bfloat16, device=DEV)
    qsl = torch.arange(M + 1, dtype=torch.int32, device=DEV)
    ops.decode_attention(q, d["k_cache"], d["v_cache"], attn, qsl, d["seq_lens"], d["block_table"],
                         ksd, vsd, sm)
    o = ops.h4mv(attn.view(M, HQ * D), Wo.to(DEV), So.to(DEV))
    h2 = ops.fused_add_rmsnorm(o, rg, wn2.to(DEV), EPS)
    wi, si = ops.interleave_gate_up(Wgu.to(DEV), Sgu.to(DEV))
    act = ops.h4mv_silu_mul(h2, wi, si)
    y = ops.h4mv(act, Wd.to(DEV), Sd.to(DEV))
    torch.cuda.synchronize()
    G = {n: t.cpu() for n, t in dict(h1=h1, res1=res1, qkv=qkv, attn=attn, o=o, res2=rg, h2=h2, act=act,
                                     y=y, kc=d["k_cache"], vc=d["v_cache"]).items()}

    f32 = lambda t: t.float().numpy()

    # ---- stage by stage: the oracle of each stage on the GPU's input to it -----------------------
    r_h1, r_res1 = ep.fused_add_rmsnorm(f32(x), f32(residual), f32(wn1), EPS)
    assert np.array_equal(f32(G["res1"]), r_res1)
    st = _steps_apart(G["h1"], r_h1)
    assert st.max() <= 1 and (st == 0).mean() >= 0.99
    assert matvec.bf16_excess_error(f32(G["qkv"]), matvec.w4mv(Wqkv.numpy(), Sqkv.numpy(), f32(G["h1"]))) < MV_EXCESS
    kc_ref = kc0.cpu().view(torch.uint8).numpy().copy()
    vc_ref = vc0.cpu().view(torch.uint8).numpy().copy()
    qkv_c = f32(G["qkv"])
    kv_cache.cache_write(qkv_c[:, HQ * D:HQ * D + HKV * D].reshape(M, HKV, D),
                         qkv_c[:, HQ * D + HKV * D:].reshape(M, HKV, D), kc_ref, vc_ref, slots.numpy(), ks, vs, 16)
    assert np.array_equal(G["kc"].view(torch.uint8).numpy(), kc_ref)
    assert np.array_equal(G["vc"].view(torch.uint8).numpy(), vc_ref)
    r_attn = attention.decode_attention(G["qkv"][:, :HQ * D].reshape(M, HQ, D), G["kc"], G["vc"],
                                        torch.arange(M + 1, dtype=torch.int32), c["seq_lens"], bt, ks, vs, sm)
    torch.testing.assert_close(G["attn"].to(torch.float64), r_attn, rtol=1e-2, atol=1e-2)
    assert matvec.bf16_excess_error(f32(G["o"]), matvec.w4mv(Wo.numpy(), So.numpy(), f32(G["attn"]).reshape(M, -1))) < MV_EXCESS
    r_h2, r_res2 = ep.fused_add_rmsnorm(f32(G["o"]), f32(G["res1"]), f32(wn2), EPS)
    assert np.array_equal(f32(G["res2"]), r_res2)
    st = _steps_apart(G["h2"], r_h2)
    assert st.max() <= 1 and (st == 0).mean() >= 0.99
    gu = matvec.w4mv(Wgu.numpy(), Sgu.numpy(), f32(G["h2"]))
    r_act = ep.silu_mul(ep.bf16_round(gu.astype(np.float32)))
    assert matvec.rel_to_max_error(f32(G["act"]), r_act) < 1e-2
    assert matvec.bf16_excess_error(f32(G["y"]), matvec.w4mv(Wd.numpy(), Sd.numpy(), f32(G["act"]))) < MV_EXCESS

    # ---- end to end: the oracle chain from the same inputs ---------------------------------------
    bf = lambda a: ep.bf16_round(np.asarray(a, np.float32))
    e_h1, e_res1 = ep.fused_add_rmsnorm(f32(x), f32(residual), f32(wn1), EPS)
    e_qkv = bf(matvec.w4mv(Wqkv.numpy(), Sqkv.numpy(), e_h1))
    kc_e = kc0.cpu().view(torch.uint8).numpy().copy()
    vc_e = vc0.cpu().view(torch.uint8).numpy().copy()
    kv_cache.cache_write(e_qkv[:, HQ * D:HQ * D + HKV * D].reshape(M, HKV, D),
                         e_qkv[:, HQ * D + HKV * D:].reshape(M, HKV, D), kc_e, vc_e, slots.numpy(), ks, vs, 16)
    e_attn = attention.decode_attention(torch.from_numpy(e_qkv[:, :HQ * D].reshape(M, HQ, D)),
                                        torch.from_numpy(kc_e), torch.from_numpy(vc_e),
                                        torch.arange(M + 1, dtype=torch.int32), c["seq_lens"], bt, ks, vs, sm)
    e_attn = bf(e_attn.numpy())
    e_o = bf(matvec.w4mv(Wo.numpy(), So.numpy(), e_attn.reshape(M, -1)))
    e_h2, _ = ep.fused_add_rmsnorm(e_o, e_res1, f32(wn2), EPS)
    e_act = ep.silu_mul(bf(matvec.w4mv(Wgu.numpy(), Sgu.numpy(), e_h2)))
    e_y = matvec.w4mv(Wd.numpy(), Sd.numpy(), e_act)
    err = matvec.rel_to_max_error(f32(G["y"]), e_y)
    print(f"configs[4] layer chain: end-to-end rel-to-max {err:.2e}")
    assert err < 2e-2
