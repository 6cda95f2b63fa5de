"""Grouped-query attention through the KV handle (model.rs:766-783).

The reference expands each K/V head to n_heads / n_kv_heads consecutive query
heads before the prefill branch's attention, and takes that branch for S = 1
too when the head counts differ (model.rs:739).  The handle keeps the
compact K/V heads; sts_kv_set_query_heads makes q and out carry the query
heads.  Checked, for the chunked prefill at every precision (with and
without the bf16 mirror) and for the fused decode step and attend:
  - bit for bit against the same call on a handle whose caches hold the
    expanded heads (the oracle's gqa_expand of the compact ones), i.e. the
    grouping changes which K/V rows a query head reads and nothing else;
  - within the precision's bar of the f64 closed form over the expanded
    caches;
  - the compact caches bit-exact against the oracle's RoPE + cache write.
"""
import numpy as np
import pytest
import torch

import oracle
import sts_attn
from cases import scale_for

pytestmark = pytest.mark.gpu

PRECS = [sts_attn.PREC_F32, sts_attn.PREC_BF16_MFMA, sts_attn.PREC_F32_SPLIT_BF16]


def tol(prec):
    return 2e-2 if prec == sts_attn.PREC_BF16_MFMA else 1e-4


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("prec,mirror", [(p, False) for p in PRECS] +
                         [(sts_attn.PREC_BF16_MFMA, True)])
@pytest.mark.parametrize("Hq,Hkv,D,M,chunks", [
    (8, 2, 128, 300, (200, 150, 1)),   # wraps on the second chunk; S = 1 last
    (12, 4, 64, 129, (60, 65)),
    (32, 8, 128, 1000, (768, 256)),    # config-3-like chunk, group 4
])
def test_gqa_prefill(gpu, prec, mirror, Hq, Hkv, D, M, chunks):
    print(f"gqa prefill Hq={Hq} Hkv={Hkv} D={D} M={M} chunks={chunks} prec={prec} "
          f"mirror={mirror}", flush=True)
    rep = Hq // Hkv
    rope = sts_attn.RoPE(D, 4096)
    tabs = oracle.rope_tables(D, 4096)
    g = sts_attn.KVCache(M, Hkv, D, bf16_mirror=mirror, n_heads=Hq)
    e = sts_attn.KVCache(M, Hq, D)   # the same rows, heads expanded
    o = oracle.KvCounters(M)
    kref = np.zeros((1, Hkv, M, D), np.float32)
    vref = np.zeros((1, Hkv, M, D), np.float32)
    for it, S in enumerate(chunks):
        q = oracle.normal(140 + it, (1, S, Hq, D))
        k = oracle.normal(150 + it, (1, S, Hkv, D))
        v = oracle.normal(160 + it, (1, S, Hkv, D))
        got = host(g.prefill(dev(q[0]), dev(k[0]), dev(v[0]), scale_for(D), prec, rope=rope))
        # The expanded handle: the same K/V rows repeated per query head.
        ke = np.repeat(k, rep, axis=2)
        ve = np.repeat(v, rep, axis=2)
        want = host(e.prefill(dev(q[0]), dev(ke[0]), dev(ve[0]), scale_for(D), prec, rope=rope))
        np.testing.assert_array_equal(got, want)
        qr = oracle.rope_apply(q, o.offset, tabs)[0]
        kr = oracle.rope_apply(k, o.offset, tabs)
        oracle.cache_write(kr, kref, o.offset % M, M)
        oracle.cache_write(v, vref, o.offset % M, M)
        o.advance(S)
        kb, vb = g.read_buffers()
        np.testing.assert_array_equal(host(kb), kref)
        np.testing.assert_array_equal(host(vb), vref)
        kx = oracle.gqa_expand(kref[0], rep)
        vx = oracle.gqa_expand(vref[0], rep)
        ref = oracle.prefill_f64(qr, kx, vx, o.window_start(), o.len, scale_for(D))
        err = np.abs(got - ref).max()
        assert err < tol(prec), (it, err)
    assert sts_attn.device_errors() == 0


@pytest.mark.parametrize("B,Hq,Hkv,D,M,use_rope", [
    (1, 32, 8, 128, 1000, True),    # the 4-wave multi-split kernel, wrapped ring
    (2, 16, 4, 64, 700, True),
    (3, 8, 8, 128, 500, False),     # group 1 through the setter's default
    (2, 8, 2, 128, 40, False),      # the one-wave kernel (window <= 64)
])
def test_gqa_decode_step_and_attend(gpu, B, Hq, Hkv, D, M, use_rope):
    print(f"gqa decode B={B} Hq={Hq} Hkv={Hkv} D={D} M={M} rope={use_rope}", flush=True)
    rep = Hq // Hkv
    rope = sts_attn.RoPE(D, 8192) if use_rope else None
    tabs = oracle.rope_tables(D, 8192) if use_rope else None
    g = sts_attn.KVCache(M, Hkv, D, n_heads=Hq)
    e = sts_attn.KVCache(M, Hq, D)
    o = oracle.KvCounters(M)
    kref = np.zeros((B, Hkv, M, D), np.float32)
    vref = np.zeros((B, Hkv, M, D), np.float32)
    shift = (M * 7 + 3) % M
    k0 = oracle.normal(B * 100 + 1, (B, M - 3, Hkv, D))
    v0 = oracle.normal(B * 100 + 2, (B, M - 3, Hkv, D))
    g.advance(shift)
    g.update(dev(k0), dev(v0))
    e.advance(shift)
    e.update(dev(np.repeat(k0, rep, axis=2)), dev(np.repeat(v0, rep, axis=2)))
    o.advance(shift)
    oracle.cache_write(k0, kref, o.offset % M, M)
    oracle.cache_write(v0, vref, o.offset % M, M)
    o.advance(M - 3)
    for step in range(5):
        pos = o.offset
        q = oracle.normal(B * 100 + 10 * step + 3, (B, 1, Hq, D))
        k = oracle.normal(B * 100 + 10 * step + 4, (B, 1, Hkv, D))
        v = oracle.normal(B * 100 + 10 * step + 5, (B, 1, Hkv, D))
        got = host(g.decode_step(dev(q[:, 0]), dev(k[:, 0]), dev(v[:, 0]), scale_for(D),
                                 rope=rope))
        want = host(e.decode_step(dev(q[:, 0]), dev(np.repeat(k, rep, axis=2)[:, 0]),
                                  dev(np.repeat(v, rep, axis=2)[:, 0]), scale_for(D), rope=rope))
        np.testing.assert_array_equal(got, want)
        qr = oracle.rope_apply(q, pos, tabs) if use_rope else q
        kr = oracle.rope_apply(k, pos, tabs) if use_rope else k
        oracle.cache_write(kr, kref, o.offset % M, M)
        oracle.cache_write(v, vref, o.offset % M, M)
        o.advance(1)
        kb, vb = g.read_buffers()
        np.testing.assert_array_equal(host(kb), kref)
        np.testing.assert_array_equal(host(vb), vref)
        for b in range(B):
            kx = oracle.gqa_expand(kref[b], rep)
            vx = oracle.gqa_expand(vref[b], rep)
            ref = oracle.attention_ring_f64(qr[b, 0], kx, vx, o.window_start(), o.len,
                                            scale_for(D))
            assert np.abs(got[b] - ref).max() < 1e-4, (step, b)
    # attend over the current window, q with the query heads.
    qa = oracle.normal(B * 100 + 99, (B, Hq, D))
    got = host(g.attend(dev(qa), scale_for(D)))
    np.testing.assert_array_equal(got, host(e.attend(dev(qa), scale_for(D))))
    for b in range(B):
        ref = oracle.attention_ring_f64(qa[b], oracle.gqa_expand(kref[b], rep),
                                        oracle.gqa_expand(vref[b], rep), o.window_start(), o.len,
                                        scale_for(D))
        assert np.abs(got[b] - ref).max() < 1e-4
