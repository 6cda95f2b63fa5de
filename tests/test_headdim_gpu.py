"""Head dims other than 64 and 128 (multiples of 4 up to 128).

The reference's shader takes any head_dim up to 128 (shader_attention.wgsl:36,
one register array of MAX_HD = 128 per lane).  Here 64 and 128 run their own
kernels and the other multiples of 4 a padded instance of the decode kernel
(lanes past the head dim load zeros and store nothing); the chunk prefill at
those dims runs the same kernel with query i as a decode over window rows
0..len-S+i (the S sequential decodes the reference's prefill stands for), in
f32 whatever precision is asked for.  Checked against the shader-order and
f64 oracles within 1e-4, with caches and appended rows bit-exact.
"""
import numpy as np
import pytest
import torch

import oracle
import sts_attn
from cases import decode_inputs, prefill_inputs, scale_for

pytestmark = pytest.mark.gpu

TOL = 1e-4


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("H,D,M,L,start", [
    (4, 96, 300, 300, 77),     # 4-wave multi-split kernel, wrapped window
    (8, 32, 200, 150, 120),
    (3, 80, 50, 37, 40),       # one-wave kernel
    (2, 4, 500, 411, 499),
    (2, 124, 1000, 999, 3),
])
def test_fused_and_ring_decode(gpu, H, D, M, L, start):
    print(f"head_dim decode H={H} D={D} M={M} L={L} start={start}", flush=True)
    q, kc, vc = decode_inputs(900 + D, H, D, M, L, start)
    s = scale_for(D)
    ref = oracle.attention_ring_f64(q, kc, vc, start, L, s)
    wg = oracle.attention_ring_wgsl(q, kc, vc, start, L, s)
    # Ragged ring decode of a batch of 2 streams over the same caches.
    lens = torch.tensor([L, L], dtype=torch.int32, device="cuda")
    starts = torch.tensor([start, start], dtype=torch.int32, device="cuda")
    qb = dev(np.stack([q, q]))
    got = host(sts_attn.decode_ring(qb, dev(np.stack([kc, kc])), dev(np.stack([vc, vc])), lens,
                                    starts, s))
    for b in range(2):
        assert np.abs(got[b] - ref).max() < TOL
        assert np.abs(got[b] - wg).max() < TOL
    np.testing.assert_array_equal(got[0], got[1])
    if start + L <= M:
        # fused_attention over a contiguous [1, H, M, D] view (rows 0..L-1 from start).
        kv = kc[:, start:start + L]
        vv = vc[:, start:start + L]
        out = host(sts_attn.fused_attention(dev(q), dev(kv[None]), dev(vv[None]), s))
        assert np.abs(out.reshape(H, D) - ref).max() < TOL


@pytest.mark.parametrize("D", [96, 32, 112])
def test_kv_handle_decode_step_and_prefill(gpu, D):
    """decode_step with RoPE and chunked prefill (every precision accepted, f32
    arithmetic) through one handle, against the oracle's RoPE + cache write and
    the f64 closed forms."""
    print(f"head_dim handle D={D}", flush=True)
    H, M = 4, 257
    rope = sts_attn.RoPE(D, 4096)
    tabs = oracle.rope_tables(D, 4096)
    c = sts_attn.KVCache(M, H, D)
    o = oracle.KvCounters(M)
    kref = np.zeros((1, H, M, D), np.float32)
    vref = np.zeros((1, H, M, D), np.float32)
    precs = [sts_attn.PREC_F32, sts_attn.PREC_BF16_MFMA, sts_attn.PREC_F32_SPLIT_BF16]
    for it, S in enumerate((200, 1, 90, 3, 17)):   # precisions f32, -, split, f32, bf16
        q = oracle.normal(700 + it, (1, S, H, D))
        k = oracle.normal(710 + it, (1, S, H, D))
        v = oracle.normal(720 + it, (1, S, H, D))
        qr = oracle.rope_apply(q, o.offset, tabs)[0]
        kr = oracle.rope_apply(k, o.offset, tabs)
        if S == 1:
            got = host(c.decode_step(dev(q[:, 0]), dev(k[:, 0]), dev(v[:, 0]), scale_for(D),
                                     rope=rope))
        else:
            got = host(c.prefill(dev(q[0]), dev(k[0]), dev(v[0]), scale_for(D),
                                 precs[it % 3], rope=rope))
        oracle.cache_write(kr, kref, o.offset % M, M)
        oracle.cache_write(v, vref, o.offset % M, M)
        o.advance(S)
        kb, vb = c.read_buffers()
        np.testing.assert_array_equal(host(kb), kref)
        np.testing.assert_array_equal(host(vb), vref)
        ref = oracle.prefill_f64(qr, kref[0], vref[0], o.window_start(), o.len, scale_for(D))
        assert np.abs(got.reshape(S, H, D) - ref).max() < TOL, it
    # The standalone prefill entry at this head dim.
    q, kc, vc = prefill_inputs(31, H, D, M, 100, 60, 230)
    got = host(sts_attn.prefill_attention(dev(q), dev(kc), dev(vc), 230, 160, scale_for(D)))
    ref = oracle.prefill_f64(q, kc, vc, 230, 160, scale_for(D))
    assert np.abs(got - ref).max() < TOL
    seq = oracle.prefill_seq_wgsl(q, kc, vc, 230, 160, scale_for(D))
    assert np.abs(got - seq).max() < TOL


@pytest.mark.parametrize("Hq,Hkv,D,M", [(8, 2, 96, 150), (6, 3, 32, 100)])
def test_gqa_at_padded_head_dims(gpu, Hq, Hkv, D, M):
    """Grouped-query attention (model.rs:766-783) at a head dim that runs the
    padded decode kernel: chunked prefill with RoPE (every precision asks for
    the same f32 per-query decodes here), the fused decode step and attend,
    bit for bit against a handle holding the expanded K/V heads and within
    1e-4 of the f64 closed form over the expanded caches."""
    print(f"gqa head_dim Hq={Hq} Hkv={Hkv} D={D} M={M}", flush=True)
    rep = Hq // Hkv
    rope = sts_attn.RoPE(D, 4096)
    tabs = oracle.rope_tables(D, 4096)
    g = sts_attn.KVCache(M, Hkv, D, n_heads=Hq)
    e = sts_attn.KVCache(M, Hq, D)
    o = oracle.KvCounters(M)
    kref = np.zeros((1, Hkv, M, D), np.float32)
    vref = np.zeros((1, Hkv, M, D), np.float32)
    for it, S in enumerate((90, 1, 45, 3, 1)):
        q = oracle.normal(400 + it, (1, S, Hq, D))
        k = oracle.normal(410 + it, (1, S, Hkv, D))
        v = oracle.normal(420 + it, (1, S, Hkv, D))
        ke, ve = np.repeat(k, rep, axis=2), np.repeat(v, rep, axis=2)
        if S == 1:
            got = host(g.decode_step(dev(q[:, 0]), dev(k[:, 0]), dev(v[:, 0]), scale_for(D),
                                     rope=rope))
            want = host(e.decode_step(dev(q[:, 0]), dev(ke[:, 0]), dev(ve[:, 0]), scale_for(D),
                                      rope=rope))
        else:
            got = host(g.prefill(dev(q[0]), dev(k[0]), dev(v[0]), scale_for(D),
                                 sts_attn.PREC_BF16_MFMA, rope=rope))
            want = host(e.prefill(dev(q[0]), dev(ke[0]), dev(ve[0]), scale_for(D),
                                  sts_attn.PREC_BF16_MFMA, rope=rope))
        np.testing.assert_array_equal(got, want)
        qr = oracle.rope_apply(q, o.offset, tabs)[0]
        kr = oracle.rope_apply(k, o.offset, tabs)
        oracle.cache_write(kr, kref, o.offset % M, M)
        oracle.cache_write(v, vref, o.offset % M, M)
        o.advance(S)
        kb, vb = g.read_buffers()
        np.testing.assert_array_equal(host(kb), kref)
        np.testing.assert_array_equal(host(vb), vref)
        kx, vx = oracle.gqa_expand(kref[0], rep), oracle.gqa_expand(vref[0], rep)
        ref = oracle.prefill_f64(qr, kx, vx, o.window_start(), o.len, scale_for(D))
        assert np.abs(got.reshape(S, Hq, D) - ref).max() < TOL, it
    qa = oracle.normal(499, (1, Hq, D))
    got = host(g.attend(dev(qa), scale_for(D)))
    np.testing.assert_array_equal(got, host(e.attend(dev(qa), scale_for(D))))
    ref = oracle.attention_ring_f64(qa[0], oracle.gqa_expand(kref[0], rep),
                                    oracle.gqa_expand(vref[0], rep), o.window_start(), o.len,
                                    scale_for(D))
    assert np.abs(got[0] - ref).max() < TOL
