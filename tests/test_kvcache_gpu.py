"""The HBM KV cache and its append on the GPU: slot indexing bit for bit.

Mirrors the reference's KVCache tests (crates/sts-wasm/src/model.rs:1459-1552)
with real data in the buffers, and checks every append against the oracle's
restatement of shader_cache_write.wgsl.  The fused decode step (RoPE + append
+ advance + attend in one launch) is checked against the unfused sequence.
"""
import numpy as np
import pytest
import torch

import oracle
import sts_attn
from cases import scale_for

pytestmark = pytest.mark.gpu


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("B,S,H,D,M,off", [(1, 1, 32, 128, 3000, 0), (1, 1, 32, 128, 3000, 2999),
                                           (1, 512, 32, 128, 3000, 2700), (2, 5, 3, 64, 7, 4),
                                           (1, 9, 16, 64, 9, 0), (3, 4, 2, 6, 5, 3),
                                           (1, 3000, 2, 64, 3000, 1)])
def test_cache_write_bit_exact(gpu, B, S, H, D, M, off):
    inp = oracle.normal(B * S + off, (B, S, H, D))
    init = oracle.normal(99, (B, H, M, D))
    ref = init.copy()
    oracle.cache_write(inp, ref, off, M)
    cache = dev(init)
    sts_attn.gpu_cache_write_v(dev(inp), cache, off, M)
    np.testing.assert_array_equal(host(cache), ref)


def test_kv_cache_ring_buffer_with_data(gpu):
    """model.rs:1459-1495 with values: max_len 4, 2 heads; entry i holds i+1."""
    c = sts_attn.KVCache(4, 2, 64)
    for i in range(5):
        k = torch.full((1, 1, 2, 64), float(i + 1), device="cuda")
        c.update(k, -k)
        s = c.state()
        assert s.len == min(i + 1, 4) and s.offset == i + 1
    kb, vb = c.read_buffers()
    kb, vb = host(kb), host(vb)
    # slots: 0 <- 5 (wrapped), 1 <- 2, 2 <- 3, 3 <- 4
    np.testing.assert_array_equal(kb[0, :, :, 0], [[5, 2, 3, 4]] * 2)
    np.testing.assert_array_equal(vb, -kb)
    assert c.window() == (1, 4)


def test_kv_cache_reset_and_keep_buffers(gpu):
    """model.rs:1497-1530: reset drops the buffers; reset_keep_buffers zero-fills."""
    c = sts_attn.KVCache(4, 2, 64)
    c.update(torch.ones((1, 1, 2, 64), device="cuda"), torch.ones((1, 1, 2, 64), device="cuda"))
    c.reset_keep_buffers()
    s = c.state()
    assert (s.len, s.offset, s.allocated) == (0, 0, 1)
    kb, vb = c.read_buffers()
    assert not host(kb).any() and not host(vb).any()
    c.reset()
    assert c.state().allocated == 0


def test_update_sequence_matches_oracle_with_rollbacks(gpu):
    """Random chunk appends and rollbacks on a wrapping ring: buffers bit-exact,
    counters equal to the oracle's, attention over the window within 1e-4."""
    H, D, M = 4, 128, 37
    rng = np.random.default_rng(3)
    c = sts_attn.KVCache(M, H, D)
    o = oracle.KvCounters(M)
    kref = np.zeros((1, H, M, D), np.float32)
    vref = np.zeros((1, H, M, D), np.float32)
    for it in range(60):
        if rng.random() < 0.25 and o.len > 0:
            n = int(rng.integers(1, o.len + 1))
            c.rollback(n)
            o.rollback(n)
        else:
            S = int(rng.integers(1, 12))
            k = oracle.normal(500 + it, (1, S, H, D))
            v = oracle.normal(900 + it, (1, S, H, D))
            oracle.cache_write(k, kref, o.offset % M, M)
            oracle.cache_write(v, vref, o.offset % M, M)
            o.advance(S)
            c.update(dev(k), dev(v))
        s = c.state()
        assert (s.offset, s.len, s.write_pos) == (o.offset, o.len, o.write_pos)
        kb, vb = c.read_buffers()
        np.testing.assert_array_equal(host(kb), kref)
        np.testing.assert_array_equal(host(vb), vref)
        if o.len == 0:
            continue
        q = oracle.normal(7000 + it, (1, H, D))
        got = host(c.attend(dev(q), scale_for(D)))[0]
        ref = oracle.attention_ring_f64(q[0], kref[0], vref[0], o.window_start(), o.len,
                                        scale_for(D))
        assert np.abs(got - ref).max() < 1e-4


@pytest.mark.parametrize("B", [1, 3])
def test_decode_step_equals_append_then_attend(gpu, B):
    """kv_decode_step (one launch) == update + attend (two launches), bit for bit,
    over 90 steps of a 40-slot ring (wraps twice), with a rollback midway."""
    H, D, M = 8, 128, 40
    fused = sts_attn.KVCache(M, H, D)
    plain = sts_attn.KVCache(M, H, D)
    o = oracle.KvCounters(M)
    kref = np.zeros((B, H, M, D), np.float32)
    vref = np.zeros((B, H, M, D), np.float32)
    for step in range(90):
        if step == 50:
            fused.rollback(17)
            plain.rollback(17)
            o.rollback(17)
        q = oracle.normal(10 * step + 1, (B, H, D))
        k = oracle.normal(10 * step + 2, (B, H, D))
        v = oracle.normal(10 * step + 3, (B, H, D))
        a = host(fused.decode_step(dev(q), dev(k), dev(v), scale_for(D)))
        plain.update(dev(k)[:, None], dev(v)[:, None])
        b = host(plain.attend(dev(q), scale_for(D)))
        np.testing.assert_array_equal(a, b)
        oracle.cache_write(k[:, None], kref, o.offset % M, M)
        oracle.cache_write(v[:, None], vref, o.offset % M, M)
        o.advance(1)
        if step % 9 == 0:
            for bb in range(B):
                ref = oracle.attention_ring_f64(q[bb], kref[bb], vref[bb], o.window_start(), o.len,
                                                scale_for(D))
                assert np.abs(a[bb] - ref).max() < 1e-4
    kb, vb = fused.read_buffers()
    np.testing.assert_array_equal(host(kb), kref)
    np.testing.assert_array_equal(host(vb), vref)


def test_decode_step_with_fused_rope(gpu):
    """The temporal decode branch (model.rs:818-831): RoPE of q and k at position
    offset, append, attend.  Cache rows must equal oracle RoPE output bit for bit."""
    H, D, M, T = 32, 128, 64, 70
    rope = sts_attn.RoPE(D, 3000)
    tabs = oracle.rope_tables(D, 3000)
    c = sts_attn.KVCache(M, H, D)
    kref = np.zeros((1, H, M, D), np.float32)
    vref = np.zeros((1, H, M, D), np.float32)
    o = oracle.KvCounters(M)
    for step in range(T):
        q = oracle.normal(3 * step + 100, (1, 1, H, D))
        k = oracle.normal(3 * step + 101, (1, 1, H, D))
        v = oracle.normal(3 * step + 102, (1, 1, H, D))
        got = host(c.decode_step(dev(q[:, 0]), dev(k[:, 0]), dev(v[:, 0]), scale_for(D), rope=rope))
        qr = oracle.rope_apply(q, o.offset, tabs)
        kr = oracle.rope_apply(k, o.offset, tabs)
        oracle.cache_write(kr, kref, o.offset % M, M)
        oracle.cache_write(v, vref, o.offset % M, M)
        o.advance(1)
        ref = oracle.attention_ring_f64(qr[0, 0], kref[0], vref[0], o.window_start(), o.len,
                                        scale_for(D))
        assert np.abs(got[0] - ref).max() < 1e-4, step
    kb, vb = c.read_buffers()
    np.testing.assert_array_equal(host(kb), kref)
    np.testing.assert_array_equal(host(vb), vref)


def test_rope_apply_bit_exact(gpu):
    D = 128
    rope = sts_attn.RoPE(D, 3000)
    tabs = oracle.rope_tables(D, 3000)
    for offset, S in ((0, 1), (2999, 1), (256, 512), (17, 3)):
        x = oracle.normal(offset + S, (2, S, 32, D))
        got = host(rope.apply_(dev(x), offset))
        np.testing.assert_array_equal(got, oracle.rope_apply(x, offset, tabs))
    with pytest.raises(sts_attn.StsError):
        rope.apply_(dev(oracle.normal(1, (1, 2, 32, D))), 2999)


def test_rope_tables_match_oracle(gpu):
    """sts_rope_create's tables, read through a rotation of unit vectors."""
    D, P = 64, 3000
    rope = sts_attn.RoPE(D, P)
    c, s = oracle.rope_tables(D, P)
    x = np.zeros((1, P, 1, D), np.float32)
    x[..., 0::2] = 1.0
    got = host(rope.apply_(dev(x), 0))
    np.testing.assert_array_equal(got[0, :, 0, 0::2], c)
    np.testing.assert_array_equal(got[0, :, 0, 1::2], s)
