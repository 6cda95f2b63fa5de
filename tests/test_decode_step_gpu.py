"""The timed headline path at its own shape: sts_kv_decode_step at the temporal
decode shape (32 heads x 128, a full 3000-row ring whose window wraps), the
multi-split 4-wave kernel with its fused RoPE + append.

The decode branch of Q4Attention::forward_with_cache (model.rs:818-831):
RoPE of q and k at position `offset`, append of k and v at write_pos,
advance(1), attention over the new window.  Checked per step against
  - the same step as separate launches (cache update with the oracle's
    rotated k, then attend with the oracle's rotated q): bit for bit;
  - the f64 closed form and the shader-order oracle: within 1e-4 (f32 bar);
  - the whole K/V buffers against the oracle's RoPE + cache write: bit for bit
    (the appended row in its slot, every other slot untouched).
"""
import numpy as np
import pytest
import torch

import oracle
import sts_attn
from cases import scale_for

pytestmark = pytest.mark.gpu

TOL = 1e-4
ROPE_ROWS = 8192


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


@pytest.fixture(scope="module")
def ropes(gpu):
    return {d: (sts_attn.RoPE(d, ROPE_ROWS), oracle.rope_tables(d, ROPE_ROWS)) for d in (64, 128)}


@pytest.mark.parametrize("B,H,D,use_rope,prefix", [
    (1, 32, 128, True, 0),    # full ring: the append overwrites the oldest row
    (1, 32, 128, False, 0),
    (3, 32, 128, True, 0),
    (1, 32, 128, True, 1),    # 2999 rows before the step: the step fills the ring
    (1, 16, 64, True, 0),
    (3, 16, 64, False, 0),
])
def test_decode_step_config2_shape(gpu, ropes, B, H, D, use_rope, prefix):
    M = 3000
    seed = 1000 * B + D + 7 * use_rope + prefix
    shift = (seed * 997 + 123) % M           # seeded write head: the window wraps
    rope, tabs = ropes[D] if use_rope else (None, None)
    fused = sts_attn.KVCache(M, H, D)
    plain = sts_attn.KVCache(M, H, D)
    o = oracle.KvCounters(M)
    kref = np.zeros((B, H, M, D), np.float32)
    vref = np.zeros((B, H, M, D), np.float32)
    n0 = M - prefix
    # The ring's existing rows (already rotated: any data will do for them):
    # M rows after a seeded advance, then `prefix` of them rolled back.
    k0 = oracle.normal(seed + 1, (B, M, H, D))
    v0 = oracle.normal(seed + 2, (B, M, H, D))
    for c in (fused, plain):
        c.advance(shift)
        c.update(dev(k0), dev(v0))
        c.rollback(prefix)
    o.advance(shift)
    oracle.cache_write(k0, kref, o.offset % M, M)
    oracle.cache_write(v0, vref, o.offset % M, M)
    o.advance(M)
    o.rollback(prefix)
    del k0, v0
    assert fused.window()[0] != 0 and fused.seq_len() == n0
    for step in range(3):
        pos = o.offset
        q = oracle.normal(seed + 10 * step + 3, (B, 1, H, D))
        k = oracle.normal(seed + 10 * step + 4, (B, 1, H, D))
        v = oracle.normal(seed + 10 * step + 5, (B, 1, H, D))
        qr = oracle.rope_apply(q, pos, tabs) if use_rope else q
        kr = oracle.rope_apply(k, pos, tabs) if use_rope else k
        got = host(fused.decode_step(dev(q[:, 0]), dev(k[:, 0]), dev(v[:, 0]), scale_for(D),
                                     rope=rope))
        plain.update(dev(kr), dev(v))
        sep = host(plain.attend(dev(qr[:, 0]), scale_for(D)))
        np.testing.assert_array_equal(got, sep)
        slot = o.write_pos
        oracle.cache_write(kr, kref, o.offset % M, M)
        oracle.cache_write(v, vref, o.offset % M, M)
        o.advance(1)
        s = fused.state()
        assert (s.offset, s.len, s.write_pos) == (o.offset, o.len, o.write_pos)
        assert o.len == M
        for b in range(B):
            ref = oracle.attention_ring_f64(qr[b, 0], kref[b], vref[b], o.window_start(), o.len,
                                            scale_for(D))
            wg = oracle.attention_ring_wgsl(qr[b, 0], kref[b], vref[b], o.window_start(), o.len,
                                            scale_for(D))
            assert np.abs(got[b] - ref).max() < TOL, (step, b)
            assert np.abs(got[b] - wg).max() < TOL, (step, b)
        kb, vb = fused.read_buffers()
        kb, vb = host(kb), host(vb)
        # The appended row, RoPE'd, in its slot; then every slot.
        np.testing.assert_array_equal(kb[:, :, slot], kr[:, 0])
        np.testing.assert_array_equal(vb[:, :, slot], v[:, 0])
        np.testing.assert_array_equal(kb, kref)
        np.testing.assert_array_equal(vb, vref)
