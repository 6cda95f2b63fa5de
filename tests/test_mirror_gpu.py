"""The bf16 mirror of the KV cache and the bf16-input prefill.

The bf16-MFMA prefill rounds the f32 K/V rows to bf16 (nearest even) in its
producers.  A KV handle created with STS_KV_BF16_MIRROR keeps those rounded
values, written by every append made through the handle, and its bf16 prefill
reads them instead: half the K/V bytes, the same stages, so the result must be
bit-identical to the f32-input kernel's.  Checked here:
  - sts_prefill_attention_bf16kv over torch's bf16 rounding of the caches
    equals sts_prefill_attention(PREC_BF16_MFMA) bit for bit (512 new rows after
    256 cached, head_dim 64, ragged last tile, wrapped windows), and is within the bf16
    bar (2e-2) of the f64 oracle;
  - the mirror equals torch's bf16 rounding of the f32 caches, bit for bit,
    after chunk appends that wrap, fused decode steps with RoPE, prefills with
    RoPE, rollbacks, resets and sts_kv_sync_mirror;
  - a mirrored handle's prefill equals an unmirrored one's, bit for bit.
"""
import numpy as np
import pytest
import torch

import oracle
import sts_attn
from cases import prefill_inputs, scale_for

pytestmark = pytest.mark.gpu


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def bf16_bits(t):
    """torch's float32 -> bfloat16 rounding (nearest even), as int16 bits."""
    return t.to(torch.bfloat16).view(torch.int16)


@pytest.mark.parametrize("H,D,M,cached,S,start", [
    (32, 128, 3000, 256, 512, 2900),  # 512 new rows after 256 cached, wrapped window
    (4, 64, 300, 100, 130, 250),      # head_dim 64, ragged last q-tile, wraps
    (2, 128, 1000, 0, 65, 990),       # empty cache before the chunk
    (3, 64, 200, 17, 1, 190),         # single query
    (2, 128, 4096, 0, 2048, 4000),    # tiles of 1..32 blocks: start stagger at its cap
])
def test_bf16kv_prefill_equals_f32_input(gpu, H, D, M, cached, S, start):
    q, kc, vc = prefill_inputs(6000 + S, H, D, M, cached, S, start)
    L = cached + S
    qd, kd, vd = dev(q), dev(kc), dev(vc)
    want = host(sts_attn.prefill_attention(qd, kd, vd, start, L, scale_for(D),
                                           sts_attn.PREC_BF16_MFMA))
    got = host(sts_attn.prefill_attention_bf16kv(qd, bf16_bits(kd), bf16_bits(vd), start, L,
                                                 scale_for(D)))
    np.testing.assert_array_equal(got, want)
    ref = oracle.prefill_f64(q, kc, vc, start, L, scale_for(D))
    assert np.abs(got - ref).max() < 2e-2
    assert sts_attn.device_errors() == 0


def _check_mirror(c):
    kb, vb = c.read_buffers()
    k16, v16 = c.mirror_buffers()
    np.testing.assert_array_equal(host(k16), host(bf16_bits(kb)))
    np.testing.assert_array_equal(host(v16), host(bf16_bits(vb)))


@pytest.mark.parametrize("D", [64, 128])
def test_mirror_tracks_every_append(gpu, D):
    H, M = 4, 97
    rope = sts_attn.RoPE(D, 4096)
    c = sts_attn.KVCache(M, H, D, bf16_mirror=True)
    assert c.state().flags == sts_attn.KV_BF16_MIRROR
    assert c.mirror_buffers() == (None, None)
    rng = np.random.default_rng(D)
    for it in range(12):
        op = it % 4
        if op == 0:    # chunk append through update (wraps over the iterations)
            S = int(rng.integers(1, 40))
            c.update(dev(oracle.normal(100 + it, (1, S, H, D))),
                     dev(oracle.normal(200 + it, (1, S, H, D))))
        elif op == 1:  # fused decode steps with RoPE
            for j in range(3):
                x = [dev(oracle.normal(300 + 10 * it + 3 * j + t, (1, H, D))) for t in range(3)]
                c.decode_step(*x, scale_for(D), rope=rope)
        elif op == 2:  # prefill with RoPE, bf16 precision (reads the mirror)
            S = int(rng.integers(1, 30))
            x = [dev(oracle.normal(400 + it * 3 + t, (S, H, D))) for t in range(3)]
            c.prefill(*x, scale_for(D), sts_attn.PREC_BF16_MFMA, rope=rope)
        else:
            c.rollback(int(rng.integers(0, 10)))
        _check_mirror(c)
    c.reset_keep_buffers()
    k16, v16 = c.mirror_buffers()
    assert not host(k16).any() and not host(v16).any()
    # Rows written into the f32 buffers directly reach the mirror by a sync.
    kp, vp, _ = c.ensure_allocated(1)
    kb = sts_attn.copy_device(kp, (1, H, M, D))
    kb.copy_(torch.randn_like(kb))
    rt = sts_attn._hip()
    rt.hipMemcpy(kp, kb.data_ptr(), kb.numel() * 4, 3)
    c.sync_mirror()
    _check_mirror(c)
    c.reset()
    assert c.mirror_buffers() == (None, None)


def test_mirrored_prefill_equals_unmirrored(gpu):
    """A config-3-shaped chunk through two handles, one mirrored: outputs of every
    precision and the f32 caches bit-identical."""
    H, D, M = 32, 128, 3000
    rope = sts_attn.RoPE(D, 8192)
    a = sts_attn.KVCache(M, H, D, bf16_mirror=True)
    b = sts_attn.KVCache(M, H, D)
    g = torch.Generator(device="cuda").manual_seed(17)
    k0 = torch.randn((1, 256, H, D), generator=g, device="cuda")
    v0 = torch.randn((1, 256, H, D), generator=g, device="cuda")
    for c in (a, b):
        c.advance(2900)
        c.update(k0, v0)
    for prec in (sts_attn.PREC_BF16_MFMA, sts_attn.PREC_F32, sts_attn.PREC_BF16_MFMA):
        q, k, v = (torch.randn((512, H, D), generator=g, device="cuda") for _ in range(3))
        got = host(a.prefill(q, k, v, scale_for(D), prec, rope=rope))
        want = host(b.prefill(q, k, v, scale_for(D), prec, rope=rope))
        np.testing.assert_array_equal(got, want)
    ka, va = a.read_buffers()
    kb, vb = b.read_buffers()
    np.testing.assert_array_equal(host(ka), host(kb))
    np.testing.assert_array_equal(host(va), host(vb))
    _check_mirror(a)
    assert sts_attn.device_errors() == 0


def test_gqa_mirror_tracks_decode_steps(gpu):
    """Grouped-query attention (32 query heads over 8 K/V heads) on a mirrored
    cache: the appended row of a fused decode step is stored by the first query
    head of its group, into the f32 cache and the mirror.  After chunk appends
    and decode steps (B = 2, RoPE, a window that wraps) the mirror equals the
    f32 cache rounded to bf16, bit for bit, and the attention output equals the
    same steps on an unmirrored handle."""
    Hq, Hkv, D, M, B = 32, 8, 128, 1000, 2
    rope = sts_attn.RoPE(D, 8192)
    a = sts_attn.KVCache(M, Hkv, D, bf16_mirror=True, n_heads=Hq)
    b = sts_attn.KVCache(M, Hkv, D, n_heads=Hq)
    g = torch.Generator(device="cuda").manual_seed(23)
    k0 = torch.randn((B, 990, Hkv, D), generator=g, device="cuda")
    v0 = torch.randn((B, 990, Hkv, D), generator=g, device="cuda")
    for c in (a, b):
        c.advance(500)
        c.update(k0, v0)
    for step in range(24):  # crosses the ring's end at row 1000
        q = torch.randn((B, Hq, D), generator=g, device="cuda")
        k = torch.randn((B, Hkv, D), generator=g, device="cuda")
        v = torch.randn((B, Hkv, D), generator=g, device="cuda")
        got = host(a.decode_step(q, k, v, scale_for(D), rope=rope))
        want = host(b.decode_step(q, k, v, scale_for(D), rope=rope))
        np.testing.assert_array_equal(got, want)
        if step % 6 == 5:
            _check_mirror(a)
    _check_mirror(a)
    ka, va = a.read_buffers()
    kb, vb = b.read_buffers()
    np.testing.assert_array_equal(host(ka), host(kb))
    np.testing.assert_array_equal(host(va), host(vb))
