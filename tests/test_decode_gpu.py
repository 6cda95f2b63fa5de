"""Decode attention on the GPU against the oracle: the plumbing case (32 x 128,
L = 256), the temporal decode (32 x 128, a wrapped 3000-row ring), the
depformer steps (16 x 64, L = 1..8, 64 streams) and ragged multi-stream decode.

Tolerance: f32 outputs within 1e-4 max-abs of the oracle (shader order and
double closed form), the north star's f32 bar.  L = 1 and repeated runs are
checked bit for bit.
"""
import os

import numpy as np
import pytest
import torch

import oracle
import sts_attn
from cases import decode_inputs, scale_for
from conftest import GOLDEN

pytestmark = pytest.mark.gpu

TOL = 1e-4


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def load_fixture(name):
    return np.load(os.path.join(GOLDEN, f"{name}.npz"))


def decode_fixture_inputs(f):
    return decode_inputs(int(f["seed"]), int(f["H"]), int(f["D"]), int(f["M"]), int(f["L"]),
                         int(f["start"]), bool(int(f["rope"])))


def test_fused_attention_config1_golden(gpu):
    """The plumbing case (1 layer, 32 x 128, L = 256) through the drop-in
    fused_attention entry point."""
    f = load_fixture("decode_config1")
    q, kc, vc = decode_fixture_inputs(f)
    H, M, D = kc.shape
    out = sts_attn.fused_attention(dev(q)[None, None], dev(kc)[None], dev(vc)[None],
                                   float(f["scale"]))
    got = host(out)[0, :, 0, :]
    assert np.abs(got - f["out_wgsl"]).max() < TOL
    assert np.abs(got - f["out_f64"]).max() < TOL


def test_fused_attention_reads_a_cache_view(gpu):
    """k, v as the reference passes them: [1, H, L, D] views of a [1, H, max_len, D]
    cache (kv_head_stride = max_len * D, model.rs:618-623); rows >= L are poison."""
    H, D, M, L = 32, 128, 3000, 777
    q, kc, vc = decode_inputs(11, H, D, M, L, 0)
    kc[:, L:] = np.nan
    vc[:, L:] = np.nan
    kd, vd = dev(kc)[None], dev(vc)[None]
    out = sts_attn.fused_attention(dev(q)[None, None], kd[:, :, :L], vd[:, :, :L], scale_for(D))
    got = host(out)[0, :, 0, :]
    ref = oracle.attention_ring_f64(q, np.nan_to_num(kc), np.nan_to_num(vc), 0, L, scale_for(D))
    assert np.isfinite(got).all()
    assert np.abs(got - ref).max() < TOL


@pytest.mark.parametrize("name", ["decode_wrap_d64", "decode_wrap_d128", "decode_len1",
                                  "decode_long", "depformer_step5"])
def test_decode_ring_fixtures(gpu, name):
    f = load_fixture(name)
    q, kc, vc = decode_fixture_inputs(f)
    H, M, D = kc.shape
    lens = torch.tensor([int(f["L"])], dtype=torch.int32, device="cuda")
    starts = torch.tensor([int(f["start"])], dtype=torch.int32, device="cuda")
    out = sts_attn.decode_ring(dev(q)[None], dev(kc)[None], dev(vc)[None], lens, starts,
                               float(f["scale"]))
    got = host(out)[0]
    assert np.abs(got - f["out_wgsl"]).max() < TOL
    assert np.abs(got - f["out_f64"]).max() < TOL
    if int(f["L"]) == 1:
        np.testing.assert_array_equal(got, vc[:, int(f["start"])])


@pytest.mark.parametrize("start", [0, 5, 15])
def test_single_row_is_exact(gpu, start):
    H, D, M = 32, 128, 16
    q, kc, vc = decode_inputs(21, H, D, M, 1, start)
    lens = torch.tensor([1], dtype=torch.int32, device="cuda")
    starts = torch.tensor([start], dtype=torch.int32, device="cuda")
    got = host(sts_attn.decode_ring(dev(q)[None], dev(kc)[None], dev(vc)[None], lens, starts,
                                    scale_for(D)))[0]
    np.testing.assert_array_equal(got, vc[:, start])


@pytest.mark.parametrize("D,L", [(128, 2), (128, 15), (128, 16), (128, 17), (128, 63),
                                 (128, 64), (128, 65), (128, 191), (128, 192), (128, 193),
                                 (64, 3), (64, 64), (64, 65), (64, 513), (128, 2999)])
def test_window_lengths_around_tile_edges(gpu, D, L):
    H, M = 4, 3000
    start = (37 * L) % M
    q, kc, vc = decode_inputs(1000 + L, H, D, M, L, start)
    lens = torch.tensor([L], dtype=torch.int32, device="cuda")
    starts = torch.tensor([start], dtype=torch.int32, device="cuda")
    got = host(sts_attn.decode_ring(dev(q)[None], dev(kc)[None], dev(vc)[None], lens, starts,
                                    scale_for(D)))[0]
    ref = oracle.attention_ring_f64(q, kc, vc, start, L, scale_for(D))
    assert np.abs(got - ref).max() < TOL


def test_config2_full_size_layers(gpu):
    """The temporal decode shape: 32 x 128, L = M = 3000, seeded write heads so the
    window wraps; three of the 24 layers checked against both oracles."""
    H, D, M = 32, 128, 3000
    rng = np.random.default_rng(2)
    for layer in range(3):
        start = int(rng.integers(0, M))
        q, kc, vc = decode_inputs(3000 + 10 * layer, H, D, M, M, start)
        lens = torch.tensor([M], dtype=torch.int32, device="cuda")
        starts = torch.tensor([start], dtype=torch.int32, device="cuda")
        got = host(sts_attn.decode_ring(dev(q)[None], dev(kc)[None], dev(vc)[None], lens, starts,
                                        scale_for(D)))[0]
        ref_w = oracle.attention_ring_wgsl(q, kc, vc, start, M, scale_for(D))
        ref_d = oracle.attention_ring_f64(q, kc, vc, start, M, scale_for(D))
        print(f"layer {layer} start {start}: max|gpu-wgsl| {np.abs(got - ref_w).max():.2e} "
              f"max|gpu-f64| {np.abs(got - ref_d).max():.2e}", flush=True)
        assert np.abs(got - ref_w).max() < TOL
        assert np.abs(got - ref_d).max() < TOL


def test_repeat_runs_are_bit_identical(gpu):
    """Split merging is order-fixed: two runs agree bit for bit (no LDS or
    counter races)."""
    H, D, M = 32, 128, 3000
    q, kc, vc = decode_inputs(77, H, D, M, M, 1234)
    args = (dev(q)[None], dev(kc)[None], dev(vc)[None],
            torch.tensor([M], dtype=torch.int32, device="cuda"),
            torch.tensor([1234], dtype=torch.int32, device="cuda"), scale_for(D))
    first = host(sts_attn.decode_ring(*args))
    for _ in range(20):
        np.testing.assert_array_equal(host(sts_attn.decode_ring(*args)), first)


def test_config5_ragged_streams(gpu):
    """Ragged multi-stream decode: 64 streams x 32 x 128, per-stream L ~ U[128, 3000] and a
    random ring start, plus edge streams (L = 0, 1, max_len; start = M - 1)."""
    B, H, D, M = 64, 32, 128, 3000
    rng = np.random.default_rng(5)
    lens = rng.integers(128, 3001, size=B).astype(np.int32)
    starts = rng.integers(0, M, size=B).astype(np.int32)
    lens[:4] = [0, 1, M, 2]
    starts[:4] = [7, M - 1, M - 1, M - 1]
    g = torch.Generator(device="cuda").manual_seed(5)
    kd = torch.randn((B, H, M, D), generator=g, device="cuda")
    vd = torch.randn((B, H, M, D), generator=g, device="cuda")
    qd = torch.randn((B, H, D), generator=g, device="cuda")
    out = sts_attn.decode_ring(qd, kd, vd, dev(lens), dev(starts), scale_for(D))
    got = host(out)
    q, kc, vc = host(qd), host(kd), host(vd)
    worst = 0.0
    for b in range(B):
        if lens[b] == 0:
            np.testing.assert_array_equal(got[b], 0.0)
            continue
        ref = oracle.attention_ring_f64(q[b], kc[b], vc[b], int(starts[b]), int(lens[b]),
                                        scale_for(D))
        worst = max(worst, float(np.abs(got[b] - ref).max()))
    print(f"ragged: worst max-abs {worst:.2e}", flush=True)
    assert worst < TOL


def test_config4_depformer_frame(gpu):
    """The depformer step attention: 6 layers x 8 steps, 64 streams, 16 x 64, M = 9, no RoPE.
    Each step appends at slot `step` from a packed qkv buffer and attends slots
    0..step; outputs and the appended cache rows are checked every step."""
    B, H, D, M, layers, steps = 64, 16, 64, 9, 6, 8
    scale = scale_for(D)
    for layer in range(layers):
        kc = torch.zeros((B, H, M, D), device="cuda")
        vc = torch.zeros((B, H, M, D), device="cuda")
        kc_ref = np.zeros((B, H, M, D), np.float32)
        vc_ref = np.zeros((B, H, M, D), np.float32)
        for step in range(steps):
            qkv = oracle.normal(40000 + 100 * layer + step, (B, 3, H, D))
            qkv_d = dev(qkv)
            out = sts_attn.depformer_step(qkv_d[:, 0], qkv_d[:, 1], qkv_d[:, 2], kc, vc, step,
                                          scale, qkv_stride=3 * H * D)
            for b in range(B):
                oracle.cache_write(qkv[b:b + 1, 1][:, None], kc_ref[b:b + 1], step, M)
                oracle.cache_write(qkv[b:b + 1, 2][:, None], vc_ref[b:b + 1], step, M)
            got = host(out)
            np.testing.assert_array_equal(host(kc), kc_ref)
            np.testing.assert_array_equal(host(vc), vc_ref)
            for b in range(0, B, 7):
                ref = oracle.attention_ring_f64(qkv[b, 0], kc_ref[b], vc_ref[b], 0, step + 1,
                                                scale)
                assert np.abs(got[b] - ref).max() < TOL, (layer, step, b)
            if step == 0:
                # L = 1: out is the appended V row exactly.
                np.testing.assert_array_equal(got, qkv[:, 2])
