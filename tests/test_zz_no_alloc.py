"""sts_decode_ring_noalloc: sts_decode_ring without any allocation.

The variant keeps its split records and arrival counters in a static device
array of the library instead of the per-stream workspace.  Its results must
equal sts_decode_ring's bit for bit (same kernel, same launch plan), on
consecutive calls that reuse the array (the second one smaller), and be
within the f32 bar (1e-4) of the f64 oracle.  Launches needing more than the
array holds are refused before any device work.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
import sts_attn
from cases import scale_for

FAKE = 0x10000  # a 16-byte aligned non-null pointer; never dereferenced


def _run(fn, q, kc, vc, lens, starts, scale, out):
    B, H, M, D = kc.shape
    return fn(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(), lens.data_ptr(),
              starts.data_ptr(), B, H, D, M, scale, None)


@pytest.mark.gpu
def test_noalloc_equals_decode_ring(gpu):
    lib = sts_attn.load()
    g = torch.Generator(device="cuda").manual_seed(31)
    # Two calls in a row on the shared array, the second smaller; then the
    # first shape again (the counters left at zero by the calls before).
    for B, H, D, M in ((4, 32, 128, 3000), (1, 8, 64, 500), (4, 32, 128, 3000)):
        print(f"noalloc decode B={B} H={H} D={D} M={M}", flush=True)
        kc = torch.randn((B, H, M, D), generator=g, device="cuda")
        vc = torch.randn((B, H, M, D), generator=g, device="cuda")
        q = torch.randn((B, H, D), generator=g, device="cuda")
        lens = torch.randint(0, M + 1, (B,), generator=g, device="cuda", dtype=torch.int32)
        lens[0] = M
        if B > 2:
            lens[1] = 0
            lens[2] = 1
        starts = torch.randint(0, M, (B,), generator=g, device="cuda", dtype=torch.int32)
        scale = scale_for(D)
        want = torch.full((B, H, D), float("nan"), device="cuda")
        got = torch.full((B, H, D), float("nan"), device="cuda")
        assert _run(lib.sts_decode_ring, q, kc, vc, lens, starts, scale, want) == 0
        assert _run(lib.sts_decode_ring_noalloc, q, kc, vc, lens, starts, scale, got) == 0
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy(), want.cpu().numpy())
        # And the f32 bar against the f64 closed form for the longest stream.
        qh, kh, vh = q[0].cpu().numpy(), kc[0].cpu().numpy(), vc[0].cpu().numpy()
        ref = oracle.attention_ring_f64(qh, kh, vh, int(starts[0]), M, scale)
        assert np.abs(got[0].cpu().numpy() - ref).max() < 1e-4
        if B > 2:
            assert not got[1].cpu().numpy().any()


def test_noalloc_refuses_launches_beyond_the_array():
    """64 streams x 32 heads over 30000-row rings need 59 splits: 15.9 M floats of
    records, beyond the 2 M the array holds.  Refused before any device work
    (fake pointers, never dereferenced), with a message naming the limit."""
    lib = sts_attn.load()
    fn = lib.sts_decode_ring_noalloc
    rc = fn(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 64, 32, 128, 30000, 0.1, None)
    assert rc == sts_attn.STS_ERR_INVALID
    msg = lib.sts_last_error().decode()
    assert "static scratch" in msg and "sts_decode_ring" in msg
    # Argument checks are those of sts_decode_ring.
    assert fn(None, FAKE, FAKE, FAKE, FAKE, FAKE, 1, 32, 128, 3000, 0.1, None) == \
        sts_attn.STS_ERR_INVALID
    assert fn(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1, 32, 102, 3000, 0.1, None) == \
        sts_attn.STS_ERR_INVALID
    assert ctypes.c_int(fn(FAKE, FAKE, FAKE, FAKE + 4, FAKE, FAKE, 1, 32, 128, 3000, 0.1,
                           None)).value == sts_attn.STS_ERR_INVALID


@pytest.mark.gpu
def test_noalloc_replays_from_a_graph(gpu):
    """The entry is for callers that cannot allocate, e.g. code under HIP graph
    capture: a split decode (4 streams x 32 heads x 128 over 3000-row rings)
    captured on a side stream replays bit-identically to an eager
    sts_decode_ring, with eager calls of both entries between the replays."""
    lib = sts_attn.load()
    B, H, D, M = 4, 32, 128, 3000
    g = torch.Generator(device="cuda").manual_seed(37)
    kc = torch.randn((B, H, M, D), generator=g, device="cuda")
    vc = torch.randn((B, H, M, D), generator=g, device="cuda")
    q = torch.randn((B, H, D), generator=g, device="cuda")
    lens = torch.tensor([M, 2000, 129, 1], dtype=torch.int32, device="cuda")
    starts = torch.tensor([1234, 2999, 0, 7], dtype=torch.int32, device="cuda")
    scale = scale_for(D)
    want = torch.full((B, H, D), float("nan"), device="cuda")
    got = torch.full((B, H, D), float("nan"), device="cuda")
    side = torch.cuda.Stream()
    sp = ctypes.c_void_p(side.cuda_stream)

    def call(fn, out):
        return fn(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(), lens.data_ptr(),
                  starts.data_ptr(), B, H, D, M, scale, sp)

    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        assert call(lib.sts_decode_ring, want) == 0
        assert call(lib.sts_decode_ring_noalloc, got) == 0  # the device's array is set up
    side.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), want.cpu().numpy())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        assert call(lib.sts_decode_ring_noalloc, got) == 0
    other = torch.full((B, H, D), float("nan"), device="cuda")
    for rep in range(4):
        got.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy(), want.cpu().numpy())
        # Eager work on the shared array between replays (the counters it
        # leaves at zero are the ones the graph's launch uses).
        with torch.cuda.stream(side):
            assert call(lib.sts_decode_ring_noalloc, other) == 0
        side.synchronize()
        np.testing.assert_array_equal(other.cpu().numpy(), want.cpu().numpy())
