"""Library-owned workspace and device error word.

- A HIP graph captured with split decodes keeps working after a larger eager
  launch on the same stream grows the workspace (the old buffers are retired,
  not freed): replays stay bit-identical to the eager result.
- A call that would allocate workspace while its stream is being captured is
  refused with STS_ERR_STATE instead of recording an allocation into the graph.
- The bf16 prefill kernels' bounded LDS waits report a give-up through the
  device error word: the test lowers the poll bound from the host so that the
  waits give up on purpose while every kernel still runs to its end.
"""
import ctypes

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


@pytest.fixture(scope="module")
def _stream_pool(gpu):
    """HIP streams created by this module, destroyed when it ends (not before,
    so that no two tests get the same stream handle)."""
    rt = ctypes.CDLL("libamdhip64.so.7")
    made = []
    yield rt, made
    torch.cuda.synchronize()
    for h in made:
        rt.hipStreamDestroy(h)


@pytest.fixture
def fresh_stream(_stream_pool):
    """A newly created HIP stream (default priority, non-blocking) wrapped for
    torch: the library has no workspace for it yet (torch's own streams come
    from a pool that earlier tests may have used)."""
    rt, made = _stream_pool
    h = ctypes.c_void_p()
    assert rt.hipStreamCreateWithFlags(ctypes.byref(h), ctypes.c_uint(1)) == 0
    made.append(h)
    s = torch.cuda.ExternalStream(h.value)
    yield s
    s.synchronize()


def test_graph_survives_workspace_growth(gpu, fresh_stream):
    H, D, M = 32, 128, 3000
    g = torch.Generator(device="cuda").manual_seed(11)
    kc = torch.randn((1, H, M, D), generator=g, device="cuda")
    vc = torch.randn((1, H, M, D), generator=g, device="cuda")
    q = torch.randn((1, H, D), generator=g, device="cuda")
    lens = torch.tensor([M], dtype=torch.int32, device="cuda")
    starts = torch.tensor([1234], dtype=torch.int32, device="cuda")
    out = torch.empty((1, H, D), device="cuda")
    s = fresh_stream
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        # Eager first: sizes this stream's workspace for the split decode.
        sts_attn.decode_ring(q, kc, vc, lens, starts, scale_for(D), out=out, stream=s)
        s.synchronize()
        want = host(out).copy()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            sts_attn.decode_ring(q, kc, vc, lens, starts, scale_for(D), out=out, stream=s)
        out.zero_()
        graph.replay()
        s.synchronize()
        np.testing.assert_array_equal(host(out), want)
        # An f32 prefill with split key ranges needs a far larger workspace on
        # the same stream: the graph's buffers are retired, not freed.
        qp = torch.randn((512, H, D), generator=g, device="cuda")
        pre = sts_attn.prefill_attention(qp, kc[0], vc[0], 2900, 768, scale_for(D),
                                         sts_attn.PREC_F32, stream=s)
        s.synchronize()
        for _ in range(3):
            out.zero_()
            graph.replay()
            s.synchronize()
            np.testing.assert_array_equal(host(out), want)
            # Eager calls on the grown workspace between the replays.
            pre2 = sts_attn.prefill_attention(qp, kc[0], vc[0], 2900, 768, scale_for(D),
                                              sts_attn.PREC_F32, stream=s)
            s.synchronize()
            np.testing.assert_array_equal(host(pre2), host(pre))
    ref = oracle.attention_ring_f64(host(q)[0], host(kc)[0], host(vc)[0], 1234, M, scale_for(D))
    assert np.abs(want[0] - ref).max() < 1e-4


def test_capture_refuses_workspace_allocation(gpu, fresh_stream):
    """A fresh stream's first split decode inside a capture needs workspace:
    STS_ERR_STATE, nothing recorded; the same call after an eager one captures."""
    H, D, M = 32, 128, 2048
    g = torch.Generator(device="cuda").manual_seed(12)
    kc = torch.randn((1, H, M, D), generator=g, device="cuda")
    vc = torch.randn((1, H, M, D), generator=g, device="cuda")
    q = torch.randn((1, H, D), generator=g, device="cuda")
    lens = torch.tensor([M], dtype=torch.int32, device="cuda")
    starts = torch.tensor([0], dtype=torch.int32, device="cuda")
    out = torch.empty((1, H, D), device="cuda")
    s = fresh_stream
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        graph = torch.cuda.CUDAGraph()
        with pytest.raises(sts_attn.StsError) as ei:
            with torch.cuda.graph(graph, stream=s):
                sts_attn.decode_ring(q, kc, vc, lens, starts, scale_for(D), out=out, stream=s)
        assert ei.value.code == sts_attn.STS_ERR_STATE
        assert "captured" in str(ei.value)
        sts_attn.decode_ring(q, kc, vc, lens, starts, scale_for(D), out=out, stream=s)
        s.synchronize()
        want = host(out).copy()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            sts_attn.decode_ring(q, kc, vc, lens, starts, scale_for(D), out=out, stream=s)
        out.zero_()
        graph.replay()
        s.synchronize()
        np.testing.assert_array_equal(host(out), want)


@pytest.mark.parametrize("prec", [sts_attn.PREC_BF16_MFMA, sts_attn.PREC_F32_SPLIT_BF16])
def test_bounded_wait_give_up_is_reported(gpu, prec):
    H, D, M, cached, S, start = 8, 128, 1000, 256, 512, 900
    q, kc, vc = prefill_inputs(21, H, D, M, cached, S, start)
    L = cached + S
    qd, kd, vd = dev(q), dev(kc), dev(vc)
    assert sts_attn.take_device_errors() == 0
    sts_attn.set_wait_limit(1)
    try:
        sts_attn.prefill_attention(qd, kd, vd, start, L, scale_for(D), prec)
        with pytest.raises(sts_attn.StsError) as ei:
            sts_attn.device_errors()
        assert ei.value.code == sts_attn.STS_ERR_DEVICE
    finally:
        sts_attn.set_wait_limit(0)
    # The word was cleared by the read; a normal launch raises nothing and is right.
    assert sts_attn.take_device_errors() == 0
    got = host(sts_attn.prefill_attention(qd, kd, vd, start, L, scale_for(D), prec))
    assert sts_attn.device_errors() == 0
    ref = oracle.prefill_f64(q, kc, vc, start, L, scale_for(D))
    tol = 2e-2 if prec == sts_attn.PREC_BF16_MFMA else 1e-4
    assert np.abs(got - ref).max() < tol



def test_capture_refused_prefill_leaves_cache_unchanged(gpu, fresh_stream):
    """An f32 chunk prefill with split key ranges (32 x 128, 512 rows) on a fresh
    stream needs workspace.  Inside a capture it is refused with STS_ERR_STATE
    before anything is appended or the counters move: the state and both
    buffers are those from before the call.  The same call then runs eagerly."""
    H, D, M = 32, 128, 3000
    s = fresh_stream
    g = torch.Generator(device="cuda").manual_seed(13)
    c = sts_attn.KVCache(M, H, D)
    c.update(torch.randn((1, 256, H, D), generator=g, device="cuda"),
             torch.randn((1, 256, H, D), generator=g, device="cuda"))
    torch.cuda.synchronize()
    before = c.state()
    k0, v0 = c.read_buffers()
    q, k, v = (torch.randn((512, H, D), generator=g, device="cuda") for _ in range(3))
    out = torch.zeros((512, H, D), device="cuda")
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        graph = torch.cuda.CUDAGraph()
        with pytest.raises(sts_attn.StsError) as ei:
            with torch.cuda.graph(graph, stream=s):
                c.prefill(q, k, v, scale_for(D), sts_attn.PREC_F32, out=out, stream=s)
        assert ei.value.code == sts_attn.STS_ERR_STATE
    torch.cuda.synchronize()
    after = c.state()
    for f in ("offset", "len", "write_pos", "batch"):
        assert getattr(after, f) == getattr(before, f), f
    k1, v1 = c.read_buffers()
    assert torch.equal(k1, k0) and torch.equal(v1, v0)
    # Eagerly on the same stream: appended and attended as usual.
    with torch.cuda.stream(s):
        got = c.prefill(q, k, v, scale_for(D), sts_attn.PREC_F32, out=out, stream=s)
    s.synchronize()
    assert c.offset() == before.offset + 512 and c.seq_len() == 768
    kc, vc = c.read_buffers()
    st, ln = c.window()
    ref = oracle.prefill_f64(host(q), host(kc)[0], host(vc)[0], st, ln, scale_for(D))
    assert np.abs(host(got) - ref).max() < 1e-4


def test_device_errors_refused_inside_capture(gpu, fresh_stream):
    """Reading the device error word needs the stream drained and the swap run
    now: inside a capture it is refused with STS_ERR_STATE (the capture stays
    valid), and the word reads normally afterwards."""
    s = fresh_stream
    x = torch.zeros(16, device="cuda")
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            x.add_(1.0)
            with pytest.raises(sts_attn.StsError) as ei:
                sts_attn.device_errors(stream=s)
            assert ei.value.code == sts_attn.STS_ERR_STATE
            assert "captured" in str(ei.value)
        graph.replay()
        graph.replay()
    s.synchronize()
    assert torch.equal(x, torch.full((16,), 2.0, device="cuda"))
    assert sts_attn.device_errors(stream=s) == 0
