"""Launches recorded into a HIP graph replay exactly like eager launches.

A serving loop records a depformer frame (48 step launches) or a temporal
frame once and replays it.  Each graph here is replayed several times with
unrelated eager work and synchronizations in between, and every replay is
compared bit for bit with the eager result of the same launches.  The
split-KV decode graph also exercises the in-kernel reset of the arrival
counters (nothing in the library records a memset).
"""
import numpy as np
import pytest
import torch

import sts_attn
from cases import scale_for

pytestmark = pytest.mark.gpu


def test_depformer_frame_graph_replays(gpu):
    B, H, D, M, layers, steps = 64, 16, 64, 9, 6, 8
    scale = scale_for(D)
    g = torch.Generator(device="cuda").manual_seed(11)
    qkv = torch.randn((steps, layers, B, 3, H, D), generator=g, device="cuda")
    kc = torch.zeros((layers, B, H, M, D), device="cuda")
    vc = torch.zeros((layers, B, H, M, D), device="cuda")
    outs = torch.empty((steps, layers, B, H, D), device="cuda")
    stream = torch.cuda.Stream()

    def frame():
        for step in range(steps):
            for layer in range(layers):
                x = qkv[step, layer]
                sts_attn.depformer_step(x[:, 0], x[:, 1], x[:, 2], kc[layer], vc[layer], step,
                                        scale, out=outs[step, layer], qkv_stride=3 * H * D,
                                        stream=stream)

    with torch.cuda.stream(stream):
        frame()
    torch.cuda.synchronize()
    eager = outs.clone()
    eager_k = kc.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        frame()
    for rep in range(4):
        outs.zero_()
        kc.zero_()
        vc.zero_()
        junk = torch.randn(1 << 20, device="cuda") * 2.0  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(outs, eager), rep
        assert torch.equal(kc, eager_k), rep
        del junk


def test_split_decode_graph_replays(gpu):
    """attend over a 3000-row wrapped window (8+ splits, last-arriver merge)."""
    H, D, M = 32, 128, 3000
    scale = scale_for(D)
    cache = sts_attn.KVCache(M, H, D)
    g = torch.Generator(device="cuda").manual_seed(12)
    cache.advance(1234)
    cache.update(torch.randn((1, M, H, D), generator=g, device="cuda"),
                 torch.randn((1, M, H, D), generator=g, device="cuda"))
    q = torch.randn((3, 1, H, D), generator=g, device="cuda")
    out = torch.empty((3, 1, H, D), device="cuda")
    stream = torch.cuda.Stream()

    def run():
        for i in range(3):
            cache.attend(q[i], scale, out=out[i], stream=stream)

    with torch.cuda.stream(stream):
        run()  # first call on this stream allocates the split workspace
    torch.cuda.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        run()
    for rep in range(5):
        out.zero_()
        with torch.cuda.stream(stream):
            cache.attend(q[rep % 3], scale, out=out[rep % 3], stream=stream)  # eager, same workspace
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out[rep % 3].cpu().numpy(), eager[rep % 3].cpu().numpy())
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep
