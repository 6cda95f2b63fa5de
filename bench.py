"""Benchmark of the sts-web attention hot path on one MI355X.

Headline (the decode configuration, config 2): one temporal frame = 24 sequential layer
decode steps, each a fused RoPE + append + attention (sts_kv_decode_step)
over a 32-head x 128 f32 ring cache holding 3000 rows, with the write head at
a seeded offset so reads wrap.  Every layer has its own 98 MB cache (2.36 GB,
beyond the 256 MB MALL).  Inputs are resident in HBM before timing.

Also reported (extra fields): decode without the append (sts_kv_attend),
chunked prefill (config 3: 512 new rows after 256 cached, 32 x 128; f32,
bf16-MFMA and split-bf16 f32), depformer step attention (config 4: 6 layers x 8
steps, 64 streams, 16 x 64), ragged multi-stream decode (config 5: 64 streams,
windows of 128-3000 rows), the Q4_K projections around attention
(in_proj / out_proj per frame, FFN shapes), the whole depformer step chain for
64 streams (depth_engine.rs:884-1491); and the CPU baseline -- the oracle's
restatement of the reference shader, timed on this host's cores on a bounded
sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only decode]
Prints ONE JSON line.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "sts-web_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # dense bf16 MFMA
FP32_PEAK_TFLOPS = 157.3       # fp32 MFMA

LAYERS, H, D, M = 24, 32, 128, 3000
CALIB_BYTES = 256 << 20

# CPUs this process may run on (the CPU baseline pins one OpenMP thread to
# each of the first `threads` of them while it is timed).
try:
    ALLOWED_CPUS = sorted(os.sched_getaffinity(0))
except AttributeError:
    ALLOWED_CPUS = list(range(os.cpu_count() or 1))


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # 50 untimed steps: a fresh process's first kernels run slow for ~40-50
    # steps (measured on the prefill: 27.9, 20.3, 19.8, 19.4 -> 19.2 us per
    # layer over its first blocks of 10 steps), and a fresh allocation's
    # first touches cost one more slow step.
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--only", default="", help="comma list of sections to run")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a plain 256 MiB device copy (counter calibration)")
    return ap.parse_args()


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Timer:
    """HIP events on the stream the kernels are launched on."""

    def __init__(self, torch, stream):
        self.torch, self.stream = torch, stream

    def __enter__(self):
        self.torch.cuda.synchronize()
        self.a = self.torch.cuda.Event(enable_timing=True)
        self.b = self.torch.cuda.Event(enable_timing=True)
        self.a.record(self.stream)
        return self

    def __exit__(self, *exc):
        self.b.record(self.stream)
        self.torch.cuda.synchronize()
        self.ms = self.a.elapsed_time(self.b)


PLAIN_READ_GRIDS = (256, 512, 1024, 2048)


def time_plain_read(torch, sts, stream, pairs, workgroups, steps, warmup, graph=False):
    """us per launch of sts_probe_stream_read over `pairs` ((a_ptr, a_bytes,
    b_ptr, b_bytes), one launch each, in order), `workgroups` workgroups of
    256 threads: a plain 16-byte nontemporal read of the same bytes a kernel
    reads, the ceiling that kernel is compared with."""
    lib = sts.load()
    sink = torch.empty(max(PLAIN_READ_GRIDS), device="cuda")
    sp = stream.cuda_stream

    def run():
        for a, na, b, nb in pairs:
            rc = lib.sts_probe_stream_read(a, na, b, nb, workgroups, sink.data_ptr(), sp)
            if rc:
                raise RuntimeError(f"sts_probe_stream_read: {lib.sts_last_error().decode()}")
    f = run
    if graph:
        run()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            run()
        f = g.replay
    for _ in range(warmup):
        f()
    with Timer(torch, stream) as t:
        for _ in range(steps):
            f()
    return t.ms * 1e3 / (steps * len(pairs))


def plain_read_block(torch, sts, stream, pairs, same_grid, kernel_us, steps, warmup,
                     graph=False):
    """The plain read of a kernel's bytes on the kernel's own grid and on the
    fastest of PLAIN_READ_GRIDS, and the kernel's time as a fraction of each
    (plain-read time / kernel time: 1.0 = the kernel runs at the plain-read rate)."""
    grids = sorted(set(PLAIN_READ_GRIDS) | {same_grid})
    t = {wg: time_plain_read(torch, sts, stream, pairs, wg, steps, warmup, graph) for wg in grids}
    best = min(t, key=t.get)
    nbytes = sum(na + nb for _, na, _, nb in pairs) / len(pairs)
    return {"bytes_per_launch": int(nbytes),
            "us_per_launch": round(t[same_grid], 3), "workgroups": same_grid,
            "gbs": round(nbytes / (t[same_grid] * 1e-6) / 1e9, 1),
            "best_us_per_launch": round(t[best], 3), "best_workgroups": best,
            "best_gbs": round(nbytes / (t[best] * 1e-6) / 1e9, 1),
            "by_workgroups_us": {str(k): round(v, 3) for k, v in t.items()},
            "kernel_us_per_launch": round(kernel_us, 3),
            "kernel_frac_of_plain_read": round(t[same_grid] / kernel_us, 4),
            "kernel_frac_of_best_plain_read": round(t[best] / kernel_us, 4)}


def decode_grid(torch):
    """Workgroups of one config-2 decode launch: splits per head x heads, the
    splits chosen as the launcher does (about one workgroup per CU, chunks of
    whole 64-row units)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    want = max(1, -(-cus // H))
    chunk = -(-(-(-M // want)) // 64) * 64
    chunk = min(max(chunk, 64), 512 // 64 * 64)
    return -(-M // chunk) * H


def bench_decode(torch, sts, stream, steps, warmup):
    """Config 2: returns dict with per-frame and per-launch timings."""
    scale = sts.softmax_scale(D)
    g = torch.Generator(device="cuda").manual_seed(2)
    caches = []
    rows = torch.empty((1, M, H, D), device="cuda")
    for layer in range(LAYERS):
        c = sts.KVCache(M, H, D)
        # Seeded write head: advance the empty ring, then append 3000 rows
        # from there, so the window starts mid-buffer and reads wrap.
        c.advance((layer * 997 + 123) % M)
        rows.normal_(generator=g)
        krows = rows.clone()
        rows.normal_(generator=g)
        c.update(krows, rows, stream)
        assert c.seq_len() == M and c.window()[0] != 0
        caches.append(c)
    q = torch.randn((LAYERS, 1, H, D), generator=g, device="cuda")
    kn = torch.randn((LAYERS, 1, H, D), generator=g, device="cuda")
    vn = torch.randn((LAYERS, 1, H, D), generator=g, device="cuda")
    out = torch.empty((LAYERS, 1, H, D), device="cuda")
    # RoPE of q and k at each cache's offset (model.rs:824): the write heads sit
    # at offsets up to 2M, and every frame moves them by one.
    rope = sts.RoPE(D, 2 * M + warmup + steps + 64)

    def frame():
        for layer in range(LAYERS):
            caches[layer].decode_step(q[layer], kn[layer], vn[layer], scale, rope=rope,
                                      out=out[layer], stream=stream)

    def frame_attend():
        for layer in range(LAYERS):
            caches[layer].attend(q[layer], scale, out=out[layer], stream=stream)

    for _ in range(warmup):
        frame()
    with Timer(torch, stream) as t:
        for _ in range(steps):
            frame()
    for _ in range(2):
        frame_attend()
    with Timer(torch, stream) as ta:
        for _ in range(steps):
            frame_attend()
    bytes_layer = 2 * M * H * D * 4 + 2 * H * D * 4   # K/V reads + Q read + O write
    us_frame = t.ms * 1e3 / steps
    us_launch = us_frame / LAYERS
    us_attend = ta.ms * 1e3 / steps / LAYERS
    # The same K/V bytes of the same 24 caches read plainly, launch by launch.
    kv_bytes = H * M * D * 4
    pairs = []
    for c in caches:
        kp, vp, _ = c.ensure_allocated(1)
        pairs.append((kp, kv_bytes, vp, kv_bytes))
    plain = plain_read_block(torch, sts, stream, pairs, decode_grid(torch), us_launch, steps,
                             min(warmup, 5))
    return {
        "plain_read": plain,
        "us_per_frame": us_frame,
        "us_per_launch": us_launch,
        "bytes_per_launch": bytes_layer,
        "gbs": bytes_layer / (us_launch * 1e-6) / 1e9,
        "attend_only_us_per_launch": us_attend,
        "attend_only_gbs": bytes_layer / (us_attend * 1e-6) / 1e9,
        "caches": caches,
        "q": q,
    }


def bench_prefill(torch, sts, stream, steps, warmup):
    """Config 3: 512 new rows after 256 cached, 24 layers, f32 and bf16-MFMA."""
    cached, S = 256, 512
    L = cached + S
    scale = sts.softmax_scale(D)
    g = torch.Generator(device="cuda").manual_seed(3)
    kc = torch.randn((LAYERS, H, M, D), generator=g, device="cuda")
    vc = torch.randn((LAYERS, H, M, D), generator=g, device="cuda")
    q = torch.randn((LAYERS, S, H, D), generator=g, device="cuda")
    out = torch.empty_like(q)
    starts = [(2900 + 37 * i) % M for i in range(LAYERS)]
    pairs = S * cached + S * (S + 1) // 2
    flops_layer = 4 * H * D * pairs
    res = {"flops_per_layer": flops_layer}
    for name, prec in (("bf16", sts.PREC_BF16_MFMA), ("f32", sts.PREC_F32),
                       ("f32split", sts.PREC_F32_SPLIT_BF16)):
        def run():
            for layer in range(LAYERS):
                sts.prefill_attention(q[layer], kc[layer], vc[layer], starts[layer], L, scale,
                                      prec, out=out[layer], stream=stream)
        for _ in range(warmup):
            run()
        with Timer(torch, stream) as t:
            for _ in range(steps):
                run()
        us_layer = t.ms * 1e3 / steps / LAYERS
        res[name] = {"us_per_layer": us_layer,
                     "tflops": flops_layer / (us_layer * 1e-6) / 1e12}
    # bf16-MFMA over a bf16 mirror of the caches (what a KV handle created with
    # STS_KV_BF16_MIRROR keeps): same result as "bf16" bit for bit, half the
    # K/V bytes.
    k16 = kc.to(torch.bfloat16)
    v16 = vc.to(torch.bfloat16)

    def run16():
        for layer in range(LAYERS):
            sts.prefill_attention_bf16kv(q[layer], k16[layer], v16[layer], starts[layer], L, scale,
                                         out=out[layer], stream=stream)
    for _ in range(warmup):
        run16()
    with Timer(torch, stream) as t:
        for _ in range(steps):
            run16()
    us_layer = t.ms * 1e3 / steps / LAYERS
    res["bf16kv"] = {"us_per_layer": us_layer,
                     "tflops": flops_layer / (us_layer * 1e-6) / 1e12}
    # The f32-input bf16 kernel with fewer cached rows before the same 512
    # queries: the longest query tile then streams 8..11 key blocks instead
    # of 12 (all other tiles one to four fewer too).  How the layer time
    # follows the longest tile's blocks bounds what balancing the tiles could
    # gain at config 3 (8.5 blocks per tile on average).
    scan = {}
    for c in (0, 64, 128, 192):
        Lc = c + S

        def run_c():
            for layer in range(LAYERS):
                sts.prefill_attention(q[layer], kc[layer], vc[layer], starts[layer], Lc, scale,
                                      sts.PREC_BF16_MFMA, out=out[layer], stream=stream)
        for _ in range(min(warmup, 10)):
            run_c()
        with Timer(torch, stream) as t:
            for _ in range(steps):
                run_c()
        scan[(Lc + 63) // 64] = t.ms * 1e3 / steps / LAYERS
    scan[(L + 63) // 64] = res["bf16"]["us_per_layer"]
    res["bf16_scan"] = scan
    # Algorithmic HBM bytes per layer: K/V rows of the window (f32, or bf16
    # for the mirror), Q read and O written (f32).
    qo = 2 * S * H * D * 4
    res["bytes_f32kv"] = 2 * L * H * D * 4 + qo
    res["bytes_bf16kv"] = 2 * L * H * D * 2 + qo
    return res


def bench_depformer(torch, sts, stream, steps, warmup):
    """Config 4: 6 layers x 8 steps, 64 streams, 16 x 64, M = 9."""
    B, Hd, Dd, Md, layers, nsteps = 64, 16, 64, 9, 6, 8
    scale = sts.softmax_scale(Dd)
    g = torch.Generator(device="cuda").manual_seed(4)
    qkv = torch.randn((nsteps, layers, B, 3, Hd, Dd), generator=g, device="cuda")
    kc = torch.zeros((layers, B, Hd, Md, Dd), device="cuda")
    vc = torch.zeros((layers, B, Hd, Md, Dd), device="cuda")
    out = torch.empty((B, Hd, Dd), device="cuda")

    def frame():
        for step in range(nsteps):
            for layer in range(layers):
                x = qkv[step, layer]
                sts.depformer_step(x[:, 0], x[:, 1], x[:, 2], kc[layer], vc[layer], step, scale,
                                   out=out, qkv_stride=3 * Hd * Dd, stream=stream)

    for _ in range(warmup):
        frame()
    with Timer(torch, stream) as t:
        for _ in range(steps):
            frame()
    us_eager = t.ms * 1e3 / steps
    # The frame recorded once as a HIP graph (what a serving loop does): the
    # 48 launches replay without per-launch host cost.
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        frame()
    for _ in range(warmup):
        graph.replay()
    with Timer(torch, stream) as tg:
        for _ in range(steps):
            graph.replay()
    us_frame = tg.ms * 1e3 / steps
    kv_bytes = sum(2 * B * Hd * (s + 1) * Dd * 4 for s in range(nsteps)) * layers
    return {"us_per_frame": us_frame, "launches_per_frame": nsteps * layers,
            "us_per_launch": us_frame / (nsteps * layers),
            "eager_us_per_frame": us_eager,
            "kv_read_gbs": kv_bytes / (us_frame * 1e-6) / 1e9}


def bench_ragged(torch, sts, stream, steps, warmup):
    """Config 5: 64 streams x 32 x 128, L ~ U[128, 3000], wrapped starts; 24
    layers cycling over 2 cache slabs (12.6 GB, beyond the MALL)."""
    B = 64
    scale = sts.softmax_scale(D)
    g = torch.Generator(device="cuda").manual_seed(5)
    slabs = []
    for _ in range(2):
        kc = torch.randn((B, H, M, D), generator=g, device="cuda")
        vc = torch.randn((B, H, M, D), generator=g, device="cuda")
        slabs.append((kc, vc))
    lens = torch.randint(128, 3001, (LAYERS, B), generator=g, device="cuda", dtype=torch.int32)
    starts = torch.randint(0, M, (LAYERS, B), generator=g, device="cuda", dtype=torch.int32)
    q = torch.randn((B, H, D), generator=g, device="cuda")
    out = torch.empty((B, H, D), device="cuda")

    def frame():
        for layer in range(LAYERS):
            kc, vc = slabs[layer % 2]
            sts.decode_ring(q, kc, vc, lens[layer], starts[layer], scale, out=out, stream=stream)

    for _ in range(warmup):
        frame()
    with Timer(torch, stream) as t:
        for _ in range(steps):
            frame()
    total_rows = int(lens.sum().item())
    bytes_frame = total_rows * H * D * 4 * 2 + LAYERS * 2 * B * H * D * 4
    us_frame = t.ms * 1e3 / steps
    return {"us_per_frame": us_frame, "us_per_layer": us_frame / LAYERS,
            "gbs": bytes_frame / (us_frame * 1e-6) / 1e9,
            "mean_len": total_rows / (LAYERS * B)}


def q4k_random(torch, g, n, k):
    """Random Q4_K blocks on the device: quant and scale bytes uniform, d and
    dmin finite positive halves in [2^-14, 2^-4)."""
    nb = n * k // 256
    raw = torch.randint(0, 256, (nb, 144), generator=g, device="cuda", dtype=torch.uint8)
    half = torch.randint(0x0400, 0x2C00, (nb, 2), generator=g, device="cuda", dtype=torch.int32)
    for i in range(2):
        raw[:, 2 * i] = (half[:, i] & 0xFF).to(torch.uint8)
        raw[:, 2 * i + 1] = (half[:, i] >> 8).to(torch.uint8)
    return raw.reshape(-1)


def bench_q4k(torch, sts, stream, steps, warmup):
    """The Q4_K projections on either side of attention, batch 1: per temporal
    frame 24 layers x (in_proj [12288, 4096] + out_proj [4096, 4096] with the
    residual), each layer with its own weights (905 MB, beyond the MALL),
    launched eagerly and replayed from a HIP graph; plus single-launch rates of
    the FFN shapes linear_in [22528, 4096] and linear_out [4096, 11264]
    (four weight sets each, 32 launches per graph replay)."""
    g = torch.Generator(device="cuda").manual_seed(6)
    K = 4096
    layers = [(sts.Q4KTensor(q4k_random(torch, g, 3 * K, K), (3 * K, K)),
               sts.Q4KTensor(q4k_random(torch, g, K, K), (K, K))) for _ in range(LAYERS)]
    x = torch.randn((1, 1, K), generator=g, device="cuda")
    qkv = torch.empty((1, 1, 3 * K), device="cuda")
    y = torch.empty((1, 1, K), device="cuda")

    def frame():
        for wi, wo in layers:
            sts.q4k_matmul(x, wi, out=qkv, stream=stream)
            sts.q4k_matmul(x, wo, residual=x, out=y, stream=stream)

    for _ in range(warmup):
        frame()
    with Timer(torch, stream) as te:
        for _ in range(steps):
            frame()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        frame()
    for _ in range(warmup):
        graph.replay()
    with Timer(torch, stream) as tg:
        for _ in range(steps):
            graph.replay()
    w_bytes = LAYERS * 4 * K * K // 256 * 144
    io_bytes = LAYERS * 4 * (K + 3 * K + K + K + K)  # x twice, qkv, residual, y
    us = tg.ms * 1e3 / steps
    res = {"us_per_frame": us, "eager_us_per_frame": te.ms * 1e3 / steps,
           "weight_bytes_per_frame": w_bytes,
           "gbs": (w_bytes + io_bytes) / (us * 1e-6) / 1e9}
    res["frac"] = res["gbs"] / HBM_PEAK_GBS
    res["_layers"] = layers
    # Per-launch figures of each projection alone (graph of its 24 launches),
    # beside a plain read of the same weight bytes (the kernels' grid is 512
    # workgroups of 256 threads at these shapes).
    for name, idx, n in (("in_proj", 0, 3 * K), ("out_proj", 1, K)):
        ws = [lw[idx] for lw in layers]
        yo = qkv if idx == 0 else y

        def proj():
            for w in ws:
                sts.q4k_matmul(x, w, residual=None if idx == 0 else x, out=yo, stream=stream)
        proj()
        gp = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gp, stream=stream):
            proj()
        for _ in range(warmup):
            gp.replay()
        with Timer(torch, stream) as tp:
            for _ in range(steps):
                gp.replay()
        us_l = tp.ms * 1e3 / (steps * LAYERS)
        nbytes = n * K // 256 * 144
        res[name + "_us_per_launch"] = us_l
        res[name + "_plain_read"] = plain_read_block(
            torch, sts, stream, [(w.raw.data_ptr(), nbytes, 0, 0) for w in ws], 512, us_l, steps,
            min(warmup, 5), graph=True)
        del gp
    for name, (n, k) in (("linear_in", (22528, K)), ("linear_out", (K, 11264))):
        ws = [sts.Q4KTensor(q4k_random(torch, g, n, k), (n, k)) for _ in range(4)]
        xi = torch.randn((1, 1, k), generator=g, device="cuda")
        yo = torch.empty((1, 1, n), device="cuda")
        for w in ws:
            sts.q4k_matmul(xi, w, out=yo, stream=stream)
        # Replayed from a graph of 32 launches: an eager Python-side launch,
        # or a graph of only a few, costs more than these kernels take.
        reps = 8
        gl = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gl, stream=stream):
            for _ in range(reps):
                for w in ws:
                    sts.q4k_matmul(xi, w, out=yo, stream=stream)
        for _ in range(warmup):
            gl.replay()
        with Timer(torch, stream) as t:
            for _ in range(steps):
                gl.replay()
        us_l = t.ms * 1e3 / (steps * reps * len(ws))
        res[name + "_us_per_launch"] = us_l
        res[name + "_gbs"] = n * k // 256 * 144 / (us_l * 1e-6) / 1e9
        del gl, ws
    return res


DEPF_STREAMS = 64


def q4k_random_scaled(torch, g, n, k):
    """Random Q4_K bytes with d = 1/(200 sqrt k) and dmin = 7.5 d, so weights
    have mean ~0 and standard deviation ~1/sqrt(k) (activations stay O(1)
    through the depformer's layers)."""
    import numpy as np
    nb = n * k // 256
    raw = torch.randint(0, 256, (nb, 144), generator=g, device="cuda", dtype=torch.uint8)
    d = np.float16(1.0 / (200.0 * np.sqrt(k)))
    for off, v in ((0, d), (2, np.float16(7.5 * float(d)))):
        bits = int(np.array(v, np.float16).view(np.uint16))
        raw[:, off] = bits & 0xFF
        raw[:, off + 1] = bits >> 8
    return raw.reshape(-1)


def q4_0_random(torch, g, vocab, dim):
    """Random Q4_0 table: nibbles uniform, f16 scales in ~[0.008, 0.06)."""
    nb = vocab * dim // 32
    raw = torch.randint(0, 256, (nb, 18), generator=g, device="cuda", dtype=torch.uint8)
    half = torch.randint(0x2000, 0x2C00, (nb,), generator=g, device="cuda", dtype=torch.int32)
    raw[:, 0] = (half & 0xFF).to(torch.uint8)
    raw[:, 1] = (half >> 8).to(torch.uint8)
    return raw.reshape(-1)


def bench_depformer_frame(torch, sts, stream, steps, warmup):
    """The whole depformer step chain (depth_engine.rs:884-1491) at the
    PersonaPlex shapes for 64 streams: 8 steps x 6 layers with per-step Q4_K
    weights (375 MB), replayed from a HIP graph."""
    cfg = sts.DepformerConfig.personaplex()
    S, L, D, F, V, T = (cfg.num_steps, cfg.num_layers, cfg.dim, cfg.ffn, cfg.out_vocab,
                        cfg.temporal_dim)
    B = DEPF_STREAMS
    g = torch.Generator(device="cuda").manual_seed(8)
    mat = lambda n, k: q4k_random_scaled(torch, g, n, k)
    w = {"input_proj": [mat(D, T) for _ in range(S)],
         "attn_in_proj": [mat(3 * D, D) for _ in range(L * S)],
         "attn_out_proj": [mat(D, D) for _ in range(L * S)],
         "ffn_linear_in": [mat(2 * F, D) for _ in range(L * S)],
         "ffn_linear_out": [mat(D, F) for _ in range(L * S)],
         "norm1_alpha": [1 + 0.1 * torch.randn(D, generator=g, device="cuda") for _ in range(L)],
         "norm2_alpha": [1 + 0.1 * torch.randn(D, generator=g, device="cuda") for _ in range(L)],
         "output_linear": [mat(V, D) for _ in range(S)],
         "text_emb": q4_0_random(torch, g, cfg.text_emb_vocab, D),
         "audio_emb": [q4_0_random(torch, g, cfg.audio_emb_vocab, D)
                       for _ in range(cfg.num_audio_emb)]}
    eng = sts.DepthEngine(cfg, w, max_batch=B)
    th = torch.randn((B, T), generator=g, device="cuda")
    text = torch.randint(0, cfg.text_emb_vocab, (B,), generator=g, device="cuda",
                         dtype=torch.int32)
    rand = torch.rand((B, S), generator=g, device="cuda")
    pt = torch.randint(0, V, (B, S, 30), generator=g, device="cuda", dtype=torch.int32)
    npn = torch.randint(0, 31, (B, S), generator=g, device="cuda", dtype=torch.int32)
    tokens = torch.empty((B, S), dtype=torch.int32, device="cuda")
    args = (th, text, 0.8, 250, 1.2, rand, pt, npn)

    def frame():
        eng.generate(*args, tokens=tokens, stream=stream)

    for _ in range(warmup):
        frame()
    with Timer(torch, stream) as te:
        for _ in range(steps):
            frame()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        frame()
    for _ in range(warmup):
        graph.replay()
    with Timer(torch, stream) as tg:
        for _ in range(steps):
            graph.replay()
    us = tg.ms * 1e3 / steps
    weights = S * (D * T + V * D) + L * S * (3 * D * D + D * D + 2 * F * D + D * F)
    flops = 2 * B * weights
    res = {"streams": B, "us_per_frame": us, "eager_us_per_frame": te.ms * 1e3 / steps,
           "tokens_per_s": B * S / (us * 1e-6),
           "launches_per_frame": 1 + S * (1 + 5 * L + 2),
           "gemm_flops_per_frame": flops, "gemm_tflops": flops / (us * 1e-6) / 1e12,
           "weight_bytes_per_frame": weights // 256 * 144}
    res["frac_of_fp32_peak"] = res["gemm_tflops"] / FP32_PEAK_TFLOPS
    res["_cpu"] = (cfg, w, args)
    return res


def cpu_info():
    """The host's CPU as this process sees it: model string, nproc, the CPUs the
    process may run on, and the threads the baseline uses -- all it may use,
    capped by OMP_NUM_THREADS when the environment sets it (the GPU box gives
    one GPU's jobs a 16-core share and sets OMP_NUM_THREADS to that)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    nproc = os.cpu_count() or 1
    allowed = len(ALLOWED_CPUS)
    env = os.environ.get("OMP_NUM_THREADS", "")
    threads = min(allowed, int(env)) if env.isdigit() and int(env) > 0 else allowed
    return {"cpu_model": model, "nproc": nproc, "affinity": allowed, "threads": threads,
            "omp_num_threads_env": env or None,
            "pinned_cpus": ALLOWED_CPUS[:threads]}


def _times_us(fn, reps):
    """Wall time of `reps` calls of fn (after the caller's warm-up): min,
    median and max in microseconds."""
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t0) * 1e6)
    ts.sort()
    return {"min_us": ts[0], "median_us": ts[len(ts) // 2], "max_us": ts[-1], "reps": reps}


class _Pinned:
    """OpenMP thread t of the oracle's `threads`-thread regions runs on
    ALLOWED_CPUS[t] inside the block; afterwards the threads may run anywhere
    again."""

    def __init__(self, oracle, threads):
        self.oracle, self.cpus = oracle, ALLOWED_CPUS[:threads]

    def __enter__(self):
        self.failed = self.oracle.bind_threads(self.cpus, True)
        return self

    def __exit__(self, *exc):
        self.oracle.bind_threads(ALLOWED_CPUS, False)
        self.oracle.set_num_threads(len(self.cpus))


def _baseline(all_threads, one_thread, info, sample, one_thread_scale=1):
    """The cpu_baseline block: `value` is the median on all allowed threads;
    the spread and the one-thread figures ride along."""
    one = {k: (v * one_thread_scale if k.endswith("_us") else v) for k, v in one_thread.items()}
    return {"value": all_threads["median_us"], "unit": "us/frame", "cores": info["threads"],
            "kind": "port", **all_threads, "one_thread_us": one["median_us"],
            "one_thread": one, **info, "sample": sample}


def cpu_baseline_depformer_frame(torch, cfg, w, args):
    """The oracle's restatement of the chain (every op in its shader's f32
    order, OpenMP inside each op) for the benchmarked frame: all 64 streams on
    the allowed threads; one thread on stream 0, scaled to 64 streams."""
    import numpy as np
    sys.path.insert(0, ROOT)
    import oracle
    info = cpu_info()
    c = {f: getattr(cfg, f) for f, _ in cfg._fields_}
    host = {f: [t.cpu().numpy() for t in w[f]] for f in oracle.DepformerWeights.FIELDS}
    ow = oracle.DepformerWeights(c, text_emb=w["text_emb"].cpu().numpy(), **host)
    th, text, temp, top_k, pen, rand, pt, npn = args
    th, text, rand = th.cpu().numpy(), text.cpu().numpy(), rand.cpu().numpy()
    pt, npn = pt.cpu().numpy().view(np.uint32), npn.cpu().numpy().view(np.uint32)

    def stream(b):
        oracle.depformer_generate(ow, th[b], int(text[b]), top_k, temp, pen, rand[b], pt[b],
                                  npn[b])
    with _Pinned(oracle, info["threads"]):
        stream(0)
        allt = _times_us(lambda: [stream(b) for b in range(DEPF_STREAMS)], 5)
    with _Pinned(oracle, 1):
        one = _times_us(lambda: stream(0), 5)
    return _baseline(allt, one, info,
                     f"all {DEPF_STREAMS} streams of the benchmarked frame, one after another "
                     f"(OpenMP inside each op), 5 repetitions; the 1-thread figures run stream 0 "
                     f"and scale x{DEPF_STREAMS}", one_thread_scale=DEPF_STREAMS)


def cpu_baseline_q4k(torch, layers):
    """The oracle's restatement of shader_q4k_matvec.wgsl (OpenMP over output
    rows): the whole frame, in_proj + out_proj of all 24 layers, on the allowed
    threads (median of 3) and on one thread."""
    import numpy as np
    sys.path.insert(0, ROOT)
    import oracle
    info = cpu_info()
    x = np.ascontiguousarray(np.random.default_rng(0).standard_normal((1, 4096)), np.float32)
    ws = [(wi.raw.cpu().numpy(), wo.raw.cpu().numpy()) for wi, wo in layers]

    def frame():
        for wi, wo in ws:
            oracle.q4k_matvec_wgsl(wi, x, 3 * 4096)
            oracle.q4k_matvec_wgsl(wo, x, 4096)
    with _Pinned(oracle, info["threads"]):
        frame()
        allt = _times_us(frame, 7)
    with _Pinned(oracle, 1):
        one = _times_us(frame, 5)
    return _baseline(allt, one, info,
                     f"the whole frame: in_proj + out_proj of all {LAYERS} layers (x0 of one "
                     f"frame), oracle shader-order f32 Q4_K matvec; 7 repetitions on all "
                     f"threads, 5 on one")


def cpu_baseline(torch, dec):
    """The oracle's restatement of shader_attention.wgsl (f32, the shader's lane
    and tree order), for the whole benchmarked decode frame: 24 layers x 32
    heads x 3000 rows, parallel over (layer, head) on the allowed threads
    (median of 5 after a warm-up) and on one thread (median of 3)."""
    import numpy as np
    sys.path.insert(0, ROOT)
    import oracle
    info = cpu_info()
    scale = float(np.float32(D) ** np.float32(-0.5))
    qs, kcs, vcs, starts, lens = [], [], [], [], []
    for layer in range(LAYERS):
        c = dec["caches"][layer]
        kb, vb = c.read_buffers()
        st, ln = c.window()
        kcs.append(np.ascontiguousarray(kb[0].cpu().numpy()))
        vcs.append(np.ascontiguousarray(vb[0].cpu().numpy()))
        qs.append(np.ascontiguousarray(dec["q"][layer, 0].cpu().numpy()))
        starts.append(st)
        lens.append(ln)
        del kb, vb

    def frame():
        oracle.decode_frame_wgsl(qs, kcs, vcs, starts, lens, scale)
    with _Pinned(oracle, info["threads"]):
        frame()
        frame()
        allt = _times_us(frame, 9)
    with _Pinned(oracle, 1):
        one = _times_us(frame, 5)
    return _baseline(allt, one, info,
                     f"the whole frame: {LAYERS} layers x {H} heads x {M} rows (the benchmarked "
                     f"caches and queries, attention only), oracle shader-order f32 attention, "
                     f"OpenMP over (layer, head); 9 repetitions on all threads, 5 on one")


def load_traffic():
    """HBM bytes per decode launch from the committed rocprofv3 --pmc summary."""
    path = os.path.join(ROOT, "profiles", "decode_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported here "
              f"(the attention path would shard by head or by stream, one GPU each; "
              f"this build runs on a single GPU)", file=sys.stderr)
        sys.exit(2)
    import torch
    import sts_attn as sts
    sts.load()
    if not torch.cuda.is_available():
        sys.exit("bench.py needs a GPU")
    only = set(filter(None, args.only.split(",")))
    want = (lambda s: not only or s in only)
    stream = torch.cuda.Stream()
    extra = {}
    with torch.cuda.stream(stream):
        if args.calib_copy:
            # A copy of known size: 256 MiB read + 256 MiB written, used to scale
            # the FETCH_SIZE / WRITE_SIZE counters of the kernels below.
            src = torch.ones(CALIB_BYTES // 4, device="cuda")
            dst = torch.empty_like(src)
            for _ in range(3):
                dst.copy_(src)
            torch.cuda.synchronize()
            del src, dst
        log("bench: decode (config 2)")
        dec = bench_decode(torch, sts, stream, args.steps, args.warmup)
        if want("prefill"):
            log("bench: prefill (config 3)")
            extra["prefill"] = bench_prefill(torch, sts, stream, args.steps, args.warmup)
        if want("depformer"):
            log("bench: depformer (config 4)")
            extra["depformer"] = bench_depformer(torch, sts, stream, args.steps, args.warmup)
        if want("ragged"):
            log("bench: ragged (config 5)")
            # Fewer steps for the long frames (12.9 ms ragged, 2.6 ms depformer);
            # at most 10 warm-up frames, past the start-up ramp.
            extra["ragged"] = bench_ragged(torch, sts, stream, max(2, args.steps // 4),
                                           min(args.warmup, 10))
        if want("q4k"):
            log("bench: q4k projections")
            extra["q4k"] = bench_q4k(torch, sts, stream, args.steps, args.warmup)
        if want("depformer_frame"):
            log("bench: depformer frame (64 streams)")
            extra["depformer_frame"] = bench_depformer_frame(torch, sts, stream,
                                                             max(3, args.steps // 2),
                                                             min(args.warmup, 10))
    cpu = None
    if not args.no_cpu:
        log("bench: cpu baseline")
        cpu = cpu_baseline(torch, dec)
    achieved = dec["gbs"]
    line = {
        "metric": "decode attn us/frame (24L, KV 3000) + achieved HBM GB/s; prefill TFLOP/s",
        "value": round(dec["us_per_frame"], 2),
        "unit": "us/frame",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["us_per_frame"] / 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (torch.randn, seeded), inputs resident in HBM",
        "config": {"workload": "temporal decode frame: 24 layers x fused RoPE+append+attention, "
                               "32 heads x 128, f32 ring KV cache of 3000 rows (wrapped), batch 1",
                   "layers": LAYERS, "heads": H, "head_dim": D, "kv_len": M},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic(),
                     "kernel": "decode_kernel<128,4>",
                     "bytes_per_launch": dec["bytes_per_launch"],
                     "us_per_launch": round(dec["us_per_launch"], 3),
                     # A plain read of the same K/V bytes, same grid, same caches.
                     "plain_read_us_per_launch": dec["plain_read"]["us_per_launch"],
                     "kernel_frac_of_plain_read": dec["plain_read"]["kernel_frac_of_plain_read"]},
        "plain_read": dec["plain_read"],
        "cpu_baseline": cpu,
        "decode_attend_only": {"us_per_launch": round(dec["attend_only_us_per_launch"], 3),
                               "gbs": round(dec["attend_only_gbs"], 1)},
    }
    if "prefill" in extra:
        p = extra["prefill"]
        line["prefill"] = {
            "flops_per_layer": p["flops_per_layer"],
            "bf16_us_per_layer": round(p["bf16"]["us_per_layer"], 3),
            "bf16_tflops": round(p["bf16"]["tflops"], 1),
            "bf16_frac_of_mfma_peak": round(p["bf16"]["tflops"] / BF16_PEAK_TFLOPS, 4),
            "f32_us_per_layer": round(p["f32"]["us_per_layer"], 3),
            "f32_tflops": round(p["f32"]["tflops"], 1),
            "f32_frac_of_fp32_peak": round(p["f32"]["tflops"] / FP32_PEAK_TFLOPS, 4),
            # f32-grade results for moderate score ranges from three bf16 MFMA
            # products per f32 product: priced against the bf16 peak at three products per flop.
            "f32split_us_per_layer": round(p["f32split"]["us_per_layer"], 3),
            "f32split_tflops": round(p["f32split"]["tflops"], 1),
            "f32split_frac_of_mfma_peak": round(3 * p["f32split"]["tflops"] / BF16_PEAK_TFLOPS, 4),
            # HBM roof of each variant: its algorithmic bytes at 8 TB/s.
            "bf16_frac_of_hbm_roof": round(p["bytes_f32kv"] / (HBM_PEAK_GBS * 1e3)
                                           / p["bf16"]["us_per_layer"], 4),
            "bf16kv_us_per_layer": round(p["bf16kv"]["us_per_layer"], 3),
            "bf16kv_tflops": round(p["bf16kv"]["tflops"], 1),
            "bf16kv_frac_of_hbm_roof": round(p["bytes_bf16kv"] / (HBM_PEAK_GBS * 1e3)
                                             / p["bf16kv"]["us_per_layer"], 4),
            # us per layer of the f32-input bf16 kernel at 512 queries after
            # 0, 64, 128, 192 and 256 cached rows, keyed by the key blocks of
            # the longest query tile (8 .. 12; 12 is config 3).
            "bf16_us_by_longest_tile_blocks": {str(k): round(v, 3)
                                               for k, v in sorted(p["bf16_scan"].items())}}
    if "depformer" in extra:
        line["depformer"] = {k: round(v, 3) for k, v in extra["depformer"].items()}
    if "ragged" in extra:
        r = extra["ragged"]
        line["ragged"] = {k: round(v, 2) for k, v in r.items()}
        line["ragged"]["frac"] = round(r["gbs"] / HBM_PEAK_GBS, 4)
    if "q4k" in extra:
        q = extra["q4k"]
        layers_all = q.pop("_layers")
        line["q4k_projections"] = {k: (round(v, 4) if isinstance(v, float) else v)
                                   for k, v in q.items()}
        if not args.no_cpu:
            log("bench: cpu baseline (q4k)")
            cq = cpu_baseline_q4k(torch, layers_all)
            line["q4k_projections"]["cpu_baseline"] = cq
            line["q4k_projections"]["gpu_vs_cpu"] = round(cq["value"] / q["us_per_frame"], 1)
    if "depformer_frame" in extra:
        f = extra["depformer_frame"]
        cfg_w_args = f.pop("_cpu")
        line["depformer_frame"] = {k: (round(v, 4) if isinstance(v, float) else v)
                                   for k, v in f.items()}
        if not args.no_cpu:
            log("bench: cpu baseline (depformer frame)")
            cf = cpu_baseline_depformer_frame(torch, *cfg_w_args)
            line["depformer_frame"]["cpu_baseline"] = cf
            line["depformer_frame"]["gpu_vs_cpu"] = round(cf["value"] / f["us_per_frame"], 1)
    if cpu is not None:
        line["gpu_vs_cpu"] = round(cpu["value"] / dec["us_per_frame"], 1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
