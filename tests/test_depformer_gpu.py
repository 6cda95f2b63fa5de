"""The depformer step chain on the GPU against the oracle.

RMSNorm and the embedding + add are bit-exact (same f32 operations in the
shader's order).  The Q4_K GEMM uses the shader's f32 weights bit for bit but
sums on the matrix cores, so it is held to the f32 rounding bound
1e-5 * sum_k (|w_k| + 2|dmin*min_k|) |x_k| against the f64 product and the
shader-order oracle; its SwiGLU variant to that bound carried through
silu(g) * v.  Sampling must pick the oracle's token wherever the draw is not
within 1e-5 of a cumulative boundary (exp differs in the last ulp between the
GPU and libm).  The whole chain (depth_engine.rs:884-1491) must reproduce the
oracle's tokens and its logits within 1e-4 of their scale, at a small shape
and at the PersonaPlex shape (lib.rs:136-143), eagerly and from a HIP graph.
"""
import numpy as np
import pytest
import torch

import oracle
import sts_attn
from test_oracle_depformer import CFG

pytestmark = pytest.mark.gpu


def dev(x, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(x))
    return t.to("cuda") if dtype is None else t.to(dtype).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def q4k_bound(blocks, x, N):
    K = x.shape[1]
    w = oracle.q4k_dequant(blocks, N, K).astype(np.float64)
    zq = blocks.reshape(-1, 144).copy()
    zq[:, 16:] = 0
    mins = -oracle.q4k_dequant(zq.reshape(-1), N, K).astype(np.float64)
    return np.abs(x.astype(np.float64)) @ (np.abs(w) + 2 * np.abs(mins)).T


@pytest.mark.parametrize("rows,D", [(5, 1024), (64, 1024), (3, 256), (2, 4096)])
def test_rmsnorm_bit_exact(gpu, rows, D):
    x = oracle.normal(rows + D, (rows, D)) * np.float32(2.5)
    alpha = (1 + 0.1 * oracle.normal(7, (D,))).astype(np.float32)
    got = host(sts_attn.rmsnorm(dev(x), dev(alpha), 1e-8))
    np.testing.assert_array_equal(got, oracle.rmsnorm_wgsl(x, alpha, 1e-8))


def test_embed_add_bit_exact(gpu):
    vocab, D, B = 2049, 1024, 7
    table = oracle.q4_0_random_table(3, vocab, D)
    proj = oracle.normal(4, (B, D))
    toks = np.array([0, 5, 2048, 2049, 77, 1000, 4000000000], np.uint32)  # two out of vocab
    got = host(sts_attn.embed_add_q4_0(dev(table), vocab, dev(toks.view(np.int32)), dev(proj)))
    want = np.stack([proj[b] + oracle.embed_q4_0(table, vocab, D, int(toks[b])) for b in range(B)])
    np.testing.assert_array_equal(got, want)
    # Strided tokens: column 2 of a [B, 4] token array.
    tk = np.zeros((B, 4), np.uint32)
    tk[:, 2] = toks
    got2 = host(sts_attn.embed_add_q4_0(dev(table), vocab, dev(tk.view(np.int32))[:, 2:], dev(proj),
                                        tok_stride=4))
    np.testing.assert_array_equal(got2, want)


@pytest.mark.parametrize("M,N,K,res", [(64, 3072, 1024, False), (64, 1024, 1024, True),
                                       (64, 1024, 2816, True), (64, 2048, 1024, False),
                                       (3, 1024, 4096, False), (17, 100, 512, True),
                                       (1, 16, 256, False), (130, 48, 768, False),
                                       (17, 300, 11264, True), (64, 1024, 8192, False),
                                       (40, 64, 4352, True)])
def test_q4k_gemm_against_oracle(gpu, M, N, K, res):
    print(f"q4k gemm M={M} N={N} K={K} res={res}", flush=True)
    blocks = oracle.q4k_random_blocks(M + N + K, N, K)
    x = oracle.normal(N * 3 + M, (M, K))
    r = oracle.normal(N * 5 + M, (M, N)) if res else None
    w = sts_attn.Q4KTensor.from_q4k_bytes(blocks, (N, K))
    got = host(sts_attn.q4k_gemm(dev(x), w, residual=dev(r) if res else None)).astype(np.float64)
    ref = oracle.q4k_matvec_f64(blocks, x, N) + (r.astype(np.float64) if res else 0)
    tol = 1e-5 * q4k_bound(blocks, x, N) + (1e-6 * np.abs(r) if res else 0)
    assert (np.abs(got - ref) <= tol).all(), np.abs(got - ref).max()
    refw = oracle.q4k_matvec_wgsl(blocks, x, N).astype(np.float64) + (r if res else 0)
    assert (np.abs(got - refw) <= 2 * tol).all()


@pytest.mark.parametrize("M,N,K,swiglu", [(64, 3072, 1024, False), (5, 5632, 1024, True),
                                          (3, 1024, 4096, False)])
def test_q4k_gemm_fused_rmsnorm(gpu, M, N, K, swiglu):
    """RMSNorm on the GEMM's input: against the shader-order RMSNorm followed
    by the f64 product (the normalised x differ in the last ulp at most)."""
    blocks = oracle.q4k_random_blocks(M * 3 + N + K, N, K)
    x = oracle.normal(M + 5, (M, K)) * np.float32(3.0)
    alpha = (1 + 0.1 * oracle.normal(K, (K,))).astype(np.float32)
    w = sts_attn.Q4KTensor.from_q4k_bytes(blocks, (N, K))
    got = host(sts_attn.q4k_gemm(dev(x), w, swiglu=swiglu, norm_alpha=dev(alpha),
                                 norm_eps=1e-8)).astype(np.float64)
    xn = oracle.rmsnorm_wgsl(x, alpha, 1e-8)
    y = oracle.q4k_matvec_f64(blocks, xn, N)
    b = 1e-5 * q4k_bound(blocks, xn, N)
    if swiglu:
        F = N // 2
        g, v = y[:, :F], y[:, F:]
        sig = 1 / (1 + np.exp(-g))
        want = g * sig * v
        # + 1e-30: silu underflows to 0 in f32 where g is very negative.
        tol = (np.abs(sig * (1 + g * (1 - sig))) * np.abs(v) * b[:, :F] + np.abs(g * sig) * b[:, F:]
               + 1e-6 * np.abs(want) + 1e-30)
    else:
        want, tol = y, b
    assert (np.abs(got - want) <= tol).all(), (np.abs(got - want) / tol).max()


def test_q4k_gemm_swiglu(gpu):
    M, F, K = 64, 2816, 1024
    blocks = oracle.q4k_random_blocks(31, 2 * F, K)
    x = oracle.normal(32, (M, K))
    w = sts_attn.Q4KTensor.from_q4k_bytes(blocks, (2 * F, K))
    got = host(sts_attn.q4k_gemm(dev(x), w, swiglu=True)).astype(np.float64)
    gv = oracle.q4k_matvec_f64(blocks, x, 2 * F)
    g, v = gv[:, :F], gv[:, F:]
    sig = 1 / (1 + np.exp(-g))
    want = g * sig * v
    b = 1e-5 * q4k_bound(blocks, x, 2 * F)
    dsilu = np.abs(sig * (1 + g * (1 - sig)))
    tol = dsilu * np.abs(v) * b[:, :F] + np.abs(g * sig) * b[:, F:] + 1e-6 * np.abs(want) + 1e-30
    assert (np.abs(got - want) <= tol).all(), (np.abs(got - want) / tol).max()
    np.testing.assert_allclose(got, oracle.swiglu(oracle.q4k_matvec_wgsl(blocks, x, 2 * F)),
                               rtol=1e-4, atol=1e-5 * np.abs(want).max())


def test_q4k_gemm_bit_repeatable_and_matmul_route(gpu):
    M, N, K = 64, 3072, 1024
    blocks = oracle.q4k_random_blocks(41, N, K)
    w = sts_attn.Q4KTensor.from_q4k_bytes(blocks, (N, K))
    x = dev(oracle.normal(42, (M, K)))
    first = host(sts_attn.q4k_gemm(x, w))
    for _ in range(3):
        np.testing.assert_array_equal(host(sts_attn.q4k_gemm(x, w)), first)
    # q4k_matmul with M > 1 (the reference's prefill route) is this GEMM.
    np.testing.assert_array_equal(host(sts_attn.q4k_matmul(x.reshape(2, 32, K), w)).reshape(M, N),
                                  first)


@pytest.mark.parametrize("V,K", [(2048, 250), (2048, 1), (2048, 20), (100, 150), (300, 2)])
def test_sample_topk_against_oracle(gpu, V, K):
    B = 16
    rng = np.random.default_rng(V * 7 + K)
    logits = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    rand = rng.random(B).astype(np.float32)
    pt = rng.integers(0, V + 3, size=(B, 30)).astype(np.uint32)
    pt[:, 5] = pt[:, 0]                                  # repeated tokens
    npn = rng.integers(0, 31, size=B).astype(np.uint32)
    got = host(sts_attn.sample_top_k(dev(logits), K, 0.8, 1.3, dev(rand), dev(pt.view(np.int32)),
                                     dev(npn.view(np.int32)))).view(np.uint32)
    for b in range(B):
        want, _ = oracle.sample_topk_wgsl(logits[b], K, 0.8, 1.3, float(rand[b]), pt[b, :npn[b]])
        assert got[b] == want, (b, got[b], want)


@pytest.mark.parametrize("V,K", [(2048, 250), (2048, 256), (2048, 20), (2048, 1), (300, 2),
                                 (100, 150), (4096, 250), (1, 2), (257, 256), (256, 256),
                                 (2049, 250)])
def test_sample_topk_ties(gpu, V, K):
    """Logits on a coarse grid, so values repeat and the k-th largest is
    tied: rows with every value equal, rows with two values, a row of -0 and
    +0 (equal as floats), rows on a 0.25 grid.  Every token equals the
    oracle's (the shader's selection by replacing the first minimum, its
    stable insertion sort and its running total; top_k = 1 its lane and tree
    argmax)."""
    B = 24
    rng = np.random.default_rng(V * 13 + K)
    logits = (np.round(rng.standard_normal((B, V)) * 4) / 4).astype(np.float32)
    logits[0:3] = np.float32(0.5)
    logits[3] = np.float32(-1.0)
    logits[3, 7::9] = np.float32(2.0)
    logits[4] = np.float32(1.0)
    logits[4, ::2] = np.float32(-2.0)
    logits[5] = np.float32(-0.0)                         # -0 and +0 tie
    logits[5, ::3] = np.float32(0.0)
    logits[5, min(10, V - 1)] = np.float32(1.0)
    rand = rng.random(B).astype(np.float32)
    rand[0] = np.float32(0.0)
    rand[1] = np.float32(0.999)
    pt = rng.integers(0, V, size=(B, 30)).astype(np.uint32)
    npn = rng.integers(0, 31, size=B).astype(np.uint32)
    npn[:6] = 0
    got = host(sts_attn.sample_top_k(dev(logits), K, 0.8, 1.3, dev(rand), dev(pt.view(np.int32)),
                                     dev(npn.view(np.int32)))).view(np.uint32)
    for b in range(B):
        want, _ = oracle.sample_topk_wgsl(logits[b], K, 0.8, 1.3, float(rand[b]), pt[b, :npn[b]])
        assert got[b] == want, (b, got[b], want)


@pytest.mark.parametrize("V,K,grid", [(2048, 250, False), (2048, 250, True), (2048, 20, False),
                                      (300, 256, True), (4096, 64, False), (100, 150, False)])
def test_sample_topk_boundary_draws(gpu, V, K, grid):
    """Draws placed on the shader's cumulative boundaries: rand equal to a
    running total (the shader moves past it: rand < total is false), one
    float below it, and at the last total (the default, the last slot).  The
    wave-scan totals differ from the shader's single-lane ones in the last
    bits, so these draws take the kernel's exact fallback; every token must
    equal the oracle's."""
    rng = np.random.default_rng(V + K + 7 * grid)
    base = rng.standard_normal(V) * 2
    if grid:
        base = np.round(base * 4) / 4  # tied values as well
    pt = rng.integers(0, V, size=30).astype(np.uint32)
    n_pen = 9
    _, _, cum = oracle.sample_topk_wgsl_detail(base.astype(np.float32), K, 0.8, 1.3, 0.5,
                                               pt[:n_pen])
    js = sorted(set(int(j) for j in rng.integers(0, K - 1, size=10)) | {0, K - 2})
    rands = []
    for j in js:
        c = np.float32(cum[j])
        rands += [c, np.nextafter(c, np.float32(-1)), np.nextafter(c, np.float32(2))]
    rands += [np.float32(cum[-1]), np.float32(np.nextafter(cum[-1], np.float32(-1)))]
    rands = np.array([r for r in rands if 0 <= r < 1], np.float32)
    B = rands.size
    logits = np.repeat(base.astype(np.float32)[None], B, axis=0)
    ptb = np.repeat(pt[None], B, axis=0)
    npn = np.full(B, n_pen, np.uint32)
    got = host(sts_attn.sample_top_k(dev(logits), K, 0.8, 1.3, dev(rands),
                                     dev(ptb.view(np.int32)),
                                     dev(npn.view(np.int32)))).view(np.uint32)
    for b in range(B):
        want, _ = oracle.sample_topk_wgsl(logits[b], K, 0.8, 1.3, float(rands[b]), pt[:n_pen])
        assert got[b] == want, (b, float(rands[b]), got[b], want)


@pytest.mark.parametrize("case", ["pair_in_top_k", "pair_at_kth"])
def test_sample_topk_rare_ties(gpu, case):
    """Distinct logits but one pair of equal values, as f32 logits of a real
    chain have now and then: the pair among the top K, or a logit left out
    equal to the K-th.  Draws land in the middle of the pair's ranks (the
    shader's selection and sort decide which index stands there) and of ranks
    elsewhere (any order of the pair gives the same token there); every token
    equals the oracle's."""
    V, K = 2048, 250
    rng = np.random.default_rng(11 if case == "pair_in_top_k" else 12)
    base = (rng.standard_normal(V) * 2).astype(np.float32)
    order = np.argsort(-base, kind="stable")
    if case == "pair_in_top_k":
        lo, hi = sorted(int(i) for i in order[[7, 31]])
        base[hi] = base[lo]          # equal values at two adjacent ranks
    else:
        kth, out = int(order[K - 1]), int(order[K + 9])
        base[out] = base[kth]        # a logit left out ties with the K-th
    _, idx, cum = oracle.sample_topk_wgsl_detail(base, K, 0.8, 1.0, 0.5)
    vals = base[idx] / np.float32(0.8)
    if case == "pair_in_top_k":
        tied = [r for r in range(K) if (r > 0 and vals[r - 1] == vals[r]) or
                (r + 1 < K and vals[r + 1] == vals[r])]
    else:
        tied = [r for r in range(K) if base[idx[r]] == base[out]]
    ranks = sorted(set(tied) | {0, 3, 100, K - 2, K - 1})
    # The shader's order at the tie is not index order (so the test tells a
    # replay from the index-ordered ranking): seeds and ranks chosen for it.
    assert tied and any(idx[r] > idx[r + 1] for r in tied[:-1]) or \
        (case == "pair_at_kth" and idx[K - 1] == out and out > kth)
    lows = np.concatenate([[0.0], cum[:-1]])
    rands = np.array([(lows[r] + cum[r]) / 2 for r in ranks], np.float32)
    B = rands.size
    logits = np.repeat(base[None], B, axis=0)
    pt = np.zeros((B, 30), np.int32)
    npn = np.zeros(B, np.int32)
    got = host(sts_attn.sample_top_k(dev(logits), K, 0.8, 1.0, dev(rands), dev(pt),
                                     dev(npn))).view(np.uint32)
    for b in range(B):
        want, _ = oracle.sample_topk_wgsl(base, K, 0.8, 1.0, float(rands[b]))
        assert got[b] == want, (case, ranks[b], got[b], want)


def _inputs(cfg, B, seed):
    S = cfg["num_steps"]
    th = oracle.normal(seed, (B, cfg["temporal_dim"]))
    rng = np.random.default_rng(seed)
    text = rng.integers(0, cfg["text_emb_vocab"], size=B).astype(np.uint32)
    rand = rng.random((B, S)).astype(np.float32)
    pt = rng.integers(0, cfg["out_vocab"], size=(B, S, 30)).astype(np.uint32)
    npn = rng.integers(0, 31, size=(B, S)).astype(np.uint32)
    return th, text, rand, pt, npn


def _device_weights(w):
    d = {f: [dev(a) for a in getattr(w, f)] for f in oracle.DepformerWeights.FIELDS}
    d["text_emb"] = dev(w.text_emb)
    return d


def _config(cfg):
    return sts_attn.DepformerConfig(**{f: cfg[f] for f, _ in sts_attn.DepformerConfig._fields_})


def _check_streams(cfg, w, th, text, rand, pt, npn, tokens, logits, top_k, temp, pen, streams):
    """Each stream's tokens and logits against the oracle run on that stream.
    Every step's token must be the oracle sampler's on the logits the chain
    produced (the sampler is exact); the logits must be within 1e-4 of the
    oracle chain's while the tokens so far agree with the oracle chain's (the
    GEMMs sum in another f32 order, so a draw within rounding of a boundary
    may go the other way, after which the streams legitimately part).
    Returns the number of steps that agreed with the oracle chain."""
    agree = 0
    for b in streams:
        otok, olog, _ = oracle.depformer_generate(w, th[b], int(text[b]), top_k, temp, pen,
                                                  rand[b], pt[b], npn[b])
        same = True
        for s in range(cfg["num_steps"]):
            want, _ = oracle.sample_topk_wgsl(logits[s, b], top_k, temp, pen, float(rand[b, s]),
                                              pt[b, s, :npn[b, s]])
            assert tokens[b, s] == want, (b, s, tokens[b, s], want)
            if same:
                np.testing.assert_allclose(logits[s, b], olog[s], rtol=0,
                                           atol=1e-4 * max(1.0, np.abs(olog[s]).max()))
                same = tokens[b, s] == otok[s]
                agree += int(same)
    return agree


def test_depformer_chain_small(gpu):
    w = oracle.DepformerWeights.synthetic(CFG, seed=3)
    B = 5
    th, text, rand, pt, npn = _inputs(CFG, B, 21)
    eng = sts_attn.DepthEngine(_config(CFG), _device_weights(w), max_batch=8)
    logits = torch.empty((CFG["num_steps"], B, CFG["out_vocab"]), device="cuda")
    tokens = eng.generate(dev(th), dev(text.view(np.int32)), 0.8, 20, 1.2, dev(rand),
                          dev(pt.view(np.int32)), dev(npn.view(np.int32)), logits=logits)
    tok = host(tokens).view(np.uint32)
    lg = host(logits)
    n = _check_streams(CFG, w, th, text, rand, pt, npn, tok, lg, 20, 0.8, 1.2, range(B))
    assert n >= B * CFG["num_steps"] - 2
    # Greedy (top_k = 1) and a second call on the same engine (caches restart).
    tok1 = eng.generate(dev(th), dev(text.view(np.int32)), 1.0, 1, 1.0, dev(rand),
                        dev(pt.view(np.int32)), dev(npn.view(np.int32)), logits=logits)
    n = _check_streams(CFG, w, th, text, rand, pt, npn, host(tok1).view(np.uint32), host(logits),
                       1, 1.0, 1.0, range(B))
    assert n >= B * CFG["num_steps"] - 2
    eng.close()


def test_depformer_chain_tied_logits(gpu):
    """Output rows duplicated in pairs, so every logit has an equal twin and
    each draw is decided by the replay of the shader's selection; the next
    step's input (the drawn token's embedding, added by the sampler) must
    still follow the oracle chain."""
    w = oracle.DepformerWeights.synthetic(CFG, seed=5)
    V = CFG["out_vocab"]
    for s, ol in enumerate(w.output_linear):
        a = np.array(ol).reshape(V, -1)
        a[1::2] = a[0::2]
        w.output_linear[s] = a.reshape(np.shape(ol))
    B = 4
    th, text, rand, pt, npn = _inputs(CFG, B, 23)
    eng = sts_attn.DepthEngine(_config(CFG), _device_weights(w), max_batch=B)
    logits = torch.empty((CFG["num_steps"], B, V), device="cuda")
    tokens = eng.generate(dev(th), dev(text.view(np.int32)), 0.8, 20, 1.2, dev(rand),
                          dev(pt.view(np.int32)), dev(npn.view(np.int32)), logits=logits)
    lg = host(logits)
    assert np.array_equal(lg[:, :, 0::2], lg[:, :, 1::2])
    n = _check_streams(CFG, w, th, text, rand, pt, npn, host(tokens).view(np.uint32), lg, 20,
                       0.8, 1.2, range(B))
    assert n >= B * CFG["num_steps"] - 2
    eng.close()


def test_depformer_chain_golden_fixture(gpu):
    """tests/golden/depformer_chain_small.npz: the GPU chain's tokens equal
    the fixture's and its logits are within 1e-4 of their scale."""
    import os
    from conftest import GOLDEN
    f = np.load(os.path.join(GOLDEN, "depformer_chain_small.npz"))
    w = oracle.DepformerWeights.synthetic(CFG, seed=int(f["wseed"]))
    th = oracle.normal(int(f["seed"]), (CFG["temporal_dim"],))[None]
    text = np.array([int(f["text_token"])], np.uint32)
    eng = sts_attn.DepthEngine(_config(CFG), _device_weights(w), max_batch=1)
    logits = torch.empty((CFG["num_steps"], 1, CFG["out_vocab"]), device="cuda")
    tok = eng.generate(dev(th), dev(text.view(np.int32)), float(f["temperature"]),
                       int(f["top_k"]), float(f["penalty"]), dev(f["rand"][None]),
                       dev(f["penalty_tokens"][None].view(np.int32)),
                       dev(f["num_penalty"][None].view(np.int32)), logits=logits)
    np.testing.assert_array_equal(host(tok).view(np.uint32)[0], f["tokens"])
    lg = host(logits)[:, 0]
    assert np.abs(lg - f["out_wgsl"]).max() <= 1e-4 * np.abs(f["out_wgsl"]).max()
    assert np.abs(lg - f["out_f64"]).max() <= 1e-4 * np.abs(f["out_f64"]).max()
    eng.close()


@pytest.mark.parametrize("top_k", [0, 200])
def test_depformer_chain_edge_cases(gpu, top_k):
    """3 steps with one audio table (steps 1 and 2 both read it), an
    out-of-vocab text token (zero embedding), penalty tokens past the vocab,
    greedy (top_k = 0) and top_k above the vocab; batch 2 of max 3."""
    cfg = dict(CFG, num_steps=3, num_audio_emb=1, kv_max_len=3)
    w = oracle.DepformerWeights.synthetic(cfg, seed=9)
    B = 2
    th, text, rand, pt, npn = _inputs(cfg, B, 5)
    text[0] = cfg["text_emb_vocab"] + 7
    pt[:, :, :4] = cfg["out_vocab"] + np.arange(4, dtype=np.uint32)
    npn[:] = 30
    eng = sts_attn.DepthEngine(_config(cfg), _device_weights(w), max_batch=3)
    logits = torch.empty((3, B, cfg["out_vocab"]), device="cuda")
    tok = eng.generate(dev(th), dev(text.view(np.int32)), 0.7, top_k, 0.9, dev(rand),
                       dev(pt.view(np.int32)), dev(npn.view(np.int32)), logits=logits)
    n = _check_streams(cfg, w, th, text, rand, pt, npn, host(tok).view(np.uint32), host(logits),
                       top_k, 0.7, 0.9, range(B))
    assert n >= B * 3 - 1
    eng.close()


@pytest.fixture(scope="module")
def full_model():
    cfg = {f: getattr(sts_attn.DepformerConfig.personaplex(), f)
           for f, _ in sts_attn.DepformerConfig._fields_}
    return cfg, oracle.DepformerWeights.synthetic(cfg, seed=5, quantize=False)


def test_depformer_chain_full_shape_and_graph(gpu, full_model):
    """PersonaPlex shapes, 64 streams; streams 0 and 63 checked against the
    oracle; a HIP-graph replay reproduces the eager tokens and logits bit
    for bit."""
    cfg, w = full_model
    B = 64
    th, text, rand, pt, npn = _inputs(cfg, B, 77)
    eng = sts_attn.DepthEngine(_config(cfg), _device_weights(w), max_batch=B)
    S, V = cfg["num_steps"], cfg["out_vocab"]
    args = (dev(th), dev(text.view(np.int32)), 0.8, 250, 1.2, dev(rand), dev(pt.view(np.int32)),
            dev(npn.view(np.int32)))
    logits = torch.empty((S, B, V), device="cuda")
    tokens = torch.empty((B, S), dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        eng.generate(*args, tokens=tokens, logits=logits, stream=s)
    tok = host(tokens).view(np.uint32)
    lg = host(logits)
    n = _check_streams(cfg, w, th, text, rand, pt, npn, tok, lg, 250, 0.8, 1.2, [0, B - 1])
    assert n >= 2 * S - 2
    g = torch.cuda.CUDAGraph()
    t2 = torch.empty_like(tokens)
    l2 = torch.empty_like(logits)
    with torch.cuda.graph(g, stream=s):
        eng.generate(*args, tokens=t2, logits=l2, stream=s)
    for _ in range(3):
        t2.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(t2), host(tokens))
        np.testing.assert_array_equal(host(l2), lg)
    eng.close()


def test_sample_topk_tie_known_answers(gpu):
    """The hand-worked shader cases (see the oracle's known-answer test):
    [0, 2, 2] with top_k 2 keeps slots [logit 2, logit 1] in that order, so
    rand 0.25 draws 2 and 0.75 draws 1 (lowest index first would give 1, 2);
    [1, 1, 2] keeps logit 1, not logit 0, and rand 0.99 draws it."""
    rows = np.array([[0, 2, 2], [0, 2, 2], [1, 1, 2]], np.float32)
    rand = np.array([0.25, 0.75, 0.99], np.float32)
    pt = np.zeros((3, 30), np.int32)
    npn = np.zeros(3, np.int32)
    got = host(sts_attn.sample_top_k(dev(rows), 2, 1.0, 1.0, dev(rand), dev(pt),
                                     dev(npn))).view(np.uint32)
    assert list(got) == [2, 1, 1]
