"""Pins for the oracle's depformer-chain functions (CPU only).

Each function is checked against something independent of its C code: numpy
float64 formulas, hand-built Q4_0 blocks whose values are known, a numpy
restatement of the sampling rules, and a float64 numpy restatement of the
whole step chain (depth_engine.rs:884-1491) fed the oracle's own tokens;
planted mistakes must fail those checks.
"""
import numpy as np
import pytest

import oracle

CFG = dict(num_steps=4, num_layers=2, dim=256, num_heads=4, ffn=512, temporal_dim=512,
           out_vocab=128, text_emb_vocab=300, audio_emb_vocab=129, num_audio_emb=3,
           kv_max_len=5, rms_eps=1e-8, attn_scale=0.125)


def _rms_f64(x, alpha, eps):
    x = x.astype(np.float64)
    return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps) * alpha.astype(np.float64)


def test_rmsnorm_against_f64():
    x = oracle.normal(1, (5, 1024)) * np.float32(3.0)
    alpha = 1 + 0.1 * oracle.normal(2, (1024,))
    got = oracle.rmsnorm_wgsl(x, alpha, 1e-8)
    np.testing.assert_allclose(got, _rms_f64(x, alpha, 1e-8), rtol=2e-6, atol=1e-7)


def test_rmsnorm_eps_inside_the_root():
    """Rows of size ~1e-5: mean(x^2) ~ 1e-10 << eps = 1e-6, so eps decides."""
    x = oracle.normal(3, (2, 512)) * np.float32(1e-5)
    alpha = np.ones(512, np.float32)
    got = oracle.rmsnorm_wgsl(x, alpha, 1e-6)
    np.testing.assert_allclose(got, _rms_f64(x, alpha, 1e-6), rtol=2e-6)
    wrong = x.astype(np.float64) / (np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True)) + 1e-6)
    assert np.abs(got - wrong).max() > 1e-3 * np.abs(got).max()


def test_swiglu_against_f64():
    gv = oracle.normal(4, (3, 2 * 700)) * np.float32(4.0)
    got = oracle.swiglu(gv)
    g, v = gv[:, :700].astype(np.float64), gv[:, 700:].astype(np.float64)
    want = g / (1 + np.exp(-g)) * v
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)
    swapped = v / (1 + np.exp(-v)) * g
    assert np.abs(got - swapped).max() > 0.1


def _q4_0_block(scale_bits, nibbles):
    b = np.zeros(18, np.uint8)
    b[0], b[1] = scale_bits & 0xFF, scale_bits >> 8
    for j in range(16):
        b[2 + j] = nibbles[j] | (nibbles[16 + j] << 4)
    return b


def test_embed_q4_0_hand_blocks():
    nib = [(5 * j + 3) % 16 for j in range(32)]
    blk = _q4_0_block(0x3C00, nib)                       # scale 1.0
    blk2 = _q4_0_block(0x3800, nib[::-1])                # scale 0.5
    table = np.concatenate([blk, blk2, blk2, blk])      # 2 rows of 64
    np.testing.assert_array_equal(oracle.embed_q4_0(table, 2, 64, 0),
                                  np.array(nib + [(n - 8) * 0.5 + 8 for n in nib[::-1]], np.float32) - 8)
    np.testing.assert_array_equal(oracle.embed_q4_0(table, 2, 64, 1)[32:], np.array(nib, np.float32) - 8)
    np.testing.assert_array_equal(oracle.embed_q4_0(table, 2, 64, 2), np.zeros(64, np.float32))
    inf = _q4_0_block(0x7C00, nib)                       # Inf scale reads as 0
    np.testing.assert_array_equal(oracle.embed_q4_0(inf, 1, 32, 0), np.zeros(32, np.float32))
    sub = _q4_0_block(0x0001, nib)                       # subnormal 2^-24, exact
    np.testing.assert_array_equal(oracle.embed_q4_0(sub, 1, 32, 0),
                                  (np.array(nib, np.float64) - 8).astype(np.float32) * np.float32(2.0 ** -24))


def _sample_np(logits, top_k, temp, penalty, rand, ptoks):
    """The sampling rules restated with numpy: returns (token, safe).  `safe`
    is False when a last-ulp difference in the logits or in exp could change
    the draw: rand within 1e-5 of a cumulative boundary, or the drawn value
    within 1e-4 (relative) of its neighbour in the sorted order (including the
    first value left out of the top k), whose order could then swap."""
    lg = np.array(logits, np.float32)
    for t in dict.fromkeys(int(t) for t in ptoks):
        if t < lg.size:
            lg[t] = lg[t] / np.float32(penalty) if lg[t] > 0 else lg[t] * np.float32(penalty)
    lg = lg / np.float32(temp)
    srt = np.argsort(-lg.astype(np.float64), kind="stable")
    vs = lg[srt].astype(np.float64)

    def near(i, j):
        return 0 <= j < vs.size and abs(vs[i] - vs[j]) <= 1e-4 * max(1.0, abs(vs[i]))

    if top_k <= 1:
        return int(srt[0]), not near(0, 1)
    k = min(top_k, lg.size)
    v = vs[:k]
    p = np.exp(v - v[0])
    cum = np.cumsum(p / p.sum())
    j = min(int(np.searchsorted(cum, rand, side="right")), top_k - 1)
    if j >= k:  # a padding entry of the shader (index 0)
        return 0, bool(np.min(np.abs(cum - rand)) > 1e-5)
    safe = np.min(np.abs(cum - rand)) > 1e-5 and not near(j, j - 1) and not near(j, j + 1)
    return int(srt[j]), bool(safe)


@pytest.mark.parametrize("V,K", [(2048, 250), (2048, 1), (128, 20), (100, 100), (300, 2)])
def test_sample_topk_against_numpy(V, K):
    rng = np.random.default_rng(V + K)
    checked = 0
    for trial in range(40):
        logits = (rng.standard_normal(V) * 2).astype(np.float32)
        ptoks = rng.integers(0, V + 5, size=int(rng.integers(0, 31)))
        if trial % 3 == 0 and ptoks.size:
            ptoks[-1] = ptoks[0]                         # a repeated token
        rand = float(np.float32(rng.random()))
        tok, lg = oracle.sample_topk_wgsl(logits, K, 0.8, 1.3, rand, ptoks)
        want, safe = _sample_np(logits, K, 0.8, 1.3, rand, ptoks)
        if safe:
            assert tok == want, (trial, tok, want)
            checked += 1
    assert checked >= 30


def test_sample_topk_penalty_once_and_temperature():
    logits = np.array([2.0, -1.0, 0.5, 3.0], np.float32)
    _, lg = oracle.sample_topk_wgsl(logits, 1, 2.0, 4.0, 0.5, [0, 1, 0, 7])
    np.testing.assert_array_equal(lg, np.array([2.0 / 4 / 2, -1.0 * 4 / 2, 0.25, 1.5], np.float32))
    tok, _ = oracle.sample_topk_wgsl(logits, 1, 2.0, 4.0, 0.5, [0, 1, 0, 7])
    assert tok == 3
    # Planted: multiplying by the temperature changes the draw.
    rng = np.random.default_rng(9)
    diff = 0
    for _ in range(30):
        lg0 = (rng.standard_normal(64) * 2).astype(np.float32)
        r = float(rng.random())
        a, _ = oracle.sample_topk_wgsl(lg0, 10, 0.3, 1.0, r)
        b, _ = oracle.sample_topk_wgsl(lg0 * np.float32(0.09), 10, 1.0, 1.0, r)  # t^2 instead of 1/t
        diff += a != b
    assert diff > 0


def test_sample_topk_k_above_vocab():
    logits = np.array([0.1, 0.7, 0.3], np.float32)
    tok, _ = oracle.sample_topk_wgsl(logits, 5, 1.0, 1.0, 0.0)
    assert tok == 1                                      # padding entries weigh exp(-huge) = 0
    tok, _ = oracle.sample_topk_wgsl(logits, 5, 1.0, 1.0, 0.99999994)
    assert tok in (0, 2)


def _chain_f64(w, th, text_token, tokens, drop_residual=False):
    """depth_engine.rs:884-1491 in float64 numpy, with the embedding inputs
    taken from `tokens` (the oracle's draws); returns logits [S][V]."""
    c = w.cfg
    S, L, D, F = c["num_steps"], c["num_layers"], c["dim"], c["ffn"]
    H = c["num_heads"]
    hd = D // H
    deq = lambda b, n, k: oracle.q4k_dequant(b, n, k).astype(np.float64)
    th = th.astype(np.float64)
    kc = np.zeros((L, H, S, hd))
    vc = np.zeros((L, H, S, hd))
    out = []
    for st in range(S):
        prev = text_token if st == 0 else int(tokens[st - 1])
        if st == 0:
            emb = oracle.embed_q4_0(w.text_emb, c["text_emb_vocab"], D, prev)
        else:
            e = min(st - 1, c["num_audio_emb"] - 1)
            emb = oracle.embed_q4_0(w.audio_emb[e], c["audio_emb_vocab"], D, prev)
        h = deq(w.input_proj[st], D, c["temporal_dim"]) @ th + emb
        for l in range(L):
            i = l * S + st
            x = _rms_f64(h[None], w.norm1_alpha[l], c["rms_eps"])[0]
            qkv = deq(w.attn_in_proj[i], 3 * D, D) @ x
            q, k, v = qkv[:D].reshape(H, hd), qkv[D:2 * D].reshape(H, hd), qkv[2 * D:].reshape(H, hd)
            kc[l, :, st], vc[l, :, st] = k, v
            s = np.einsum("hd,hpd->hp", q, kc[l, :, :st + 1]) * c["attn_scale"]
            p = np.exp(s - s.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            a = np.einsum("hp,hpd->hd", p, vc[l, :, :st + 1]).reshape(D)
            h = deq(w.attn_out_proj[i], D, D) @ a + (0 if drop_residual else h)
            x = _rms_f64(h[None], w.norm2_alpha[l], c["rms_eps"])[0]
            gv = deq(w.ffn_linear_in[i], 2 * F, D) @ x
            sw = gv[:F] / (1 + np.exp(-gv[:F])) * gv[F:]
            h = deq(w.ffn_linear_out[i], D, F) @ sw + h
        out.append(deq(w.output_linear[st], c["out_vocab"], D) @ h)
    return np.array(out)


@pytest.fixture(scope="module")
def small_model():
    return oracle.DepformerWeights.synthetic(CFG, seed=3)


def test_chain_against_f64_restatement(small_model):
    w = small_model
    th = oracle.normal(11, (CFG["temporal_dim"],))
    rand = [0.2, 0.7, 0.45, 0.05]
    pt = np.zeros((4, 30), np.uint32)
    pt[2, :3] = [5, 9, 5]
    tok, logits, hidden = oracle.depformer_generate(w, th, 17, 20, 0.8, 1.2, rand, pt, [0, 0, 3, 0])
    ref = _chain_f64(w, th, 17, tok)
    scale = np.abs(ref).max()
    np.testing.assert_allclose(logits, ref, rtol=0, atol=2e-5 * scale)
    # The draws follow the sampling rules on the oracle's own logits.
    for st in range(4):
        want, safe = _sample_np(logits[st], 20, 0.8, 1.2, rand[st], pt[st, :[0, 0, 3, 0][st]])
        if safe:
            assert tok[st] == want


def test_chain_planted_mistakes_are_caught(small_model):
    """Wrong embedding table for step 1 and a dropped residual must both move
    the logits far outside the tolerance of the f64 restatement."""
    w = small_model
    th = oracle.normal(12, (CFG["temporal_dim"],))
    tok, logits, _ = oracle.depformer_generate(w, th, 3, 1, 1.0, 1.0, [0.5] * 4,
                                               np.zeros((4, 30)), [0] * 4)
    ref = _chain_f64(w, th, 3, tok)
    tol = 2e-5 * np.abs(ref).max()
    assert np.abs(logits - ref).max() <= tol
    bad = oracle.DepformerWeights(CFG, **{f: getattr(w, f) for f in oracle.DepformerWeights.FIELDS},
                                  text_emb=w.text_emb)
    bad.audio_emb = [w.audio_emb[1], w.audio_emb[2], w.audio_emb[0]]  # step 1 reads table 1
    _, lb, _ = oracle.depformer_generate(bad, th, 3, 1, 1.0, 1.0, [0.5] * 4, np.zeros((4, 30)), [0] * 4)
    assert np.abs(lb[1] - ref[1]).max() > 100 * tol
    np.testing.assert_array_equal(lb[0], logits[0])   # step 0 does not read audio tables
    dropped = _chain_f64(w, th, 3, tok, drop_residual=True)
    assert np.abs(dropped - logits).max() > 100 * tol


def test_sampler_tie_known_answers():
    """The shader's tie behaviour, worked out by hand from
    shader_sample_topk.wgsl:134-196 (slots start with logits 0..K-1; a logit
    strictly above the minimum replaces the first slot holding it; the
    insertion sort is stable, so equal values keep slot order), where it
    differs from 'lowest index first':
      [0, 2, 2], K=2: slot 0 (value 0) takes logit 2 -> slots [2 (i2), 2 (i1)],
        sorted i2 then i1, each weight 1/2: rand 0.25 -> 2, rand 0.75 -> 1.
      [1, 1, 2], K=2: logit 2 replaces slot 0 -> [2 (i2), 1 (i1)]: logit 1 is
        kept, not logit 0; rand 0.99 -> 1.
    Temperature 1, no penalty."""
    lg = np.array([0, 2, 2], np.float32)
    assert oracle.sample_topk_wgsl(lg, 2, 1.0, 1.0, 0.25)[0] == 2
    assert oracle.sample_topk_wgsl(lg, 2, 1.0, 1.0, 0.75)[0] == 1
    tok, idx, cum = oracle.sample_topk_wgsl_detail(lg, 2, 1.0, 1.0, 0.25)
    assert list(idx) == [2, 1] and cum[0] == np.float32(0.5)
    lg = np.array([1, 1, 2], np.float32)
    tok, idx, _ = oracle.sample_topk_wgsl_detail(lg, 2, 1.0, 1.0, 0.99)
    assert list(idx) == [2, 1] and tok == 1


def test_sampler_draw_on_a_boundary():
    """rand < running total picks the slot, so rand equal to a total moves to
    the next slot, and rand at or past the last total takes the last slot."""
    rng = np.random.default_rng(5)
    lg = rng.standard_normal(300).astype(np.float32)
    _, idx, cum = oracle.sample_topk_wgsl_detail(lg, 40, 0.9, 1.0, 0.5)
    assert np.all(np.diff(cum) >= 0)
    for j in (0, 7, 38):
        assert oracle.sample_topk_wgsl(lg, 40, 0.9, 1.0, float(cum[j]))[0] == idx[j + 1]
        below = float(np.nextafter(cum[j], np.float32(-1)))
        assert oracle.sample_topk_wgsl(lg, 40, 0.9, 1.0, below)[0] == idx[j]
    assert oracle.sample_topk_wgsl(lg, 40, 0.9, 1.0, float(cum[-1]))[0] == idx[-1]
