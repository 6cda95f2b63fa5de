"""Writes the golden fixtures of tests/golden/ from the CPU oracle.

Run from the repository root after `make -C oracle`:
    python tests/golden/make_golden.py

Inputs are regenerated at test time from the SplitMix64/Box-Muller spec
(oracle.normal); each fixture stores the seeds, shapes, the SHA-256 of the
generated inputs (so a changed generator is caught) and the expected outputs:
`out_wgsl` (the shader's own f32 order) and `out_f64` (closed form in double).
Q4_K cases also store their weight blocks and the dequantised weights; the
depformer chain case stores its tokens, per-step logits and sampling inputs
(its weights are regenerated from a seed and checked by hash).
RoPE (theta 1e4, interleaved) is applied to Q and K at their logical
positions, as the configs specify.
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))
import oracle  # noqa: E402
from cases import decode_inputs, prefill_inputs, scale_for  # noqa: E402


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def decode_case(seed, H, D, M, L, start, rope=True):
    """One decode: window of L rows at ring slot `start`, query at position L-1."""
    scale = scale_for(D)
    q, kc, vc = decode_inputs(seed, H, D, M, L, start, rope)
    out_w = oracle.attention_ring_wgsl(q, kc, vc, start, L, scale)
    out_d = oracle.attention_ring_f64(q, kc, vc, start, L, scale)
    return dict(seed=seed, H=H, D=D, M=M, L=L, start=start, rope=int(rope), scale=scale,
                input_sha=sha(q, kc, vc), out_wgsl=out_w, out_f64=out_d)


def prefill_case(seed, H, D, M, cached, S, start):
    scale = scale_for(D)
    L = cached + S
    q, kc, vc = prefill_inputs(seed, H, D, M, cached, S, start)
    out_d = oracle.prefill_f64(q, kc, vc, start, L, scale)
    out_w = oracle.prefill_seq_wgsl(q, kc, vc, start, L, scale)
    return dict(seed=seed, H=H, D=D, M=M, cached=cached, S=S, start=start, scale=scale,
                input_sha=sha(q, kc, vc), out_wgsl=out_w, out_f64=out_d)


def q4k_case(seed, N, K, B, quantized=False):
    """Q4_K matvec: blocks from random bytes (every scale and quant pattern)
    or from the reference's quantizer applied to normal data."""
    if quantized:
        blocks = oracle.q4k_quantize(oracle.normal(seed, (N, K)) * 0.05)
    else:
        blocks = oracle.q4k_random_blocks(seed, N, K)
    x = oracle.normal(seed + 1, (B, K))
    return dict(seed=seed, N=N, K=K, B=B, quantized=int(quantized), input_sha=sha(blocks, x),
                blocks=blocks, dequant=oracle.q4k_dequant(blocks, N, K),
                out_wgsl=oracle.q4k_matvec_wgsl(blocks, x, N),
                out_f64=oracle.q4k_matvec_f64(blocks, x, N))


DEPF_CFG = dict(num_steps=4, num_layers=2, dim=256, num_heads=4, ffn=512, temporal_dim=512,
                out_vocab=128, text_emb_vocab=300, audio_emb_vocab=129, num_audio_emb=3,
                kv_max_len=5, rms_eps=1e-8, attn_scale=0.125)


def depformer_case(seed, wseed):
    """The depformer step chain on one stream at a small shape: weights from
    oracle.DepformerWeights.synthetic(seed=wseed) (hashed, not stored), the
    temporal hidden state from oracle.normal(seed), top_k 20, temperature
    0.8, penalty 1.2.  out_wgsl: the oracle's logits per step; out_f64: the
    float64 restatement of the chain fed the same tokens."""
    from test_oracle_depformer import _chain_f64
    w = oracle.DepformerWeights.synthetic(DEPF_CFG, seed=wseed)
    S = DEPF_CFG["num_steps"]
    th = oracle.normal(seed, (DEPF_CFG["temporal_dim"],))
    rand = np.array([0.31, 0.77, 0.05, 0.52], np.float32)
    pt = np.zeros((S, 30), np.uint32)
    pt[1, :4] = [3, 9, 3, 200]
    npn = np.array([0, 4, 0, 0], np.uint32)
    tokens, logits, _ = oracle.depformer_generate(w, th, 17, 20, 0.8, 1.2, rand, pt, npn)
    weights = [a for f in oracle.DepformerWeights.FIELDS for a in getattr(w, f)] + [w.text_emb]
    return dict(seed=seed, wseed=wseed, text_token=17, top_k=20, temperature=0.8, penalty=1.2,
                rand=rand, penalty_tokens=pt, num_penalty=npn,
                input_sha=sha(th, *weights), tokens=tokens, out_wgsl=logits,
                out_f64=_chain_f64(w, th, 17, tokens))


CASES = {
    # The plumbing case: 1 layer, 32 x 128, L = 256, window at slot 0.
    "decode_config1": lambda: decode_case(101, 32, 128, 256, 256, 0),
    # Small wrapped windows (both head sizes), L = 1, and a window longer than 256 lanes.
    "decode_wrap_d64": lambda: decode_case(202, 4, 64, 9, 7, 5),
    "decode_wrap_d128": lambda: decode_case(303, 3, 128, 40, 33, 29),
    "decode_len1": lambda: decode_case(404, 2, 128, 16, 1, 11),
    "decode_long": lambda: decode_case(505, 2, 128, 700, 611, 400),
    # Depformer-shaped (16 x 64, no RoPE, M = 9).
    "depformer_step5": lambda: decode_case(606, 16, 64, 9, 6, 0, rope=False),
    # Chunked prefill, small: 70 new rows after 45 cached, wrapped ring.
    "prefill_small": lambda: prefill_case(707, 1, 128, 128, 45, 70, 100),
    "prefill_small_d64": lambda: prefill_case(808, 2, 64, 100, 30, 33, 90),
    # Q4_K projections: random blocks over three super-blocks per row, batch 2;
    # and quantizer-made blocks.
    "q4k_random": lambda: q4k_case(909, 6, 768, 2),
    "q4k_quantized": lambda: q4k_case(1010, 4, 512, 1, quantized=True),
    # The depformer step chain (depth_engine.rs:884-1491), one stream, small shape.
    "depformer_chain_small": lambda: depformer_case(1111, 3),
}


def main():
    for name, fn in CASES.items():
        d = fn()
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **{k: np.asarray(v) for k, v in d.items()})
        print(f"{name}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
