"""Seeded input builders shared by the fixture generator and the GPU tests.

All inputs follow one recipe: Q, K, V drawn N(0,1) from
the oracle's SplitMix64 / Box-Muller generator, RoPE (theta 1e4, interleaved)
applied to Q and K at their logical positions, K/V rows written into a ring
cache [B, H, M, D] whose window starts at slot `start` (so reads wrap).
"""
import numpy as np

import oracle


def scale_for(d: int) -> float:
    return float(np.float32(d) ** np.float32(-0.5))


def decode_inputs(seed, H, D, M, L, start, rope=True, theta=10000.0):
    """q [H, D] for the newest row (position L-1); caches [H, M, D]."""
    q = oracle.normal(seed, (1, 1, H, D))
    k_rows = oracle.normal(seed + 1, (1, L, H, D))
    v_rows = oracle.normal(seed + 2, (1, L, H, D))
    if rope:
        tabs = oracle.rope_tables(D, max(L, 1), theta)
        q = oracle.rope_apply(q, L - 1, tabs)
        k_rows = oracle.rope_apply(k_rows, 0, tabs)
    kc = np.zeros((1, H, M, D), np.float32)
    vc = np.zeros((1, H, M, D), np.float32)
    oracle.cache_write(k_rows, kc, start, M)
    oracle.cache_write(v_rows, vc, start, M)
    return q.reshape(H, D), kc[0], vc[0]


def prefill_inputs(seed, H, D, M, cached, S, start):
    """q [S, H, D] at positions cached..cached+S-1; caches [H, M, D] holding
    cached + S rows starting at slot `start`."""
    L = cached + S
    q = oracle.normal(seed, (1, S, H, D))
    k_rows = oracle.normal(seed + 1, (1, L, H, D))
    v_rows = oracle.normal(seed + 2, (1, L, H, D))
    tabs = oracle.rope_tables(D, L, 10000.0)
    q = oracle.rope_apply(q, cached, tabs)
    k_rows = oracle.rope_apply(k_rows, 0, tabs)
    kc = np.zeros((1, H, M, D), np.float32)
    vc = np.zeros((1, H, M, D), np.float32)
    oracle.cache_write(k_rows, kc, start, M)
    oracle.cache_write(v_rows, vc, start, M)
    return q.reshape(S, H, D), kc[0], vc[0]
