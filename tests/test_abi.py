"""The C ABI on the host (no GPU needed): exports, argument checks, KV counters.

Argument errors are detected before any device work, so they are exercised
here without a GPU; every one must return a negative status with a message
and never abort the process.  The KV counter tests restate the reference's
unit tests (crates/sts-wasm/src/model.rs:1459-1552, depth.rs:1091-1118)
against the library's KVCache handle; counters move without device buffers.
"""
import ctypes
import os
import re

import pytest

import oracle
import sts_attn
from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "sts_attn.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sts_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_functions() == sorted(sts_attn.SIGNATURES)


def test_precision_constants_match_header():
    """The binding's precision codes are the header's enum values."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    enum = dict((k, int(v)) for k, v in re.findall(r"\b(STS_PREC_[A-Z0-9_]+)\s*=\s*(\d+)", text))
    assert enum == {"STS_PREC_F32": sts_attn.PREC_F32,
                    "STS_PREC_BF16_MFMA": sts_attn.PREC_BF16_MFMA,
                    "STS_PREC_F32_SPLIT_BF16": sts_attn.PREC_F32_SPLIT_BF16}


def test_library_exports_every_declared_symbol():
    lib = sts_attn.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.sts_abi_version() == 3
    # The header's version macro agrees with the library's.
    text = open(HEADER).read()
    assert int(re.search(r"#define STS_ATTN_ABI_VERSION (\d+)", text).group(1)) == 3


def test_kv_state_layout_matches_header():
    """sts_kv_state field order and types as the header declares them."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    body = re.search(r"typedef struct sts_kv_state \{(.*?)\} sts_kv_state;", text, re.S).group(1)
    fields = re.findall(r"(u?int\d+_t)\s+(\w+);", body)
    ctypes_of = {"uint64_t": ctypes.c_uint64, "int32_t": ctypes.c_int32}
    assert [(n, ctypes_of[t]) for t, n in fields] == list(sts_attn.KvState._fields_)
    assert ctypes.sizeof(sts_attn.KvState) == 72


def test_query_heads_argument_errors():
    """Grouped-query setter: a multiple of the K/V heads, at least them, at most
    65535; a rejected call leaves the handle's query heads unchanged."""
    lib = sts_attn.load()
    c = sts_attn.KVCache(16, 4, 64)
    s = lib.sts_kv_set_query_heads
    assert "null" in _err(s(None, 8))
    assert "multiple" in _err(s(c.handle, 6))
    assert "multiple" in _err(s(c.handle, 2))
    assert "multiple" in _err(s(c.handle, 4 * 65536))
    assert c.state().q_heads == 4
    assert s(c.handle, 12) == 0
    assert c.state().q_heads == 12 and c.state().heads == 4
    g = sts_attn.KVCache(16, 2, 128, n_heads=8)
    assert (g.state().heads, g.state().q_heads) == (2, 8)


def test_status_constants_match_header():
    """The binding's status and device-error codes are the header's enum values."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    enum = dict((k, int(v)) for k, v in
                re.findall(r"\b(STS_(?:ERR|DEVERR)_[A-Z0-9_]+|STS_OK)\s*=\s*(-?\d+)", text))
    assert enum == {"STS_OK": sts_attn.STS_OK, "STS_ERR_INVALID": sts_attn.STS_ERR_INVALID,
                    "STS_ERR_HIP": sts_attn.STS_ERR_HIP, "STS_ERR_STATE": sts_attn.STS_ERR_STATE,
                    "STS_ERR_NOMEM": sts_attn.STS_ERR_NOMEM,
                    "STS_ERR_DEVICE": sts_attn.STS_ERR_DEVICE,
                    "STS_DEVERR_WAIT_TIMEOUT": sts_attn.DEVERR_WAIT_TIMEOUT}


def _err(rc):
    assert rc < 0
    msg = sts_attn.load().sts_last_error().decode()
    assert msg
    return msg


FAKE = 0x10000  # a 16-byte aligned non-null pointer; never dereferenced


def test_fused_attention_argument_errors():
    lib = sts_attn.load()
    f = lib.sts_fused_attention
    assert "null" in _err(f(None, FAKE, FAKE, FAKE, 32, 128, 10, 0.1, 1280, None))
    # Any multiple of 4 up to 128 is taken (the shader's limit); others are not.
    assert "head_dim" in _err(f(FAKE, FAKE, FAKE, FAKE, 32, 102, 10, 0.1, 1020, None))
    assert "head_dim" in _err(f(FAKE, FAKE, FAKE, FAKE, 32, 0, 10, 0.1, 0, None))
    assert "head_dim" in _err(f(FAKE, FAKE, FAKE, FAKE, 32, 132, 10, 0.1, 1320, None))
    assert "head_dim" in _err(f(FAKE, FAKE, FAKE, FAKE, 32, 256, 10, 0.1, 2560, None))
    assert "seq_len" in _err(f(FAKE, FAKE, FAKE, FAKE, 32, 128, 0, 0.1, 1280, None))
    assert "stride" in _err(f(FAKE, FAKE, FAKE, FAKE, 32, 128, 10, 0.1, 128, None))
    assert "aligned" in _err(f(FAKE + 4, FAKE, FAKE, FAKE, 32, 128, 10, 0.1, 1280, None))
    assert "scale" in _err(f(FAKE, FAKE, FAKE, FAKE, 32, 128, 10, float("nan"), 1280, None))


def test_cache_write_argument_errors():
    f = sts_attn.load().sts_cache_write
    assert "null" in _err(f(None, FAKE, 0, 1, 1, 32, 128, 3000, None))
    assert "collide" in _err(f(FAKE, FAKE, 0, 1, 3001, 32, 128, 3000, None))
    assert "max_len" in _err(f(FAKE, FAKE, 0, 1, 1, 32, 128, 0, None))


def test_decode_ring_and_depformer_argument_errors():
    lib = sts_attn.load()
    assert "null" in _err(lib.sts_decode_ring(FAKE, FAKE, FAKE, FAKE, None, FAKE, 4, 32, 128,
                                              3000, 0.1, None))
    assert "head_dim" in _err(lib.sts_decode_ring(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, 32, 98,
                                                  3000, 0.1, None))
    assert "step" in _err(lib.sts_depformer_step(FAKE, FAKE, FAKE, 3072, FAKE, FAKE, FAKE, 64,
                                                 16, 64, 9, 9, 0.125, None))
    assert "qkv_stride" in _err(lib.sts_depformer_step(FAKE, FAKE, FAKE, 100, FAKE, FAKE, FAKE,
                                                       64, 16, 64, 9, 0, 0.125, None))


def test_prefill_argument_errors():
    f = sts_attn.load().sts_prefill_attention
    assert "seq" in _err(f(FAKE, FAKE, FAKE, FAKE, 0, 32, 128, 3000, 0, 768, 0.1, 0, None))
    assert "seq" in _err(f(FAKE, FAKE, FAKE, FAKE, 800, 32, 128, 3000, 0, 768, 0.1, 0, None))
    assert "win_len" in _err(f(FAKE, FAKE, FAKE, FAKE, 512, 32, 128, 700, 0, 768, 0.1, 0, None))
    assert "win_start" in _err(f(FAKE, FAKE, FAKE, FAKE, 512, 32, 128, 3000, 3000, 768, 0.1, 0,
                                 None))
    assert "precision" in _err(f(FAKE, FAKE, FAKE, FAKE, 512, 32, 128, 3000, 0, 768, 0.1, 7,
                                 None))


def test_kv_prefill_rejects_before_any_device_work():
    """sts_kv_prefill validates every argument before it allocates, appends or
    moves the counters: on an unallocated cache a rejected call leaves it
    unallocated and at offset 0."""
    lib = sts_attn.load()
    c = sts_attn.KVCache(64, 4, 128)
    cases = [
        ("precision", (None, FAKE, FAKE, FAKE, FAKE, 5, 0.1, 9)),
        ("aligned", (None, FAKE + 4, FAKE, FAKE, FAKE, 5, 0.1, 0)),
        ("scale", (None, FAKE, FAKE, FAKE, FAKE, 5, float("inf"), 0)),
        ("seq", (None, FAKE, FAKE, FAKE, FAKE, 65, 0.1, 0)),
        ("null", (None, None, FAKE, FAKE, FAKE, 5, 0.1, 0)),
    ]
    for word, (rope, q, k, v, out, seq, scale, prec) in cases:
        assert word in _err(lib.sts_kv_prefill(c.handle, rope, q, k, v, out, seq, scale, prec,
                                               None))
        s = c.state()
        assert (s.offset, s.len, s.write_pos, s.allocated) == (0, 0, 0, 0)


def test_bf16kv_prefill_needs_its_head_dims():
    """The bf16-K/V prefill has no padded form: head dims other than 64 and 128
    are refused before any device work."""
    lib = sts_attn.load()
    assert "bf16 K/V" in _err(lib.sts_prefill_attention_bf16kv(FAKE, FAKE, FAKE, FAKE, 4, 2, 96,
                                                                100, 0, 50, 0.1, None))


def test_padded_head_dim_prefill_length_checked_first():
    """At head dims other than 64/128 a chunk runs as one decode launch with
    the queries as streams (at most 65535): a longer chunk is refused before
    anything is appended (fake pointers, never dereferenced)."""
    lib = sts_attn.load()
    c = sts_attn.KVCache(100000, 2, 96)
    rc = lib.sts_kv_prefill(c.handle, None, FAKE, FAKE, FAKE, FAKE, 70000, 0.1,
                            sts_attn.PREC_F32, None)
    assert "too long" in _err(rc)
    s = c.state()
    assert (s.offset, s.len, s.allocated) == (0, 0, 0)


def test_kv_handle_argument_errors():
    lib = sts_attn.load()
    h = ctypes.c_void_p()
    assert "head_dim" in _err(lib.sts_kv_create(3000, 32, 102, ctypes.byref(h)))
    assert "head_dim" in _err(lib.sts_kv_create(3000, 32, 192, ctypes.byref(h)))
    assert "max_len" in _err(lib.sts_kv_create(0, 32, 128, ctypes.byref(h)))
    assert "null" in _err(lib.sts_kv_advance(None, 1))
    c = sts_attn.KVCache(8, 2, 64)
    # attend before anything was appended: a state error, no device call
    assert lib.sts_kv_attend(c.handle, FAKE, FAKE, 0.125, None) == sts_attn.STS_ERR_STATE
    # a chunk longer than the ring is rejected before any allocation
    assert "seq" in _err(lib.sts_kv_update(c.handle, FAKE, FAKE, 1, 9, None))
    assert not c.state().allocated


def test_rope_argument_errors():
    lib = sts_attn.load()
    h = ctypes.c_void_p()
    assert "head_dim" in _err(lib.sts_rope_create(102, 3000, 1e4, ctypes.byref(h)))
    assert "theta" in _err(lib.sts_rope_create(128, 3000, -1.0, ctypes.byref(h)))
    assert "null" in _err(lib.sts_rope_apply(None, FAKE, 1, 1, 32, 0, None))


# --- KVCache counters through the C ABI (no device buffers needed) ----------

def test_kv_cache_ring_buffer_counters():
    """model.rs:1459-1495 with advance() in place of update(): max_len 4."""
    c = sts_attn.KVCache(4, 2, 64)
    assert (c.seq_len(), c.offset()) == (0, 0)
    for i in range(3):
        c.advance(1)
        assert c.seq_len() == i + 1
    assert c.offset() == 3
    c.advance(1)
    assert c.seq_len() == 4
    c.advance(1)
    assert (c.seq_len(), c.offset()) == (4, 5)


def test_kv_cache_reset_counters():
    """model.rs:1497-1530."""
    c = sts_attn.KVCache(4, 2, 64)
    c.advance(1)
    c.reset()
    assert (c.seq_len(), c.offset(), c.write_pos()) == (0, 0, 0)
    c.advance(2)
    c.reset_keep_buffers()
    assert (c.seq_len(), c.offset()) == (0, 0)
    assert not c.state().allocated


def test_layer_caches_counters():
    """model.rs:1532-1552: LayerCaches::seq_len follows layer 0."""
    lc = sts_attn.LayerCaches(3, 10, 2, 64)
    assert lc.seq_len() == 0
    lc.get_mut(0).advance(1)
    assert lc.seq_len() == 1
    assert lc.get_mut(3) is None
    lc.reset()
    assert lc.seq_len() == 0


def test_depformer_cache_counters():
    """depth.rs:1091-1118: cache (20, 2, 32-dim in the reference; 64 here)."""
    c = sts_attn.KVCache(20, 2, 64)
    for i in range(3):
        c.advance(1)
        assert c.seq_len() == i + 1
    c.reset_keep_buffers()
    assert c.seq_len() == 0


@pytest.mark.parametrize("M", [1, 4, 9, 3000])
def test_counters_match_oracle_over_random_walk(M):
    """Any sequence of advance / rollback / reset agrees with the oracle's
    restatement of model.rs:293-362, and the window start stays in range."""
    import random
    rnd = random.Random(M)
    c = sts_attn.KVCache(M, 1, 64)
    o = oracle.KvCounters(M)
    for _ in range(400):
        op = rnd.random()
        if op < 0.6:
            n = rnd.randint(0, 2 * M + 3)
            c.advance(n)
            o.advance(n)
        elif op < 0.95:
            n = rnd.randint(0, M + 2)
            c.rollback(n)
            o.rollback(n)
        else:
            c.reset()
            o.reset()
        s = c.state()
        assert (s.offset, s.len, s.write_pos) == (o.offset, o.len, o.write_pos)
        start, ln = c.window()
        assert ln == o.len and start == o.window_start() and 0 <= start < M


def test_depformer_chain_argument_errors():
    """Rejected before any device work (no GPU needed)."""
    lib = sts_attn.load()
    assert "multiple of 256" in _err(lib.sts_q4k_gemm(FAKE, FAKE, 1000, None, 0.0, None, 0, FAKE,
                                                      3072, 64, 1000, 3072, 0, None))
    assert "SwiGLU" in _err(lib.sts_q4k_gemm(FAKE, FAKE, 1024, None, 0.0, FAKE, 5632, FAKE, 2816,
                                             64, 1024, 5632, 1, None))
    # Above k = 4096 (summed slices) no fused RMSNorm; beyond 16384 nothing.
    assert "RMSNorm" in _err(lib.sts_q4k_gemm(FAKE, FAKE, 11264, FAKE, 1e-5, None, 0, FAKE, 4096,
                                              64, 11264, 4096, 0, None))
    assert "multiple of 256" in _err(lib.sts_q4k_gemm(FAKE, FAKE, 16640, None, 0.0, None, 0, FAKE,
                                                      4096, 64, 16640, 4096, 0, None))
    # The summed-slice route checks the shape and alignment before it takes
    # any workspace.
    assert "too large" in _err(lib.sts_q4k_gemm(FAKE, FAKE, 11264, None, 0.0, None, 0, FAKE, 4096,
                                                16 * 65536 + 1, 11264, 4096, 0, None))
    assert "aligned" in _err(lib.sts_q4k_gemm(FAKE, FAKE + 4, 11264, None, 0.0, None, 0, FAKE, 4096,
                                              64, 11264, 4096, 0, None))
    assert "aligned" in _err(lib.sts_q4k_gemm(FAKE + 4, FAKE, 11264, None, 0.0, None, 0, FAKE, 4096,
                                              64, 11264, 4096, 0, None))
    assert "strides" in _err(lib.sts_q4k_gemm(FAKE, FAKE, 512, None, 0.0, None, 0, FAKE, 3072, 64,
                                              1024, 3072, 0, None))
    assert "norm_eps" in _err(lib.sts_q4k_gemm(FAKE, FAKE, 1024, FAKE, -1.0, None, 0, FAKE, 3072,
                                               64, 1024, 3072, 0, None))
    assert "null" in _err(lib.sts_rmsnorm(None, FAKE, FAKE, 4, 1024, 1e-8, None))
    assert "eps" in _err(lib.sts_rmsnorm(FAKE, FAKE, FAKE, 4, 1024, float("nan"), None))
    assert "multiple of 32" in _err(lib.sts_embed_add_q4_0(FAKE, 10, FAKE, 1, FAKE, FAKE, 2, 100,
                                                          None))
    assert "aligned" in _err(lib.sts_embed_add_q4_0(FAKE + 1, 10, FAKE, 1, FAKE, FAKE, 2, 128,
                                                   None))
    assert "vocab" in _err(lib.sts_sample_topk(FAKE, 5000, 2, 5000, 10, 1.0, 1.0, FAKE, FAKE, 30,
                                               FAKE, 1, FAKE, 1, None))
    assert "top_k" in _err(lib.sts_sample_topk(FAKE, 2048, 2, 2048, 257, 1.0, 1.0, FAKE, FAKE, 30,
                                               FAKE, 1, FAKE, 1, None))
    assert "temperature" in _err(lib.sts_sample_topk(FAKE, 2048, 2, 2048, 5, 0.0, 1.0, FAKE, FAKE,
                                                     30, FAKE, 1, FAKE, 1, None))
    cfg = sts_attn.DepformerConfig.personaplex()
    cfg.num_heads = 12  # head_dim 85
    h = ctypes.c_void_p()
    w = sts_attn.DepformerWeightPtrs()
    assert "bad layers" in _err(lib.sts_depformer_create(ctypes.byref(cfg), ctypes.byref(w), 4,
                                                          ctypes.byref(h)))
    cfg = sts_attn.DepformerConfig.personaplex()
    cfg.kv_max_len = 4
    assert "kv_max_len" in _err(lib.sts_depformer_create(ctypes.byref(cfg), ctypes.byref(w), 4,
                                                          ctypes.byref(h)))
    cfg = sts_attn.DepformerConfig.personaplex()
    assert "null weight" in _err(lib.sts_depformer_create(ctypes.byref(cfg), ctypes.byref(w), 4,
                                                           ctypes.byref(h)))
    assert "null" in _err(lib.sts_depformer_generate(None, FAKE, FAKE, 1, 1, 1.0, 1.0, FAKE, FAKE,
                                                     FAKE, FAKE, None, None))
