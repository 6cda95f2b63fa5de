"""CPU oracle for sts-web's attention hot path (ctypes view of liboracle.so).

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker or the timed CPU baseline -- the product library never calls it.

The C sources (oracle.c) restate the reference algorithm function by function,
each citing the reference file:line it follows; the numpy helpers below only
marshal arrays.  Build with ``make -C oracle``.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64


class KvState(ctypes.Structure):
    _fields_ = [("offset", _u64), ("len", _u64), ("write_pos", _u64), ("max_len", _u64)]

    def as_tuple(self):
        return (self.offset, self.len, self.write_pos, self.max_len)


class DepformerCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "num_steps", "num_layers", "dim", "num_heads", "ffn", "temporal_dim", "out_vocab",
        "text_emb_vocab", "audio_emb_vocab", "num_audio_emb", "kv_max_len")] + [
        ("rms_eps", ctypes.c_float), ("attn_scale", ctypes.c_float)]


_vpp = ctypes.POINTER(ctypes.c_void_p)


class DepformerWeightPtrs(ctypes.Structure):
    _fields_ = [("input_proj", _vpp), ("attn_in_proj", _vpp), ("attn_out_proj", _vpp),
                ("ffn_linear_in", _vpp), ("ffn_linear_out", _vpp), ("norm1_alpha", _vpp),
                ("norm2_alpha", _vpp), ("output_linear", _vpp), ("text_emb", ctypes.c_void_p),
                ("audio_emb", _vpp)]


def _load():
    if not os.path.exists(_LIB_PATH):
        raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run `make -C oracle`)")
    lib = ctypes.CDLL(_LIB_PATH)
    sig = {
        "orc_splitmix64": (_u64, [_u64, _u64]),
        "orc_fill_normal": (None, [_u64, _u64, _u64, _f32p]),
        "orc_rope_tables": (None, [_u32, _u32, ctypes.c_float, _f32p, _f32p]),
        "orc_rope_apply": (None, [_f32p, _u32, _u32, _u32, _u32, _u32, _f32p, _f32p]),
        "orc_cache_write": (None, [_f32p, _f32p, _u32, _u32, _u32, _u32, _u32, _u32]),
        "orc_gqa_expand": (None, [_f32p, _f32p, _u32, _u32, _u32, _u64]),
        "orc_kv_init": (None, [ctypes.POINTER(KvState), _u64]),
        "orc_kv_advance": (None, [ctypes.POINTER(KvState), _u64]),
        "orc_kv_update": (None, [ctypes.POINTER(KvState)]),
        "orc_kv_reset": (None, [ctypes.POINTER(KvState)]),
        "orc_kv_rollback": (None, [ctypes.POINTER(KvState), _u64]),
        "orc_attention_wgsl": (None, [_f32p, _f32p, _f32p, _f32p, _u32, _u32, _u32,
                                      ctypes.c_float, _u64]),
        "orc_attention_ring_wgsl": (None, [_f32p, _f32p, _f32p, _f32p, _u32, _u32, _u32,
                                           _u32, _u32, ctypes.c_float]),
        "orc_decode_frame_wgsl": (None, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_void_p, _u32, _u32, _u32, _u32,
                                         ctypes.POINTER(_u32), ctypes.POINTER(_u32),
                                         ctypes.c_float]),
        "orc_attention_ring_f64": (None, [_f32p, _f32p, _f32p, _f64p, _u32, _u32, _u32,
                                          _u32, _u32, ctypes.c_double]),
        "orc_prefill_f64": (None, [_f32p, _f32p, _f32p, _f64p, _u32, _u32, _u32, _u32,
                                   _u32, _u32, ctypes.c_double]),
        "orc_prefill_seq_wgsl": (None, [_f32p, _f32p, _f32p, _f32p, _u32, _u32, _u32, _u32,
                                        _u32, _u32, ctypes.c_float]),
        "orc_f16_to_f32_n": (None, [ctypes.c_void_p, _f32p, _u64]),
        "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
        "orc_q4k_scale_min": (None, [ctypes.c_void_p, _u32, ctypes.POINTER(_u32),
                                     ctypes.POINTER(_u32)]),
        "orc_q4k_dequant": (None, [ctypes.c_void_p, _u32, _u32, _f32p]),
        "orc_q4k_quantize": (None, [_f32p, _u32, _u32, ctypes.c_void_p]),
        "orc_q4k_matvec_wgsl": (None, [ctypes.c_void_p, _f32p, _f32p, _u32, _u32, _u32]),
        "orc_q4k_matvec_f64": (None, [ctypes.c_void_p, _f32p, _f64p, _u32, _u32, _u32]),
        "orc_rmsnorm_wgsl": (None, [_f32p, _f32p, _f32p, _u32, ctypes.c_float]),
        "orc_swiglu": (None, [_f32p, _f32p, _u32]),
        "orc_embed_q4_0": (None, [ctypes.c_void_p, _u32, _u32, _u32, _f32p]),
        "orc_sample_topk_wgsl": (_u32, [_f32p, _u32, _u32, ctypes.c_float, ctypes.c_float,
                                        ctypes.c_float, ctypes.POINTER(_u32), _u32]),
        "orc_sample_topk_wgsl_ex": (_u32, [_f32p, _u32, _u32, ctypes.c_float, ctypes.c_float,
                                        ctypes.c_float, ctypes.POINTER(_u32), _u32, ctypes.POINTER(_u32), _f32p]),
        "orc_depformer_generate": (None, [ctypes.POINTER(DepformerCfg),
                                          ctypes.POINTER(DepformerWeightPtrs), _f32p, _u32,
                                          _u32, ctypes.c_float, ctypes.c_float, _f32p,
                                          ctypes.POINTER(_u32), ctypes.POINTER(_u32),
                                          ctypes.POINTER(_u32), _f32p, _f32p]),
        "orc_num_threads": (ctypes.c_int, []),
        "orc_set_num_threads": (None, [ctypes.c_int]),
        "orc_bind_threads": (ctypes.c_int, [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _p32(a):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_f32p)


def _p64(a):
    assert a.dtype == np.float64 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_f64p)


# ---- RNG ------------------------------------------------------------------

def splitmix64(seed: int, i: int) -> int:
    return lib().orc_splitmix64(seed, i)


def normal(seed: int, shape, first: int = 0) -> np.ndarray:
    """N(0,1) f32 samples first..first+n-1 of stream `seed`, shaped `shape`."""
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, dtype=np.float32)
    if n:
        lib().orc_fill_normal(seed, first, n, _p32(out))
    return out.reshape(shape)


# ---- RoPE -----------------------------------------------------------------

def rope_tables(head_dim: int, max_seq_len: int, theta: float = 10000.0):
    half = head_dim // 2
    c = np.empty((max_seq_len, half), dtype=np.float32)
    s = np.empty((max_seq_len, half), dtype=np.float32)
    lib().orc_rope_tables(head_dim, max_seq_len, theta, _p32(c), _p32(s))
    return c, s


def rope_apply(x: np.ndarray, offset: int, tables) -> np.ndarray:
    """Rotated copy of x [B,S,H,D] at positions offset.. (model.rs:79-105)."""
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    B, S, H, D = y.shape
    c, s = tables
    assert offset + S <= c.shape[0]
    lib().orc_rope_apply(_p32(y), B, S, H, D, offset, _p32(c), _p32(s))
    return y


# ---- KV append / counters ---------------------------------------------------

def cache_write(inp: np.ndarray, cache: np.ndarray, pos_offset: int, max_len: int) -> None:
    """In place: cache [B,H,M,D] <- inp [B,S,H,D] at (pos_offset+s) % M."""
    B, S, H, D = inp.shape
    assert cache.shape == (B, H, max_len, D)
    lib().orc_cache_write(_p32(np.ascontiguousarray(inp)), _p32(cache), pos_offset, B, S, H, D,
                          max_len)


def gqa_expand(kv: np.ndarray, rep: int) -> np.ndarray:
    """K/V heads repeated for grouped-query attention (model.rs:766-783):
    kv [..., nkv, S, D] -> [..., nkv * rep, S, D], head j * rep + r = head j.
    The leading axes (if any) are batch."""
    kv = np.ascontiguousarray(kv, np.float32)
    *lead, nkv, S, D = kv.shape
    B = int(np.prod(lead)) if lead else 1
    out = np.empty((*lead, nkv * rep, S, D), np.float32)
    lib().orc_gqa_expand(_p32(kv), _p32(out), B, nkv, rep, S * D)
    return out


class KvCounters:
    """KVCache counters (model.rs:195-363) evaluated by the C oracle."""

    def __init__(self, max_len: int):
        self._s = KvState()
        lib().orc_kv_init(ctypes.byref(self._s), max_len)

    def advance(self, n: int):
        lib().orc_kv_advance(ctypes.byref(self._s), n)

    def update(self):
        lib().orc_kv_update(ctypes.byref(self._s))

    def reset(self):
        lib().orc_kv_reset(ctypes.byref(self._s))

    def rollback(self, n: int):
        lib().orc_kv_rollback(ctypes.byref(self._s), n)

    @property
    def offset(self):
        return self._s.offset

    @property
    def len(self):
        return self._s.len

    @property
    def write_pos(self):
        return self._s.write_pos

    def window_start(self):
        m = self._s.max_len
        return (self._s.write_pos + m - self._s.len) % m


# ---- attention --------------------------------------------------------------

def attention_wgsl(q, k, v, seq_len: int, scale: float, kv_head_stride: int) -> np.ndarray:
    """shader_attention.wgsl in its own f32 order; q [H,D], k/v flat buffers."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    H, D = q.shape
    k = np.ascontiguousarray(k, dtype=np.float32).reshape(-1)
    v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
    assert k.size >= (H - 1) * kv_head_stride + seq_len * D
    out = np.empty((H, D), dtype=np.float32)
    lib().orc_attention_wgsl(_p32(q), _p32(k), _p32(v), _p32(out), H, D, seq_len, scale,
                             kv_head_stride)
    return out


def attention_ring_wgsl(q, kc, vc, start: int, length: int, scale: float) -> np.ndarray:
    """Shader-order decode over ring window; q [H,D], kc/vc [H,M,D]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    H, M, D = kc.shape
    out = np.empty((H, D), dtype=np.float32)
    lib().orc_attention_ring_wgsl(_p32(q), _p32(np.ascontiguousarray(kc)),
                                  _p32(np.ascontiguousarray(vc)), _p32(out), H, D, M, start,
                                  length, scale)
    return out


def decode_frame_wgsl(qs, kcs, vcs, starts, lens, scale: float) -> list:
    """Shader-order decode of every (layer, head), parallel over (layer, head):
    qs[l] [H,D], kcs[l]/vcs[l] [H,M,D], window of layer l = lens[l] rows from
    slot starts[l].  Returns the outputs [H,D] per layer.  The arrays are used
    in place (they must be C-contiguous float32)."""
    L = len(qs)
    H, M, D = kcs[0].shape
    for a in list(qs) + list(kcs) + list(vcs):
        assert a.dtype == np.float32 and a.flags.c_contiguous
    outs = [np.empty((H, D), np.float32) for _ in range(L)]
    arr = lambda xs: (ctypes.c_void_p * L)(*[x.ctypes.data for x in xs])
    st = (_u32 * L)(*[int(x) for x in starts])
    ln = (_u32 * L)(*[int(x) for x in lens])
    lib().orc_decode_frame_wgsl(arr(qs), arr(kcs), arr(vcs), arr(outs), L, H, D, M, st, ln,
                                scale)
    return outs


def attention_ring_f64(q, kc, vc, start: int, length: int, scale: float) -> np.ndarray:
    """Closed-form decode in double over ring window; q [H,D], kc/vc [H,M,D]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    H, M, D = kc.shape
    out = np.empty((H, D), dtype=np.float64)
    lib().orc_attention_ring_f64(_p32(q), _p32(np.ascontiguousarray(kc)),
                                 _p32(np.ascontiguousarray(vc)), _p64(out), H, D, M, start,
                                 length, scale)
    return out


def prefill_f64(q, kc, vc, start: int, length: int, scale: float) -> np.ndarray:
    """Causal chunk attention in double; q [S,H,D], kc/vc [H,M,D]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    S, H, D = q.shape
    M = kc.shape[1]
    assert kc.shape == (H, M, D) and S <= length <= M
    out = np.empty((S, H, D), dtype=np.float64)
    lib().orc_prefill_f64(_p32(q), _p32(np.ascontiguousarray(kc)),
                          _p32(np.ascontiguousarray(vc)), _p64(out), S, H, D, M, start,
                          length, scale)
    return out


def prefill_seq_wgsl(q, kc, vc, start: int, length: int, scale: float) -> np.ndarray:
    """The reference's prefill: S sequential shader-order decodes."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    S, H, D = q.shape
    M = kc.shape[1]
    assert kc.shape == (H, M, D) and S <= length <= M
    out = np.empty((S, H, D), dtype=np.float32)
    lib().orc_prefill_seq_wgsl(_p32(q), _p32(np.ascontiguousarray(kc)),
                               _p32(np.ascontiguousarray(vc)), _p32(out), S, H, D, M, start,
                               length, scale)
    return out


def num_threads() -> int:
    return lib().orc_num_threads()


def set_num_threads(n: int) -> None:
    lib().orc_set_num_threads(n)


def bind_threads(cpus, pin: bool = True) -> int:
    """Runs OpenMP thread t of the following len(cpus)-thread regions on cpus[t]
    (pin) or on any of cpus (unpin); returns how many bindings failed."""
    arr = (ctypes.c_int * len(cpus))(*cpus)
    return lib().orc_bind_threads(arr, len(cpus), 1 if pin else 0)


# ---- Q4_K -------------------------------------------------------------------

Q4K_BLOCK_BYTES = 144
QK_K = 256


def _u8(a):
    a = np.ascontiguousarray(a, dtype=np.uint8)
    return a, a.ctypes.data_as(ctypes.c_void_p)


def f16_to_f32(bits):
    """unpack2x16float (shader_q4k_matvec.wgsl:82) elementwise on a uint16 array."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().orc_f16_to_f32_n(b.ctypes.data_as(ctypes.c_void_p), _p32(out), b.size)
    return out


def f32_to_f16(x):
    """Round-to-nearest-even f32 -> f16 bits (scalar)."""
    return int(lib().orc_f32_to_f16(float(np.float32(x))))


def q4k_scale_min(scales12, j):
    s, _ = _u8(scales12)
    sc, mn = _u32(), _u32()
    lib().orc_q4k_scale_min(s.ctypes.data_as(ctypes.c_void_p), j, ctypes.byref(sc),
                            ctypes.byref(mn))
    return sc.value, mn.value


def q4k_dequant(blocks, N, K):
    """[N][K] f32 weights from N*K/256 blocks of 144 bytes."""
    b, bp = _u8(blocks)
    assert b.size == N * K // QK_K * Q4K_BLOCK_BYTES
    w = np.empty((N, K), np.float32)
    lib().orc_q4k_dequant(bp, N, K, _p32(w))
    return w


def q4k_quantize(x):
    """scripts/quantize.py quantize_q4_k applied row by row to x [N][K]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    N, K = x.shape
    out = np.empty(N * K // QK_K * Q4K_BLOCK_BYTES, np.uint8)
    lib().orc_q4k_quantize(_p32(x), N, K, out.ctypes.data_as(ctypes.c_void_p))
    return out


def q4k_matvec_wgsl(blocks, x, N):
    """x [B][K] -> y [B][N] in the matvec shader's f32 order."""
    b, bp = _u8(blocks)
    x = np.ascontiguousarray(x, dtype=np.float32)
    B, K = x.shape
    y = np.empty((B, N), np.float32)
    lib().orc_q4k_matvec_wgsl(bp, _p32(x), _p32(y), B, K, N)
    return y


def q4k_matvec_f64(blocks, x, N):
    b, bp = _u8(blocks)
    x = np.ascontiguousarray(x, dtype=np.float32)
    B, K = x.shape
    y = np.empty((B, N), np.float64)
    lib().orc_q4k_matvec_f64(bp, _p32(x), y.ctypes.data_as(_f64p), B, K, N)
    return y


def q4k_random_blocks(seed, N, K):
    """Random Q4_K blocks: every scale/quant byte uniform, d and dmin finite
    positive halves in [2^-14, 2^-4) so weights stay O(1)."""
    rng = np.random.default_rng(seed)
    nb = N * K // QK_K
    blk = rng.integers(0, 256, size=(nb, Q4K_BLOCK_BYTES), dtype=np.uint8)
    for off in (0, 2):
        half = rng.integers(0x0400, 0x2C00, size=nb, dtype=np.uint16)  # exponents 1..10
        blk[:, off] = (half & 0xFF).astype(np.uint8)
        blk[:, off + 1] = (half >> 8).astype(np.uint8)
    return blk.reshape(-1)


# ---- depformer step chain (depth_engine.rs:884-1491) ------------------------

Q4_0_BLOCK_BYTES = 18


def rmsnorm_wgsl(x, alpha, eps):
    """shader_rmsnorm.wgsl on each row of x [R][D]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    a = np.ascontiguousarray(alpha, dtype=np.float32)
    out = np.empty_like(x)
    for r in range(x.shape[0]):
        lib().orc_rmsnorm_wgsl(_p32(x[r]), _p32(a), _p32(out[r]), x.shape[1], float(eps))
    return out


def swiglu(gv):
    """shader_swiglu.wgsl on each row of gv [R][2F] -> [R][F]."""
    gv = np.ascontiguousarray(gv, dtype=np.float32)
    F = gv.shape[1] // 2
    out = np.empty((gv.shape[0], F), np.float32)
    for r in range(gv.shape[0]):
        lib().orc_swiglu(_p32(gv[r]), _p32(out[r]), F)
    return out


def embed_q4_0(table, vocab, dim, token):
    t, tp = _u8(table)
    assert t.size == vocab * dim // 32 * Q4_0_BLOCK_BYTES
    out = np.empty(dim, np.float32)
    lib().orc_embed_q4_0(tp, vocab, dim, int(token), _p32(out))
    return out


def sample_topk_wgsl(logits, top_k, temperature, penalty, rand, penalty_tokens=()):
    """shader_sample_topk.wgsl on one row; returns (token, logits after penalty
    and temperature)."""
    lg = np.array(logits, dtype=np.float32, copy=True)
    pt = np.ascontiguousarray(np.asarray(penalty_tokens, dtype=np.uint32).reshape(-1))
    tok = lib().orc_sample_topk_wgsl(_p32(lg), lg.size, int(top_k), float(temperature),
                                     float(penalty), float(rand),
                                     pt.ctypes.data_as(ctypes.POINTER(_u32)), pt.size)
    return int(tok), lg


def sample_topk_wgsl_detail(logits, top_k, temperature, penalty, rand, penalty_tokens=()):
    """shader_sample_topk.wgsl on one row (top_k > 1); returns (token, the
    logit indices of the sorted slots, the draw's running totals)."""
    lg = np.array(logits, dtype=np.float32, copy=True)
    pt = np.ascontiguousarray(np.asarray(penalty_tokens, dtype=np.uint32).reshape(-1))
    idx = np.zeros(top_k, np.uint32)
    cum = np.zeros(top_k, np.float32)
    tok = lib().orc_sample_topk_wgsl_ex(_p32(lg), lg.size, int(top_k), float(temperature),
                                        float(penalty), float(rand),
                                        pt.ctypes.data_as(ctypes.POINTER(_u32)), pt.size,
                                        idx.ctypes.data_as(ctypes.POINTER(_u32)), _p32(cum))
    return int(tok), idx, cum


def q4_0_random_table(seed, vocab, dim, scale_lo=0x2000, scale_hi=0x2C00):
    """Random Q4_0 embedding table [vocab][dim]: nibbles uniform, f16 scales
    uniform over the bit patterns [scale_lo, scale_hi) (default ~0.008..0.06)."""
    rng = np.random.default_rng(seed)
    nb = vocab * dim // 32
    blk = rng.integers(0, 256, size=(nb, Q4_0_BLOCK_BYTES), dtype=np.uint8)
    half = rng.integers(scale_lo, scale_hi, size=nb, dtype=np.uint16)
    blk[:, 0] = (half & 0xFF).astype(np.uint8)
    blk[:, 1] = (half >> 8).astype(np.uint8)
    return blk.reshape(-1)


class DepformerWeights:
    """Host copies of a depformer's weights (numpy), in the layout of
    orc_depformer_weights: Q4_K bytes per matrix, f32 alphas, Q4_0 tables."""

    FIELDS = ("input_proj", "attn_in_proj", "attn_out_proj", "ffn_linear_in",
              "ffn_linear_out", "norm1_alpha", "norm2_alpha", "output_linear", "audio_emb")

    def __init__(self, cfg, **arrays):
        self.cfg = dict(cfg)
        for k, v in arrays.items():
            setattr(self, k, v)

    @classmethod
    def synthetic(cls, cfg, seed=0, quantize=True):
        """Weights ~ N(0, 1/K) per matrix, quantised with scripts/quantize.py's
        scheme (quantize=True) or random Q4_K bytes scaled to the same size
        (quantize=False, fast, for large shapes); alphas ~ 1 + N(0, 0.1^2)."""
        c = cfg
        S, L, D, F = c["num_steps"], c["num_layers"], c["dim"], c["ffn"]

        def mat(tag, n, k):
            if quantize:
                w = normal(seed * 1000003 + tag, (n, k)) / np.float32(np.sqrt(k))
                return q4k_quantize(w)
            return _random_q4k_scaled(seed * 1000003 + tag, n, k)

        tag = iter(range(1, 1 << 30))
        w = dict(
            input_proj=[mat(next(tag), D, c["temporal_dim"]) for _ in range(S)],
            attn_in_proj=[mat(next(tag), 3 * D, D) for _ in range(L * S)],
            attn_out_proj=[mat(next(tag), D, D) for _ in range(L * S)],
            ffn_linear_in=[mat(next(tag), 2 * F, D) for _ in range(L * S)],
            ffn_linear_out=[mat(next(tag), D, F) for _ in range(L * S)],
            norm1_alpha=[(1 + 0.1 * normal(seed * 7 + 1 + l, (D,))).astype(np.float32)
                         for l in range(L)],
            norm2_alpha=[(1 + 0.1 * normal(seed * 7 + 101 + l, (D,))).astype(np.float32)
                         for l in range(L)],
            output_linear=[mat(next(tag), c["out_vocab"], D) for _ in range(S)],
            text_emb=q4_0_random_table(seed * 13 + 1, c["text_emb_vocab"], D),
            audio_emb=[q4_0_random_table(seed * 13 + 2 + i, c["audio_emb_vocab"], D)
                       for i in range(c["num_audio_emb"])],
        )
        return cls(cfg, **w)


def _random_q4k_scaled(seed, n, k):
    """Random Q4_K bytes with d = dmin / 7.5 chosen so weights have mean ~0 and
    standard deviation ~1/sqrt(k)."""
    rng = np.random.default_rng(seed)
    nb = n * k // QK_K
    blk = rng.integers(0, 256, size=(nb, Q4K_BLOCK_BYTES), dtype=np.uint8)
    # w = d*sc*q - dmin*m with sc, m ~ U[0,64), q ~ U[0,16): E[w] = 0 when
    # dmin = 7.5 d; std(w) ~ 200 d.
    d = np.float16(1.0 / (200.0 * np.sqrt(k)))
    dm = np.float16(7.5 * float(d))
    for off, v in ((0, d), (2, dm)):
        bits = int(np.array(v, np.float16).view(np.uint16))
        blk[:, off] = bits & 0xFF
        blk[:, off + 1] = bits >> 8
    return blk.reshape(-1)


def _ptrs(arrs):
    keep = [np.ascontiguousarray(a) for a in arrs]
    arr = (ctypes.c_void_p * len(keep))(*[a.ctypes.data for a in keep])
    return arr, keep


def depformer_cfg_struct(cfg):
    return DepformerCfg(**{f: cfg[f] for f, _ in DepformerCfg._fields_})


def depformer_generate(weights, temporal_hidden, text_token, top_k, temperature, penalty,
                       rand, penalty_tokens, num_penalty):
    """orc_depformer_generate for one stream: returns (tokens [S], logits
    [S][out_vocab], hidden [S][dim])."""
    c = weights.cfg
    S = c["num_steps"]
    keep = []
    fields = {}
    for f in DepformerWeights.FIELDS:
        arr, k = _ptrs(getattr(weights, f))
        keep += k
        fields[f] = ctypes.cast(arr, _vpp)
        keep.append(arr)
    te = np.ascontiguousarray(weights.text_emb)
    keep.append(te)
    wp = DepformerWeightPtrs(text_emb=te.ctypes.data, **fields)
    cs = depformer_cfg_struct(c)
    th = np.ascontiguousarray(temporal_hidden, dtype=np.float32).reshape(-1)
    rd = np.ascontiguousarray(rand, dtype=np.float32).reshape(S)
    pt = np.zeros((S, 30), np.uint32)
    pt[:, :np.asarray(penalty_tokens).shape[-1]] = np.asarray(penalty_tokens, np.uint32).reshape(S, -1)[:, :30]
    npn = np.ascontiguousarray(num_penalty, dtype=np.uint32).reshape(S)
    tokens = np.empty(S, np.uint32)
    logits = np.empty((S, c["out_vocab"]), np.float32)
    hidden = np.empty((S, c["dim"]), np.float32)
    u32p = ctypes.POINTER(_u32)
    lib().orc_depformer_generate(ctypes.byref(cs), ctypes.byref(wp), _p32(th), int(text_token),
                                 int(top_k), float(temperature), float(penalty), _p32(rd),
                                 pt.ctypes.data_as(u32p), npn.ctypes.data_as(u32p),
                                 tokens.ctypes.data_as(u32p), _p32(logits), _p32(hidden))
    return tokens, logits, hidden
