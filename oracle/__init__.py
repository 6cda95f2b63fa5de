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
        "orc_kv_init": (None, [ctypes.POINTER(KvState), _u64]),
        "orc_kv_advance": (None, [ctypes.POINTER(KvState), _u64]),
        "orc_kv_update": (None, [ctypes.POINTER(KvState)]),
        "orc_kv_reset": (None, [ctypes.POINTER(KvState)]),
        "orc_kv_rollback": (None, [ctypes.POINTER(KvState), _u64]),
        "orc_attention_wgsl": (None, [_f32p, _f32p, _f32p, _f32p, _u32, _u32, _u32,
                                      ctypes.c_float, _u64]),
        "orc_attention_ring_wgsl": (None, [_f32p, _f32p, _f32p, _f32p, _u32, _u32, _u32,
                                           _u32, _u32, ctypes.c_float]),
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
        "orc_num_threads": (ctypes.c_int, []),
        "orc_set_num_threads": (None, [ctypes.c_int]),
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
