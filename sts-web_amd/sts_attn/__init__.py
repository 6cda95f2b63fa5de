"""Python view of libsts_attn.so, the MI355X attention hot path of sts-web.

This module mirrors the reference's Rust interface for the path
(crates/sts-wasm/src/model.rs of idle-intelligence/sts-web):

    fused_attention(q, k, v, scale)               model.rs:598-668
    gpu_cache_write_v(v, cache, offset, max_len)  model.rs:143-188
    KVCache / LayerCaches                          model.rs:195-411
    RoPE                                           model.rs:38-122
    Q4KTensor / q4k_matmul / Q4KLinear             gguf.rs:520-905
    DepthEngine.generate                           depth_engine.rs:884-1491

over the C ABI declared in include/sts_attn.h.  Device memory comes from
torch tensors (float32, on a ROCm device); every call goes through the HIP
library, and importing this module without the built library raises.
Errors from the library raise StsError with the library's message, the
counterpart of the reference's `.expect(...)` panics.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import torch  # loaded first so the process has one HIP runtime

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "libsts_attn.so")

STS_OK = 0
STS_ERR_INVALID = -1
STS_ERR_HIP = -2
STS_ERR_STATE = -3
STS_ERR_NOMEM = -4
STS_ERR_DEVICE = -5
DEVERR_WAIT_TIMEOUT = 1
PREC_F32 = 0
PREC_BF16_MFMA = 1
PREC_F32_SPLIT_BF16 = 2
KV_BF16_MIRROR = 1

_vp = ctypes.c_void_p
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64
_f32 = ctypes.c_float
_int = ctypes.c_int


class StsError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"sts_attn error {code}: {msg}")
        self.code = code


class KvState(ctypes.Structure):
    _fields_ = [("offset", _u64), ("len", _u64), ("write_pos", _u64), ("max_len", _u64),
                ("heads", _u64), ("head_dim", _u64), ("batch", _u64), ("allocated", ctypes.c_int32),
                ("flags", ctypes.c_int32), ("q_heads", _u64)]


# name -> (restype, argtypes); the exported set of include/sts_attn.h.
SIGNATURES = {
    "sts_last_error": (ctypes.c_char_p, []),
    "sts_abi_version": (_int, []),
    "sts_fused_attention": (_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _f32, _u64, _vp]),
    "sts_cache_write": (_int, [_vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _vp]),
    "sts_decode_ring": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _f32, _vp]),
    "sts_decode_ring_noalloc": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _f32,
                                       _vp]),
    "sts_depformer_step": (_int, [_vp, _vp, _vp, _u64, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
                                  _u32, _f32, _vp]),
    "sts_prefill_attention": (_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _f32,
                                     _int, _vp]),
    "sts_rope_create": (_int, [_u32, _u32, _f32, ctypes.POINTER(_vp)]),
    "sts_rope_destroy": (_int, [_vp]),
    "sts_rope_apply": (_int, [_vp, _vp, _u32, _u32, _u32, _u32, _vp]),
    "sts_kv_create": (_int, [_u64, _u64, _u64, ctypes.POINTER(_vp)]),
    "sts_kv_create_ex": (_int, [_u64, _u64, _u64, _u32, ctypes.POINTER(_vp)]),
    "sts_kv_mirror": (_int, [_vp, ctypes.POINTER(_vp), ctypes.POINTER(_vp)]),
    "sts_kv_sync_mirror": (_int, [_vp, _vp]),
    "sts_kv_set_query_heads": (_int, [_vp, _u64]),
    "sts_prefill_attention_bf16kv": (_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32,
                                            _u32, _f32, _vp]),
    "sts_kv_destroy": (_int, [_vp]),
    "sts_kv_ensure_allocated": (_int, [_vp, _u64, ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                                       ctypes.POINTER(_u64), _vp]),
    "sts_kv_get_state": (_int, [_vp, ctypes.POINTER(KvState)]),
    "sts_kv_window": (_int, [_vp, ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "sts_kv_advance": (_int, [_vp, _u64]),
    "sts_kv_update": (_int, [_vp, _vp, _vp, _u64, _u64, _vp]),
    "sts_kv_reset": (_int, [_vp]),
    "sts_kv_reset_keep_buffers": (_int, [_vp, _vp]),
    "sts_kv_rollback": (_int, [_vp, _u64]),
    "sts_kv_attend": (_int, [_vp, _vp, _vp, _f32, _vp]),
    "sts_kv_decode_step": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _u64, _f32, _vp]),
    "sts_kv_prefill": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _u64, _f32, _int, _vp]),
    "sts_device_errors": (_int, [_vp, ctypes.POINTER(_u32)]),
    "sts_debug_set_wait_limit": (_int, [_u32]),
    "sts_q4k_matvec": (_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _vp]),
    "sts_q4k_dequant": (_int, [_vp, _vp, _u32, _u32, _vp]),
    "sts_q4k_gemm": (_int, [_vp, _vp, _u64, _vp, _f32, _vp, _u64, _vp, _u64, _u32, _u32, _u32,
                            _int, _vp]),
    "sts_rmsnorm": (_int, [_vp, _vp, _vp, _u32, _u32, _f32, _vp]),
    "sts_embed_add_q4_0": (_int, [_vp, _u32, _vp, _u64, _vp, _vp, _u32, _u32, _vp]),
    "sts_sample_topk": (_int, [_vp, _u64, _u32, _u32, _u32, _f32, _f32, _vp, _vp, _u64, _vp,
                               _u64, _vp, _u64, _vp]),
    "sts_depformer_create": (_int, [_vp, _vp, _u32, ctypes.POINTER(_vp)]),
    "sts_depformer_destroy": (_int, [_vp]),
    "sts_depformer_generate": (_int, [_vp, _vp, _vp, _u32, _u32, _f32, _f32, _vp, _vp, _vp, _vp,
                                      _vp, _vp]),
    "sts_probe_stream_read": (_int, [_vp, _u64, _vp, _u64, _u32, _vp, _vp]),
}

_lib = None


def load():
    """Loads libsts_attn.so (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (run `make -C sts-web_amd`)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def _check(rc: int) -> None:
    if rc != STS_OK:
        msg = load().sts_last_error().decode(errors="replace")
        raise StsError(rc, msg)


def _stream(stream) -> Optional[int]:
    """hipStream_t of `stream` (a torch stream, an int handle, or None = current)."""
    if stream is None:
        if torch.cuda.is_available():
            return torch.cuda.current_stream().cuda_stream
        return None
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    if t is None:
        return None
    if t.dtype != torch.float32 and t.dtype != torch.int32:
        raise TypeError(f"expected float32/int32 tensor, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return t.data_ptr()


# ---------------------------------------------------------------------------
# Stateless ops
# ---------------------------------------------------------------------------

def fused_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
                    seq_len: Optional[int] = None, stream=None) -> torch.Tensor:
    """Decode attention, the fused_attention op (model.rs:598-668).

    q: [1, 1, H, D] (or [H, D]); k, v: [1, H, L, D] cache views -- either
    contiguous [1, H, S, D] or a [1, H, max_len, D] cache with `seq_len` valid
    rows (the head stride is taken from the tensor, as the reference reads
    k.strides[1]).  Returns [1, H, 1, D].
    """
    H, D = q.shape[-2], q.shape[-1]
    if k.dim() == 4:
        hs = k.stride(1)
        L = k.shape[2] if seq_len is None else seq_len
    else:
        hs = k.stride(0)
        L = k.shape[1] if seq_len is None else seq_len
    if k.stride(-1) != 1 or k.stride(-2) != D or v.stride() != k.stride():
        raise ValueError("k/v rows must be contiguous with identical strides")
    out = torch.empty((1, H, 1, D), dtype=torch.float32, device=q.device)
    _check(load().sts_fused_attention(_ptr(q.contiguous()), k.data_ptr(), v.data_ptr(), _ptr(out),
                                      H, D, L, scale, hs, _stream(stream)))
    return out


def gpu_cache_write_v(v: torch.Tensor, cache: torch.Tensor, offset: int, max_len: int,
                      stream=None) -> None:
    """Ring append, gpu_cache_write_v (model.rs:143-188): v [B,S,H,D] -> cache [B,H,M,D]."""
    B, S, H, D = v.shape
    if cache.numel() < B * H * max_len * D:
        raise ValueError("cache smaller than [B, H, max_len, D]")
    _check(load().sts_cache_write(_ptr(v.contiguous()), _ptr(cache), offset, B, S, H, D, max_len,
                                  _stream(stream)))


def decode_ring(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                lens: torch.Tensor, starts: torch.Tensor, scale: float,
                out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Ragged multi-stream decode; q [B,H,D], caches [B,H,M,D], lens/starts int32 [B]."""
    B, H, M, D = k_cache.shape
    if out is None:
        out = torch.empty((B, H, D), dtype=torch.float32, device=q.device)
    _check(load().sts_decode_ring(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), _ptr(lens),
                                  _ptr(starts), B, H, D, M, scale, _stream(stream)))
    return out


def depformer_step(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                   k_cache: torch.Tensor, v_cache: torch.Tensor, step: int, scale: float,
                   out: Optional[torch.Tensor] = None, qkv_stride: Optional[int] = None,
                   stream=None) -> torch.Tensor:
    """Batched depformer step (append at slot `step`, attend slots 0..step).

    q, k_new, v_new: [B, H, D] views whose stream stride is `qkv_stride`
    elements (default H*D); caches [B, H, max_len, D].
    """
    B, H, M, D = k_cache.shape
    if qkv_stride is None:
        qkv_stride = q.stride(0)
    if out is None:
        out = torch.empty((B, H, D), dtype=torch.float32, device=k_cache.device)
    _check(load().sts_depformer_step(q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), qkv_stride,
                                     _ptr(k_cache), _ptr(v_cache), _ptr(out), B, H, D, M, step,
                                     scale, _stream(stream)))
    return out


def prefill_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                      win_start: int, win_len: int, scale: float, precision: int = PREC_F32,
                      out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Causal chunk attention; q [S,H,D], caches [H,M,D] (or [1,H,M,D])."""
    S, H, D = q.shape
    M = k_cache.shape[-2]
    if out is None:
        out = torch.empty_like(q)
    _check(load().sts_prefill_attention(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), S, H, D,
                                        M, win_start, win_len, scale, precision, _stream(stream)))
    return out


def prefill_attention_bf16kv(q: torch.Tensor, k16: torch.Tensor, v16: torch.Tensor,
                             win_start: int, win_len: int, scale: float,
                             out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Causal chunk attention (bf16 MFMA) over bf16 copies of the caches: q [S,H,D]
    f32, k16/v16 [H,M,D] (or [1,H,M,D]) torch.bfloat16 or int16 bit patterns."""
    S, H, D = q.shape
    M = k16.shape[-2]
    for t in (k16, v16):
        if t.dtype not in (torch.bfloat16, torch.int16) or not t.is_contiguous():
            raise ValueError("k16/v16 must be contiguous bfloat16 (or int16 bits)")
    if out is None:
        out = torch.empty_like(q)
    _check(load().sts_prefill_attention_bf16kv(_ptr(q), k16.data_ptr(), v16.data_ptr(), _ptr(out),
                                               S, H, D, M, win_start, win_len, scale,
                                               _stream(stream)))
    return out


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------

# Handles whose Python object was released while the current stream was being
# captured into a graph: destroying them then would free device memory inside
# the capture (which invalidates it), so they are destroyed by the next handle
# release or creation outside a capture.
_deferred = []


def _capturing() -> bool:
    try:
        return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()
    except Exception:
        return False


def _release(destroy, handle) -> None:
    """Destroys `handle` with `destroy` (a library entry point), or defers it
    while the current stream is being captured; runs deferred ones when it can."""
    if _capturing():
        _deferred.append((destroy, handle))
        return
    while _deferred:
        d, h = _deferred.pop()
        getattr(load(), d)(h)
    getattr(load(), destroy)(handle)


def _drain_deferred() -> None:
    if _deferred and not _capturing():
        while _deferred:
            d, h = _deferred.pop()
            getattr(load(), d)(h)


class RoPE:
    """RoPE::new / apply (model.rs:44-121) with tables held by the library."""

    def __init__(self, head_dim: int, max_seq_len: int, theta: float = 10000.0):
        _drain_deferred()
        h = _vp()
        _check(load().sts_rope_create(head_dim, max_seq_len, theta, ctypes.byref(h)))
        self._h = h
        self.head_dim = head_dim
        self.max_seq_len = max_seq_len

    @property
    def handle(self):
        return self._h

    def apply_(self, x: torch.Tensor, offset: int, stream=None) -> torch.Tensor:
        """Rotates x [B,S,H,D] in place at positions offset.. and returns it."""
        B, S, H, D = x.shape
        _check(load().sts_rope_apply(self._h, _ptr(x), B, S, H, offset, _stream(stream)))
        return x

    def apply(self, q: torch.Tensor, k: torch.Tensor, offset: int, stream=None):
        """Rotated copies of q and k, RoPE::apply (model.rs:111-120)."""
        return (self.apply_(q.contiguous().clone(), offset, stream),
                self.apply_(k.contiguous().clone(), offset, stream))

    def close(self):
        if self._h:
            _release("sts_rope_destroy", self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# KV cache
# ---------------------------------------------------------------------------

class KVCache:
    """Ring-buffer KV cache in HBM, KVCache (model.rs:195-363)."""

    def __init__(self, max_len: int, n_kv_heads: int, head_dim: int, bf16_mirror: bool = False,
                 n_heads: Optional[int] = None):
        """n_heads: query heads when they outnumber the K/V heads (grouped-query
        attention, model.rs:766-783); q and out then have n_heads heads."""
        _drain_deferred()
        h = _vp()
        _check(load().sts_kv_create_ex(max_len, n_kv_heads, head_dim,
                                       KV_BF16_MIRROR if bf16_mirror else 0, ctypes.byref(h)))
        self._h = h
        self.n_kv_heads = n_kv_heads
        self.n_heads = n_heads or n_kv_heads
        self.head_dim = head_dim
        if self.n_heads != n_kv_heads:
            _check(load().sts_kv_set_query_heads(h, self.n_heads))

    @property
    def handle(self):
        return self._h

    def state(self) -> KvState:
        s = KvState()
        _check(load().sts_kv_get_state(self._h, ctypes.byref(s)))
        return s

    def max_len(self) -> int:
        return self.state().max_len

    def offset(self) -> int:
        return self.state().offset

    def seq_len(self) -> int:
        return self.state().len

    def write_pos(self) -> int:
        return self.state().write_pos

    def window(self):
        st, ln = _u64(), _u64()
        _check(load().sts_kv_window(self._h, ctypes.byref(st), ctypes.byref(ln)))
        return st.value, ln.value

    def ensure_allocated(self, batch: int, stream=None):
        """Allocates the buffers if needed; returns (k_ptr, v_ptr, write_pos)."""
        kp, vp, wp = _vp(), _vp(), _u64()
        _check(load().sts_kv_ensure_allocated(self._h, batch, ctypes.byref(kp), ctypes.byref(vp),
                                              ctypes.byref(wp), _stream(stream)))
        return kp.value, vp.value, wp.value

    def read_buffers(self):
        """Copies of the K and V buffers as torch tensors [B, H, max_len, D]."""
        s = self.state()
        if not s.allocated:
            return None, None
        kp, vp, _ = self.ensure_allocated(s.batch)
        shape = (s.batch, s.heads, s.max_len, s.head_dim)
        return copy_device(kp, shape), copy_device(vp, shape)

    def mirror_buffers(self):
        """Copies of the bf16 mirror [B, H, max_len, D] (torch.int16 bit patterns),
        or (None, None) when there is none."""
        s = self.state()
        kp, vp = _vp(), _vp()
        _check(load().sts_kv_mirror(self._h, ctypes.byref(kp), ctypes.byref(vp)))
        if not kp.value:
            return None, None
        shape = (s.batch, s.heads, s.max_len, s.head_dim)
        return (copy_device(kp.value, shape, torch.int16),
                copy_device(vp.value, shape, torch.int16))

    def sync_mirror(self, stream=None) -> None:
        _check(load().sts_kv_sync_mirror(self._h, _stream(stream)))

    def advance(self, num_steps: int) -> None:
        _check(load().sts_kv_advance(self._h, num_steps))

    def update(self, k: torch.Tensor, v: torch.Tensor, stream=None) -> None:
        """Appends k, v [B, S, H, D] at (offset + s) % max_len and advances S."""
        B, S, H, D = k.shape
        _check(load().sts_kv_update(self._h, _ptr(k.contiguous()), _ptr(v.contiguous()), B, S,
                                    _stream(stream)))

    def reset(self) -> None:
        _check(load().sts_kv_reset(self._h))

    def reset_keep_buffers(self, stream=None) -> None:
        _check(load().sts_kv_reset_keep_buffers(self._h, _stream(stream)))

    def rollback(self, n: int) -> None:
        _check(load().sts_kv_rollback(self._h, n))

    def attend(self, q: torch.Tensor, scale: float, out: Optional[torch.Tensor] = None,
               stream=None) -> torch.Tensor:
        """Decode attention over the current window; q [B, H, D] -> [B, H, D]."""
        if out is None:
            out = torch.empty_like(q)
        _check(load().sts_kv_attend(self._h, _ptr(q.contiguous()), _ptr(out), scale,
                                    _stream(stream)))
        return out

    def decode_step(self, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                    scale: float, rope: Optional[RoPE] = None,
                    out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
        """Fused RoPE + append + advance(1) + attend; tensors [B, H, D]."""
        B = q.shape[0]
        if out is None:
            out = torch.empty_like(q)
        _check(load().sts_kv_decode_step(self._h, rope.handle if rope is not None else None,
                                         _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(out), B, scale,
                                         _stream(stream)))
        return out

    def prefill(self, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, scale: float,
                precision: int = PREC_F32, rope: Optional[RoPE] = None,
                out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
        """Appends S rows and runs causal chunk attention; tensors [S, H, D].
        With `rope`, q and k_new are unrotated and rotated at offset..offset+S-1
        (the prefill branch, model.rs:760-797)."""
        S = q.shape[0]
        if out is None:
            out = torch.empty_like(q)
        _check(load().sts_kv_prefill(self._h, rope.handle if rope is not None else None, _ptr(q),
                                     _ptr(k_new), _ptr(v_new), _ptr(out), S, scale, precision,
                                     _stream(stream)))
        return out

    def close(self):
        if self._h:
            _release("sts_kv_destroy", self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class LayerCaches:
    """One KVCache per layer, LayerCaches (model.rs:365-411)."""

    def __init__(self, n_layers: int, max_len: int, n_kv_heads: int, head_dim: int,
                 n_heads: Optional[int] = None):
        self.caches = [KVCache(max_len, n_kv_heads, head_dim, n_heads=n_heads)
                       for _ in range(n_layers)]

    def get_mut(self, layer: int) -> Optional[KVCache]:
        return self.caches[layer] if 0 <= layer < len(self.caches) else None

    def seq_len(self) -> int:
        return self.caches[0].seq_len() if self.caches else 0

    def reset(self) -> None:
        for c in self.caches:
            c.reset()

    def reset_keep_buffers(self, stream=None) -> None:
        for c in self.caches:
            c.reset_keep_buffers(stream)

    def rollback(self, n: int) -> None:
        for c in self.caches:
            c.rollback(n)


_hiprt = None


def _hip():
    """The HIP runtime already loaded in this process (torch's), via its soname."""
    global _hiprt
    if _hiprt is None:
        rt = ctypes.CDLL("libamdhip64.so.7")
        rt.hipMemcpy.argtypes = [_vp, _vp, ctypes.c_size_t, ctypes.c_int]
        rt.hipMemcpy.restype = ctypes.c_int
        _hiprt = rt
    return _hiprt


def copy_device(ptr: int, shape: Sequence[int], dtype=torch.float32) -> torch.Tensor:
    """A torch copy of `shape` elements of `dtype` at device address `ptr`."""
    t = torch.empty(tuple(shape), dtype=dtype, device="cuda")
    torch.cuda.synchronize()
    rc = _hip().hipMemcpy(t.data_ptr(), ptr, t.numel() * t.element_size(), 3)  # device to device
    if rc != 0:
        raise StsError(STS_ERR_HIP, f"hipMemcpy failed with code {rc}")
    return t


def device_errors(stream=None) -> int:
    """Synchronises `stream`, reads and clears the device error word; raises
    StsError (STS_ERR_DEVICE) when a kernel raised a flag, else returns 0."""
    flags = _u32()
    _check(load().sts_device_errors(_stream(stream), ctypes.byref(flags)))
    return flags.value


def take_device_errors(stream=None) -> int:
    """The device error flags (read and cleared) without raising."""
    flags = _u32()
    rc = load().sts_device_errors(_stream(stream), ctypes.byref(flags))
    if rc not in (STS_OK, STS_ERR_DEVICE):
        _check(rc)
    return flags.value


def set_wait_limit(polls: int) -> None:
    """Test hook: polls after which the kernels' bounded waits give up (0 = default)."""
    _check(load().sts_debug_set_wait_limit(polls))


def probe_stream_read(a: torch.Tensor, b: Optional[torch.Tensor], workgroups: int,
                      sink: torch.Tensor, stream=None) -> None:
    """Plain-read roofline probe: reads a and b once (16-byte nontemporal
    loads, `workgroups` workgroups of 256 threads); one float per workgroup
    goes to sink."""
    _check(load().sts_probe_stream_read(_ptr(a), a.numel() * a.element_size(), _ptr(b),
                                        0 if b is None else b.numel() * b.element_size(),
                                        workgroups, _ptr(sink), _stream(stream)))


def softmax_scale(head_dim: int) -> float:
    """head_dim^-0.5 as the reference computes it in f32 (model.rs:705)."""
    import numpy as np
    return float(np.float32(head_dim) ** np.float32(-0.5))


# ---------------------------------------------------------------------------
# Q4_K projections (gguf.rs:520-625, 808-905)
# ---------------------------------------------------------------------------

Q4K_BLOCK_BYTES = 144
QK_K = 256
GEMM_MAX_K = 16384  # sts_q4k_gemm's largest k (above 4096 as summed slices of 4096)


class Q4KTensor:
    """A Q4_K weight matrix [n, k] on the GPU, as Q4KTensor::from_q4k_bytes
    (gguf.rs:530-563) holds it: the raw GGUF bytes, n*k/256 blocks of 144."""

    def __init__(self, raw: torch.Tensor, shape: Sequence[int]):
        n, k = int(shape[0]), int(shape[1])
        if (n * k) % QK_K != 0:
            raise StsError(STS_ERR_INVALID,
                           f"Q4_K requires element count divisible by 256, got {n * k}")
        expected = n * k // QK_K * Q4K_BLOCK_BYTES
        if raw.dtype != torch.uint8 or raw.numel() != expected:
            raise StsError(STS_ERR_INVALID, f"Q4_K byte count mismatch: expected {expected} "
                           f"uint8 bytes for {n * k // QK_K} blocks, got {raw.numel()}")
        self.raw = raw.contiguous()
        self._shape = (n, k)

    @classmethod
    def from_q4k_bytes(cls, raw_bytes, shape: Sequence[int], device="cuda") -> "Q4KTensor":
        t = torch.as_tensor(raw_bytes, dtype=torch.uint8).reshape(-1).to(device)
        return cls(t, shape)

    def shape(self):
        return self._shape

    def num_blocks(self) -> int:
        return self._shape[0] * self._shape[1] // QK_K

    def dequant(self, stream=None) -> torch.Tensor:
        """[n, k] f32 weights, rounded as the reference shader computes them."""
        n, k = self._shape
        out = torch.empty((n, k), dtype=torch.float32, device=self.raw.device)
        _check(load().sts_q4k_dequant(self.raw.data_ptr(), _ptr(out), k, n, _stream(stream)))
        return out


def q4k_matmul(input: torch.Tensor, weights: Q4KTensor, residual: Optional[torch.Tensor] = None,
               out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """q4k_matmul / q4k_matmul_with_residual (gguf.rs:808-905): input
    [B, M, K] (or [B, K]) -> [B, M, N] = input @ W^T (+ residual).  M = 1 runs
    the matvec (the reference's single-token path), M > 1 the GEMM (its
    prefill path; K above 4096, the temporal FFN's linear_out at 11264, as
    summed slices)."""
    n, k = weights.shape()
    if input.shape[-1] != k:
        raise StsError(STS_ERR_INVALID,
                       f"K dimension mismatch: input has {input.shape[-1]}, weights have {k}")
    B = input.shape[0] if input.dim() >= 2 else 1
    Mrows = input.shape[1] if input.dim() == 3 else 1
    x = input.reshape(B * Mrows, k).contiguous()
    if out is None:
        out = torch.empty((B, Mrows, n), dtype=torch.float32, device=input.device)
    res = None
    if residual is not None:
        res = residual.reshape(B * Mrows, n).contiguous()
    if Mrows == 1 or k > GEMM_MAX_K:
        _check(load().sts_q4k_matvec(weights.raw.data_ptr(), _ptr(x), _ptr(res), _ptr(out),
                                     B * Mrows, k, n, _stream(stream)))
    else:
        _check(load().sts_q4k_gemm(weights.raw.data_ptr(), _ptr(x), k, None, 0.0, _ptr(res), n,
                                   _ptr(out), n, B * Mrows, k, n, 0, _stream(stream)))
    return out


def q4k_matmul_with_residual(input: torch.Tensor, weights: Q4KTensor, residual: torch.Tensor,
                             stream=None) -> torch.Tensor:
    """output = matmul(input, weights) + residual (gguf.rs:899-905), one launch."""
    return q4k_matmul(input, weights, residual=residual, stream=stream)


class Q4KLinear:
    """Q4KLinear (gguf.rs:595-625): Q4_K weights with an optional f32 bias."""

    def __init__(self, weights: Q4KTensor, bias: Optional[torch.Tensor] = None):
        self.weights = weights
        self.bias = bias

    def forward(self, x: torch.Tensor, stream=None) -> torch.Tensor:
        out = q4k_matmul(x, self.weights, stream=stream)
        return out if self.bias is None else out + self.bias

    def forward_with_residual(self, x: torch.Tensor, residual: torch.Tensor,
                              stream=None) -> torch.Tensor:
        out = q4k_matmul_with_residual(x, self.weights, residual, stream=stream)
        return out if self.bias is None else out + self.bias


# ---------------------------------------------------------------------------
# Depformer step chain (depth_engine.rs:884-1491), batched over streams
# ---------------------------------------------------------------------------

def q4k_gemm(x: torch.Tensor, weights: Q4KTensor, residual: Optional[torch.Tensor] = None,
             swiglu: bool = False, norm_alpha: Optional[torch.Tensor] = None,
             norm_eps: float = 0.0, out: Optional[torch.Tensor] = None,
             stream=None) -> torch.Tensor:
    """x [R, K] -> [R, N] = x @ W^T (+ residual); with swiglu, W has 2F rows and
    the result is silu(G[:, :F]) * G[:, F:] ([R, F]); with norm_alpha, x is
    RMS-normalised first."""
    n, k = weights.shape()
    R = x.shape[0]
    x = x.reshape(R, k).contiguous()
    nout = n // 2 if swiglu else n
    if out is None:
        out = torch.empty((R, nout), dtype=torch.float32, device=x.device)
    res = residual.reshape(R, n).contiguous() if residual is not None else None
    _check(load().sts_q4k_gemm(weights.raw.data_ptr(), _ptr(x), k, _ptr(norm_alpha), norm_eps,
                               _ptr(res), n, _ptr(out), nout, R, k, n, 1 if swiglu else 0,
                               _stream(stream)))
    return out


def rmsnorm(x: torch.Tensor, alpha: torch.Tensor, eps: float,
            out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """shader_rmsnorm.wgsl on every row of x [..., D]."""
    D = x.shape[-1]
    x = x.contiguous()
    if out is None:
        out = torch.empty_like(x)
    _check(load().sts_rmsnorm(_ptr(x), _ptr(alpha.contiguous()), _ptr(out), x.numel() // D, D,
                              eps, _stream(stream)))
    return out


def embed_add_q4_0(table: torch.Tensor, vocab: int, tokens: torch.Tensor, proj: torch.Tensor,
                   out: Optional[torch.Tensor] = None, tok_stride: int = 1,
                   stream=None) -> torch.Tensor:
    """proj [B, D] + the Q4_0 embedding rows of tokens (uint32 device tensor)."""
    B, D = proj.shape
    if out is None:
        out = torch.empty_like(proj)
    _check(load().sts_embed_add_q4_0(table.data_ptr(), vocab, tokens.data_ptr(), tok_stride,
                                     _ptr(proj.contiguous()), _ptr(out), B, D, _stream(stream)))
    return out


def sample_top_k(logits: torch.Tensor, top_k: int, temperature: float, penalty: float,
                 rand: torch.Tensor, penalty_tokens: torch.Tensor, num_penalty: torch.Tensor,
                 out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """shader_sample_topk.wgsl for each row of logits [B, V]: rand [B] f32,
    penalty_tokens [B, 30] and num_penalty [B] uint32 -> tokens [B] uint32."""
    B, V = logits.shape
    if out is None:
        out = torch.empty(B, dtype=torch.uint32, device=logits.device)
    _check(load().sts_sample_topk(_ptr(logits.contiguous()), V, B, V, top_k, temperature,
                                  penalty, _ptr(rand), penalty_tokens.data_ptr(),
                                  penalty_tokens.stride(0), num_penalty.data_ptr(), 1,
                                  out.data_ptr(), 1, _stream(stream)))
    return out


class DepformerConfig(ctypes.Structure):
    """DepthEngineConfig (depth_engine.rs:50-107)."""
    _fields_ = [(n, _u32) for n in (
        "num_steps", "num_layers", "dim", "num_heads", "ffn", "temporal_dim", "out_vocab",
        "text_emb_vocab", "audio_emb_vocab", "num_audio_emb", "kv_max_len")] + [
        ("rms_eps", _f32), ("attn_scale", _f32)]

    @classmethod
    def personaplex(cls, num_steps: int = 8) -> "DepformerConfig":
        """DepthEngineConfig::from_sts_config of the default StsConfig
        (lib.rs:123-170, depth_engine.rs:86-107)."""
        return cls(num_steps=num_steps, num_layers=6, dim=1024, num_heads=16, ffn=2816,
                   temporal_dim=4096, out_vocab=2048, text_emb_vocab=32001,
                   audio_emb_vocab=2049, num_audio_emb=15, kv_max_len=9, rms_eps=1e-8,
                   attn_scale=float((1024 / 16) ** -0.5))


_vpp = ctypes.POINTER(_vp)


class DepformerWeightPtrs(ctypes.Structure):
    _fields_ = [("input_proj", _vpp), ("attn_in_proj", _vpp), ("attn_out_proj", _vpp),
                ("ffn_linear_in", _vpp), ("ffn_linear_out", _vpp), ("norm1_alpha", _vpp),
                ("norm2_alpha", _vpp), ("output_linear", _vpp), ("text_emb", _vp),
                ("audio_emb", _vpp)]


class DepthEngine:
    """DepthEngine (depth_engine.rs:177-1510) for a batch of streams.

    `weights` maps each field of sts_depformer_weights to device tensors:
    uint8 Q4_K/Q4_0 bytes for the matrices and tables (lists, indexed as the
    header documents), float32 alphas per layer.  The tensors must outlive the
    engine."""

    LIST_FIELDS = ("input_proj", "attn_in_proj", "attn_out_proj", "ffn_linear_in",
                   "ffn_linear_out", "norm1_alpha", "norm2_alpha", "output_linear", "audio_emb")

    def __init__(self, config: DepformerConfig, weights: dict, max_batch: int):
        self.config = config
        self.max_batch = max_batch
        self._weights = weights
        arrays = {}
        self._keep = []
        for f in self.LIST_FIELDS:
            arr = (_vp * len(weights[f]))(*[t.data_ptr() for t in weights[f]])
            self._keep.append(arr)
            arrays[f] = ctypes.cast(arr, _vpp)
        wp = DepformerWeightPtrs(text_emb=weights["text_emb"].data_ptr(), **arrays)
        h = _vp()
        _check(load().sts_depformer_create(ctypes.byref(config), ctypes.byref(wp), max_batch,
                                           ctypes.byref(h)))
        self._h = h

    def generate(self, temporal_hidden: torch.Tensor, text_token: torch.Tensor, audio_temp: float,
                 audio_top_k: int, audio_penalty: float, rand: torch.Tensor,
                 penalty_tokens: torch.Tensor, num_penalty: torch.Tensor,
                 tokens: Optional[torch.Tensor] = None, logits: Optional[torch.Tensor] = None,
                 stream=None) -> torch.Tensor:
        """DepthEngine::generate (depth_engine.rs:884-1441) for B streams:
        temporal_hidden [B, temporal_dim], text_token [B] uint32, rand
        [B, num_steps] f32, penalty_tokens [B, num_steps, 30] and num_penalty
        [B, num_steps] uint32 -> tokens [B, num_steps] uint32 (on the device,
        not read back).  logits, if given, [num_steps, B, out_vocab] f32."""
        B = temporal_hidden.shape[0]
        S = self.config.num_steps
        if tokens is None:
            tokens = torch.empty((B, S), dtype=torch.uint32, device=temporal_hidden.device)
        _check(load().sts_depformer_generate(
            self._h, _ptr(temporal_hidden.contiguous()), text_token.data_ptr(), B, audio_top_k,
            audio_temp, audio_penalty, _ptr(rand), penalty_tokens.data_ptr(),
            num_penalty.data_ptr(), tokens.data_ptr(), _ptr(logits), _stream(stream)))
        return tokens

    def close(self):
        if getattr(self, "_h", None):
            _check(load().sts_depformer_destroy(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
