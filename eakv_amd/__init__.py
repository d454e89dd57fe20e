"""eakv_amd — Python binding of libeakv.so (Q4_1 KV cache on MI355X).

The library is the C ABI declared in include/eakv.h (the reference eakv API,
reference include/eakv.h:14-83) and include/eakv_hip.h (device-pointer,
batched and fused extensions).  This module loads it with ctypes and offers

  * ``lib()``     the raw ctypes handle, with argtypes set for every symbol;
  * ``Cache``     an object wrapper whose methods mirror the C calls one to one
                  and take / return numpy arrays for the host-pointer calls;
  * ``EakvError`` raised for non-zero return codes and recorded errors.

There is no fallback: if libeakv.so is missing or cannot be loaded, every entry
point raises.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

EAKV_OK = 0
EAKV_ERR_IO = -1
EAKV_ERR_FORMAT = -2
EAKV_ERR_ALLOC = -3
EAKV_ERR_INVALID = -4
EAKV_ERR_DEVICE = -5

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libeakv.so")

_f32p = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)
_vp = C.c_void_p

# name -> (restype, argtypes); every symbol exported by libeakv.so
SIGNATURES = {
    # include/eakv.h
    "eakv_cache_create": (_vp, [C.c_int, C.c_int, C.c_int, C.c_int]),
    "eakv_cache_free": (None, [_vp]),
    "eakv_cache_load_raw": (C.c_int, [_vp, _vp, C.c_int]),
    "eakv_cache_append": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_int]),
    "eakv_cache_advance": (C.c_int, [_vp, C.c_int]),
    "eakv_cache_clear": (None, [_vp]),
    "eakv_checkpoint": (C.c_int, [_vp]),
    "eakv_restore": (C.c_int, [_vp, C.c_int]),
    "eakv_attention_scores": (None, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp]),
    "eakv_attention_output": (None, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp]),
    "eakv_cache_save": (C.c_int, [_vp, C.c_char_p]),
    "eakv_cache_load": (C.c_int, [C.c_char_p, C.POINTER(_vp)]),
    "eakv_cache_seq_len": (C.c_int, [_vp]),
    "eakv_cache_n_layers": (C.c_int, [_vp]),
    "eakv_cache_n_heads": (C.c_int, [_vp]),
    "eakv_cache_head_dim": (C.c_int, [_vp]),
    "eakv_cache_max_seq_len": (C.c_int, [_vp]),
    "eakv_cache_compression_ratio": (C.c_float, [_vp]),
    # include/eakv_hip.h
    "eakv_last_error": (C.c_int, []),
    "eakv_last_error_message": (C.c_char_p, []),
    "eakv_clear_error": (None, []),
    "eakv_cache_device": (C.c_int, [_vp]),
    "eakv_cache_stream": (_vp, [_vp]),
    "eakv_cache_sync": (C.c_int, [_vp]),
    "eakv_cache_read_planes": (C.c_int, [_vp, C.c_int, C.c_int, _vp, _vp, _vp]),
    "eakv_cache_load_raw_device": (C.c_int, [_vp, _vp, C.c_int, _vp]),
    "eakv_cache_append_device": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp]),
    "eakv_append_batch_device": (C.c_int, [_vp, C.c_int, _vp, C.c_int, _vp]),
    "eakv_attention_scores_device": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp, _vp]),
    "eakv_attention_output_device": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp, _vp]),
    "eakv_attention_fused": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp]),
    "eakv_attention_fused_batch_device": (
        C.c_int, [_vp, C.c_int, C.c_int, _vp, C.c_int, C.c_int, _vp, _vp]),
    "eakv_attention_fused_batch_device_noalloc": (
        C.c_int, [_vp, C.c_int, C.c_int, _vp, C.c_int, C.c_int, _vp, _vp]),
    "eakv_attention_fused_plan": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.c_int, _vp]),
    "eakv_dequantize_range_device": (
        C.c_int, [_vp, C.c_int, C.c_int, C.c_int64, C.c_int64, _vp, _vp]),
    "eakv_dequantize_range": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int64, C.c_int64, _vp]),
    "eakv_validate": (C.c_int, [_vp, _vp]),
    "eakv_ggml_quantize_row_device": (C.c_int, [_vp, _vp, C.c_int64, _vp]),
    "eakv_ggml_dequantize_row_device": (C.c_int, [_vp, _vp, C.c_int64, _vp]),
    "eakv_ggml_vec_dot_device": (C.c_int, [C.c_int, _vp, C.c_size_t, _vp, C.c_size_t, _vp,
                                           C.c_size_t, C.c_int, _vp]),
}

_LIB = None


class EakvError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"eakv error {code}: {msg}")
        self.code = code


def lib():
    """Load libeakv.so (once) and return the ctypes handle."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() "
                "(make -C eakv_amd)")
        h = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = h
    return _LIB


def last_error():
    L = lib()
    return L.eakv_last_error(), (L.eakv_last_error_message() or b"").decode()


def _check(rc: int):
    if rc != EAKV_OK:
        code, msg = last_error()
        raise EakvError(rc, msg)
    return rc


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_vp)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class Cache:
    """An eakv_cache_t* on the current HIP device.

    Methods mirror include/eakv.h (reference include/eakv.h:25-83); host
    buffers are numpy arrays.
    """

    def __init__(self, n_layers, n_kv_heads, head_dim, max_seq_len, _handle=None):
        L = lib()
        if _handle is None:
            _handle = L.eakv_cache_create(n_layers, n_kv_heads, head_dim, max_seq_len)
            if not _handle:
                code, msg = last_error()
                raise EakvError(code or EAKV_ERR_INVALID, msg or "cache_create failed")
        self.h = _handle

    # -- lifecycle
    def free(self):
        if self.h:
            lib().eakv_cache_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.free()

    # -- info
    @property
    def seq_len(self):
        return lib().eakv_cache_seq_len(self.h)

    @property
    def n_layers(self):
        return lib().eakv_cache_n_layers(self.h)

    @property
    def n_heads(self):
        return lib().eakv_cache_n_heads(self.h)

    @property
    def head_dim(self):
        return lib().eakv_cache_head_dim(self.h)

    @property
    def max_seq_len(self):
        return lib().eakv_cache_max_seq_len(self.h)

    @property
    def compression_ratio(self):
        return lib().eakv_cache_compression_ratio(self.h)

    @property
    def stream(self):
        return lib().eakv_cache_stream(self.h)

    # -- quantization
    def load_raw(self, data, seq_len):
        d = _f32(data)
        return _check(lib().eakv_cache_load_raw(self.h, _ptr(d), seq_len))

    def append(self, data, layer, kv_idx, n_tokens):
        d = _f32(data)
        return _check(lib().eakv_cache_append(self.h, _ptr(d), layer, kv_idx, n_tokens))

    def advance(self, n_tokens):
        return _check(lib().eakv_cache_advance(self.h, n_tokens))

    def clear(self):
        lib().eakv_cache_clear(self.h)

    def checkpoint(self):
        return lib().eakv_checkpoint(self.h)

    def restore(self, seq_len):
        return _check(lib().eakv_restore(self.h, seq_len))

    # -- attention (host pointers)
    def attention_scores(self, queries, layer, n_q, n_kv):
        q = _f32(queries)
        out = np.zeros((n_q, self.seq_len), np.float32)
        L = lib()
        L.eakv_clear_error()
        L.eakv_attention_scores(self.h, _ptr(q), layer, n_q, n_kv, _ptr(out))
        code, msg = last_error()
        if code:
            raise EakvError(code, msg)
        return out

    def attention_output(self, weights, layer, n_q, n_kv):
        w = _f32(weights)
        out = np.zeros((n_q, self.head_dim), np.float32)
        L = lib()
        L.eakv_clear_error()
        L.eakv_attention_output(self.h, _ptr(w), layer, n_q, n_kv, _ptr(out))
        code, msg = last_error()
        if code:
            raise EakvError(code, msg)
        return out

    def attention_fused(self, queries, layer, n_q, n_kv):
        q = _f32(queries)
        out = np.zeros((n_q, self.head_dim), np.float32)
        _check(lib().eakv_attention_fused(self.h, _ptr(q), layer, n_q, n_kv, _ptr(out)))
        return out

    # -- planes
    def read_planes(self, layer, kv_idx):
        ng = self.n_heads * self.max_seq_len * self.head_dim // 64
        w = np.zeros((ng, 32), np.uint8)
        s = np.zeros(ng, np.float32)
        b = np.zeros(ng, np.float32)
        _check(lib().eakv_cache_read_planes(self.h, layer, kv_idx, _ptr(w), _ptr(s), _ptr(b)))
        return w, s, b

    def dequantize_range(self, layer, kv_idx, group_start, group_count):
        """f32[group_count][64] of plane groups [group_start, +group_count)."""
        out = np.zeros((group_count, 64), np.float32)
        _check(lib().eakv_dequantize_range(self.h, layer, kv_idx, group_start, group_count,
                                           _ptr(out)))
        return out

    def validate(self):
        """int32[n_layers * 2]: the integrity code of every (layer, kv) block."""
        res = np.zeros(2 * self.n_layers, np.int32)
        _check(lib().eakv_validate(self.h, _ptr(res)))
        return res

    def sync(self):
        return _check(lib().eakv_cache_sync(self.h))

    # -- files
    def save(self, path):
        return _check(lib().eakv_cache_save(self.h, os.fsencode(path)))

    @classmethod
    def load(cls, path):
        out = _vp()
        _check(lib().eakv_cache_load(os.fsencode(path), C.byref(out)))
        return cls(0, 0, 0, 0, _handle=out.value)


def handles(caches):
    """ctypes array of eakv_cache_t* for the batched entry points."""
    arr = (_vp * len(caches))()
    for i, c in enumerate(caches):
        arr[i] = c.h
    return arr


FUSED_PLAN_KEYS = ("mfma", "chunks", "merge_levels", "tile_tokens", "waves_per_block",
                   "tiles_per_wave", "quads", "split")


def fused_plan(caches, n_q, n_kv, noalloc=False):
    """The launch eakv_attention_fused_batch_device (or, noalloc, its
    allocation-free form) makes for these caches at their current seq_len:
    a dict over FUSED_PLAN_KEYS (eakv_attention_fused_plan)."""
    plan = (C.c_int32 * 8)()
    _check(lib().eakv_attention_fused_plan(handles(caches), len(caches), n_q, n_kv,
                                           int(bool(noalloc)), plan))
    return dict(zip(FUSED_PLAN_KEYS, list(plan)))
