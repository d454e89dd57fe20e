"""ctypes binding of the CPU oracle (liboracle.so) — TEST INFRASTRUCTURE ONLY.

Loaded by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg as
the oracle the HIP results are compared against; never by the eakv_amd
package.  ``OracleCache`` offers the same
methods as ``eakv_amd.Cache`` so one test body can drive either.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libggml_ref.so")
REF_AVX512_PATH = os.path.join(HERE, "_ref", "libggml_ref_avx512.so")

_vp = C.c_void_p
_i64 = C.c_int64

_SIG = {
    "orc_quantize_split": (None, [_vp, _vp, _vp, _vp, _i64]),
    "orc_reduce16": (C.c_float, [_vp]),
    "orc_dequantize": (None, [_vp, _vp, _vp, _vp, _i64]),
    "orc_dequantize_range": (None, [_vp, _vp, _vp, _vp, _i64, _i64]),
    "orc_validate": (C.c_int32, [_vp, _vp, _i64]),
    "orc_ggml_quantize_row": (None, [_vp, _vp, _i64]),
    "orc_ggml_dequantize_row": (None, [_vp, _vp, _i64]),
    "orc_ggml_vec_dot": (None, [C.c_int, _vp, C.c_size_t, _vp, C.c_size_t, _vp, C.c_size_t,
                                C.c_int]),
    "orc_to_i32": (C.c_int32, [C.c_float]),
    "orc_k_score_mha": (None, [C.c_int, _vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int, _i64]),
    "orc_k_score_gqa": (None, [C.c_int, _vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, _i64]),
    "orc_v_sum_mha": (None, [C.c_int, _vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int, _i64]),
    "orc_v_sum_gqa": (None, [C.c_int, _vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, _i64]),
    "orc_fused_attention": (None, [C.c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                   C.c_int, C.c_int, C.c_int, _i64]),
    "orc_softmax_rows": (None, [_vp, _vp, C.c_int, C.c_int]),
    "orc_cache_create": (_vp, [C.c_int] * 4),
    "orc_cache_free": (None, [_vp]),
    "orc_cache_load_raw": (C.c_int, [_vp, _vp, C.c_int]),
    "orc_cache_append": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_int]),
    "orc_cache_advance": (C.c_int, [_vp, C.c_int]),
    "orc_cache_clear": (None, [_vp]),
    "orc_checkpoint": (C.c_int, [_vp]),
    "orc_restore": (C.c_int, [_vp, C.c_int]),
    "orc_attention_scores": (None, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp]),
    "orc_attention_output": (None, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp]),
    "orc_attention_fused": (None, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp]),
    "orc_attention_fused_avx512": (None, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp]),
    "orc_attention_scores_avx512": (None, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp]),
    "orc_attention_output_avx512": (None, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp]),
    "orc_avx512_available": (C.c_int, []),
    "orc_cache_seq_len": (C.c_int, [_vp]),
    "orc_cache_n_layers": (C.c_int, [_vp]),
    "orc_cache_n_heads": (C.c_int, [_vp]),
    "orc_cache_head_dim": (C.c_int, [_vp]),
    "orc_cache_max_seq_len": (C.c_int, [_vp]),
    "orc_cache_compression_ratio": (C.c_float, [_vp]),
    "orc_cache_weights": (_vp, [_vp, C.c_int, C.c_int]),
    "orc_cache_scales": (_vp, [_vp, C.c_int, C.c_int]),
    "orc_cache_biases": (_vp, [_vp, C.c_int, C.c_int]),
    "orc_cache_max_groups": (_i64, [_vp]),
    "orc_cache_save": (C.c_int, [_vp, C.c_char_p]),
    "orc_cache_load": (C.c_int, [C.c_char_p, C.POINTER(_vp)]),
}

_LIB = None
_REF = None


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} not built (make -C oracle)")
        h = C.CDLL(LIB_PATH)
        for n, (r, a) in _SIG.items():
            f = getattr(h, n)
            f.restype, f.argtypes = r, a
        _LIB = h
    return _LIB


def _cpu_has_avx512():
    try:
        flags = open("/proc/cpuinfo").read()
    except OSError:
        return False
    return all(f in flags for f in ("avx512f", "avx512bw", "avx512vl", "avx512dq"))


_REF_AVX = None


def ref_lib(avx512=False):
    """The reference's own src/ggml_type.c, built by `make -C oracle ref`:
    its scalar paths, or (avx512=True) its AVX-512 paths, the latter only on
    a CPU with AVX-512 (None when not built or not runnable)."""
    global _REF, _REF_AVX
    if avx512:
        if _REF_AVX is None and os.path.exists(REF_AVX512_PATH) and _cpu_has_avx512():
            _REF_AVX = _bind_ref(C.CDLL(REF_AVX512_PATH))
        return _REF_AVX
    if _REF is None and os.path.exists(REF_LIB_PATH):
        _REF = _bind_ref(C.CDLL(REF_LIB_PATH))
    return _REF


def _bind_ref(h):
    h.eakv_quantize_row.restype = None
    h.eakv_quantize_row.argtypes = [_vp, _vp, C.c_int64]
    h.eakv_dequantize_row.restype = None
    h.eakv_dequantize_row.argtypes = [_vp, _vp, C.c_int64]
    h.eakv_vec_dot_q4_f32.restype = None
    h.eakv_vec_dot_q4_f32.argtypes = [C.c_int, _vp, C.c_size_t, _vp, C.c_size_t,
                                      _vp, C.c_size_t, C.c_int]
    return h


def _p(a):
    return a.ctypes.data_as(_vp)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- kernels

def quantize(x):
    """x: f32[..., 64*n] -> (weights u8[n,32], scales f32[n], biases f32[n])."""
    x = _f32(x).reshape(-1)
    assert x.size % 64 == 0
    n = x.size // 64
    w = np.zeros((n, 32), np.uint8)
    s = np.zeros(n, np.float32)
    b = np.zeros(n, np.float32)
    lib().orc_quantize_split(_p(x), _p(w), _p(s), _p(b), n)
    return w, s, b


def dequantize(w, s, b):
    """Groups -> f32[n, 64], value j = fma(nibble_j, scale, bias)."""
    w = np.ascontiguousarray(w, np.uint8).reshape(-1, 32)
    n = w.shape[0]
    out = np.zeros((n, 64), np.float32)
    lib().orc_dequantize(_p(w), _p(_f32(s)), _p(_f32(b)), _p(out), n)
    return out


def dequantize_range(w, s, b, group_start, group_count):
    """Plane groups [group_start, +group_count) -> f32[group_count, 64]."""
    w = np.ascontiguousarray(w, np.uint8).reshape(-1, 32)
    out = np.zeros((group_count, 64), np.float32)
    lib().orc_dequantize_range(_p(w), _p(_f32(s)), _p(_f32(b)), _p(out), group_start,
                               group_count)
    return out


def validate(s, b, n_groups):
    """Integrity code of groups 0..n_groups-1 (0 ok, 1 NaN scale, 2 NaN bias,
    3 negative scale)."""
    return int(lib().orc_validate(_p(_f32(s)), _p(_f32(b)), n_groups))


def ggml_quantize_row(x):
    """f32[k] (k % 64 == 0) -> u8[k/64, 40] blocks (qs[32], d, m)."""
    x = _f32(x).reshape(-1)
    out = np.zeros((x.size // 64, 40), np.uint8)
    lib().orc_ggml_quantize_row(_p(x), _p(out), x.size)
    return out


def ggml_dequantize_row(blocks):
    """u8[nb, 40] blocks -> f32[nb*64]."""
    blocks = np.ascontiguousarray(blocks, np.uint8).reshape(-1, 40)
    out = np.zeros(blocks.shape[0] * 64, np.float32)
    lib().orc_ggml_dequantize_row(_p(blocks), _p(out), out.size)
    return out


def ggml_vec_dot(blocks, y):
    """Row r of blocks (u8[nrc, nb*40]) dotted with row r of y (f32[nrc, nb*64])."""
    blocks = np.ascontiguousarray(blocks, np.uint8)
    y = _f32(y)
    nrc, n = y.shape
    s = np.zeros(nrc, np.float32)
    lib().orc_ggml_vec_dot(n, _p(s), 4, _p(blocks), blocks.shape[1], _p(y), n * 4, nrc)
    return s


def k_score(head_dim, q, w, s, b, seq_len, n_q, n_kv, gph):
    q = _f32(q)
    out = np.zeros((n_q, seq_len), np.float32)
    lib().orc_k_score_gqa(head_dim, _p(q), _p(w), _p(_f32(s)), _p(_f32(b)), _p(out),
                          seq_len, n_q, n_kv, gph)
    return out


def v_sum(head_dim, wts, w, s, b, seq_len, n_q, n_kv, gph):
    wts = _f32(wts)
    out = np.zeros((n_q, head_dim), np.float32)
    lib().orc_v_sum_gqa(head_dim, _p(wts), _p(w), _p(_f32(s)), _p(_f32(b)), _p(out),
                        seq_len, n_q, n_kv, gph)
    return out


def avx512_available():
    """Whether this CPU runs the AVX-512 restatement of the fused kernel."""
    return bool(lib().orc_avx512_available())


def softmax_rows(scores):
    sc = _f32(scores)
    n, L = sc.shape
    out = np.zeros_like(sc)
    lib().orc_softmax_rows(_p(sc), _p(out), n, L)
    return out


# ---------------------------------------------------------------- cache

class OracleCache:
    """Host-memory cache: restatement of reference src/cache.c, attention.c."""

    def __init__(self, n_layers, n_kv_heads, head_dim, max_seq_len, _handle=None):
        L = lib()
        if _handle is None:
            _handle = L.orc_cache_create(n_layers, n_kv_heads, head_dim, max_seq_len)
            if not _handle:
                raise ValueError("orc_cache_create: invalid shape")
        self.h = _handle

    def free(self):
        if self.h:
            lib().orc_cache_free(self.h)
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

    seq_len = property(lambda self: lib().orc_cache_seq_len(self.h))
    n_layers = property(lambda self: lib().orc_cache_n_layers(self.h))
    n_heads = property(lambda self: lib().orc_cache_n_heads(self.h))
    head_dim = property(lambda self: lib().orc_cache_head_dim(self.h))
    max_seq_len = property(lambda self: lib().orc_cache_max_seq_len(self.h))
    compression_ratio = property(lambda self: lib().orc_cache_compression_ratio(self.h))

    def _rc(self, rc):
        if rc != 0:
            raise OracleError(rc)
        return rc

    def load_raw(self, data, seq_len):
        d = _f32(data)
        return self._rc(lib().orc_cache_load_raw(self.h, _p(d), seq_len))

    def append(self, data, layer, kv_idx, n_tokens):
        d = _f32(data)
        return self._rc(lib().orc_cache_append(self.h, _p(d), layer, kv_idx, n_tokens))

    def advance(self, n):
        return self._rc(lib().orc_cache_advance(self.h, n))

    def clear(self):
        lib().orc_cache_clear(self.h)

    def checkpoint(self):
        return lib().orc_checkpoint(self.h)

    def restore(self, n):
        return self._rc(lib().orc_restore(self.h, n))

    def attention_scores(self, q, layer, n_q, n_kv):
        q = _f32(q)
        out = np.zeros((n_q, self.seq_len), np.float32)
        lib().orc_attention_scores(self.h, _p(q), layer, n_q, n_kv, _p(out))
        return out

    def attention_output(self, w, layer, n_q, n_kv):
        w = _f32(w)
        out = np.zeros((n_q, self.head_dim), np.float32)
        lib().orc_attention_output(self.h, _p(w), layer, n_q, n_kv, _p(out))
        return out

    def attention_fused(self, q, layer, n_q, n_kv):
        q = _f32(q)
        out = np.zeros((n_q, self.head_dim), np.float32)
        lib().orc_attention_fused(self.h, _p(q), layer, n_q, n_kv, _p(out))
        return out

    def attention_scores_avx512(self, q, layer, n_q, n_kv):
        """attention_scores on AVX-512 (bit-identical); needs avx512_available()."""
        if not avx512_available():
            raise RuntimeError("this CPU lacks AVX-512 (F, BW, DQ, VL)")
        q = _f32(q)
        out = np.zeros((n_q, self.seq_len), np.float32)
        lib().orc_attention_scores_avx512(self.h, _p(q), layer, n_q, n_kv, _p(out))
        return out

    def attention_output_avx512(self, w, layer, n_q, n_kv):
        """attention_output on AVX-512 (bit-identical); needs avx512_available()."""
        if not avx512_available():
            raise RuntimeError("this CPU lacks AVX-512 (F, BW, DQ, VL)")
        w = _f32(w)
        out = np.zeros((n_q, self.head_dim), np.float32)
        lib().orc_attention_output_avx512(self.h, _p(w), layer, n_q, n_kv, _p(out))
        return out

    def attention_fused_avx512(self, q, layer, n_q, n_kv):
        """orc_attention_fused on AVX-512 (bit-identical); needs
        avx512_available()."""
        if not avx512_available():
            raise RuntimeError("this CPU lacks AVX-512 (F, BW, DQ, VL)")
        q = _f32(q)
        out = np.zeros((n_q, self.head_dim), np.float32)
        lib().orc_attention_fused_avx512(self.h, _p(q), layer, n_q, n_kv, _p(out))
        return out

    def read_planes(self, layer, kv_idx):
        L = lib()
        ng = L.orc_cache_max_groups(self.h)
        w = np.ctypeslib.as_array(C.cast(L.orc_cache_weights(self.h, layer, kv_idx),
                                         C.POINTER(C.c_uint8)), (ng, 32)).copy()
        s = np.ctypeslib.as_array(C.cast(L.orc_cache_scales(self.h, layer, kv_idx),
                                         C.POINTER(C.c_float)), (ng,)).copy()
        b = np.ctypeslib.as_array(C.cast(L.orc_cache_biases(self.h, layer, kv_idx),
                                         C.POINTER(C.c_float)), (ng,)).copy()
        return w, s, b

    def validate(self):
        """Per (layer, kv) block, the code of q4_validate over the first
        n_kv_heads*head_dim*seq_len/64 groups (reference src/cli.c:39-98)."""
        L = lib()
        n = (L.orc_cache_n_heads(self.h) * L.orc_cache_head_dim(self.h) *
             L.orc_cache_seq_len(self.h)) // 64
        out = []
        for layer in range(L.orc_cache_n_layers(self.h)):
            for kv in range(2):
                out.append(int(L.orc_validate(L.orc_cache_scales(self.h, layer, kv),
                                              L.orc_cache_biases(self.h, layer, kv), n)))
        return np.array(out, np.int32)

    def plane_views(self, layer, kv_idx):
        """Writable numpy views of the oracle cache's (weights, scales,
        biases) planes (tests plant values through them)."""
        L = lib()
        ng = L.orc_cache_max_groups(self.h)
        w = np.ctypeslib.as_array(C.cast(L.orc_cache_weights(self.h, layer, kv_idx),
                                         C.POINTER(C.c_uint8)), (ng, 32))
        s = np.ctypeslib.as_array(C.cast(L.orc_cache_scales(self.h, layer, kv_idx),
                                         C.POINTER(C.c_float)), (ng,))
        b = np.ctypeslib.as_array(C.cast(L.orc_cache_biases(self.h, layer, kv_idx),
                                         C.POINTER(C.c_float)), (ng,))
        return w, s, b

    def save(self, path):
        return self._rc(lib().orc_cache_save(self.h, os.fsencode(path)))

    @classmethod
    def load(cls, path):
        out = _vp()
        rc = lib().orc_cache_load(os.fsencode(path), C.byref(out))
        if rc != 0:
            raise OracleError(rc)
        return cls(0, 0, 0, 0, _handle=out.value)


class OracleError(RuntimeError):
    def __init__(self, code):
        super().__init__(f"oracle error {code}")
        self.code = code
