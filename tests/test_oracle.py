"""Pins the CPU oracle (oracle/eakv_oracle.c) before it is trusted.

Each check is chosen so a plausible restatement mistake fails it:
  * the quantizer against the reference's own src/ggml_type.c (built from the
    reference sources into oracle/_ref), bit for bit, plus closed forms;
  * to_i32 and the 16-lane reduce order against their stated definitions;
  * K-score against an f64 brute force, one-hot queries (exact), GQA row
    replication; V-sum against one-hot weights (exact) and f64;
  * fused attention against scores -> softmax -> V-sum and against f64.
"""
import ctypes as C
import math

import numpy as np
import pytest

import oracle as O
from conftest import tol_close


def _groups(rng, n, kind="normal"):
    if kind == "normal":
        return rng.standard_normal((n, 64)).astype(np.float32)
    if kind == "scaled":
        return (rng.standard_normal((n, 64)) *
                np.exp(rng.uniform(-8, 8, (n, 1)))).astype(np.float32)
    if kind == "ints":
        return rng.integers(-3, 4, (n, 64)).astype(np.float32)
    raise ValueError(kind)


# --------------------------------------------------------------- quantizer

def _ref_quantize(x):
    """reference src/ggml_type.c eakv_quantize_row (scalar path)."""
    R = O.ref_lib()
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    n = x.size // 64
    blk = np.zeros(n * 40, np.uint8)
    R.eakv_quantize_row(x.ctypes.data_as(C.c_void_p), blk.ctypes.data_as(C.c_void_p), x.size)
    blk = blk.reshape(n, 40)
    return blk[:, :32].copy(), blk[:, 32:36].copy().view(np.float32)[:, 0], \
        blk[:, 36:40].copy().view(np.float32)[:, 0]


@pytest.mark.parametrize("kind", ["normal", "scaled", "ints"])
def test_quantizer_matches_reference_ggml_type(rng, kind):
    if O.ref_lib() is None:
        pytest.skip("oracle/_ref not built (reference sources absent)")
    x = _groups(rng, 4096, kind)
    w, s, b = O.quantize(x)
    rw, rs, rb = _ref_quantize(x)
    assert np.array_equal(w, rw)
    assert np.array_equal(b.view(np.uint32), rb.view(np.uint32))
    rng_pos = (x.max(1) - x.min(1)) > 0
    assert np.array_equal(s.view(np.uint32)[rng_pos], rs.view(np.uint32)[rng_pos])
    # only difference allowed: a constant group gets scale 1.0 (Ea) vs 0.0
    assert np.all(s[~rng_pos] == 1.0) and np.all(rs[~rng_pos] == 0.0)


def test_quantizer_closed_forms():
    # constant group: scale 1, bias = value, all nibbles 0 (quantize_simd.ea:32-38)
    w, s, b = O.quantize(np.full(64, 2.5, np.float32))
    assert s[0] == 1.0 and b[0] == 2.5 and not w.any()
    # 0..63: range 63, scale 63/15, bias 0 (reference tests/test_ggml_type.c:121-152)
    x = np.arange(64, dtype=np.float32)
    w, s, b = O.quantize(x)
    assert s[0] == np.float32(63.0) / np.float32(15.0) and b[0] == 0.0
    d = O.dequantize(w, s, b)[0]
    assert np.all(np.diff(d) >= 0) and d[0] == 0.0
    assert d[63] == np.float32(15.0 * float(s[0]))      # fma(15, 63/15, 0)
    # split packing: byte k = q(x[k+32])*16 + q(x[k])
    q = np.floor(x * (np.float32(15.0) / np.float32(63.0)) + 0.5).astype(np.int64)
    assert np.array_equal(w[0], (q[32:] * 16 + q[:32]).astype(np.uint8))


def test_quantizer_min_max_nibbles_and_error(rng):
    x = _groups(rng, 512, "scaled")
    w, s, b = O.quantize(x)
    nib = np.concatenate([w & 15, w >> 4], axis=1)
    assert np.all(nib[np.arange(512), x.argmin(1)] == 0)
    assert np.all(nib[np.arange(512), x.argmax(1)] == 15)
    d = O.dequantize(w, s, b)
    err = np.abs(d.astype(np.float64) - x) / s[:, None]
    assert err.max() <= 0.5 + 1e-5


def test_quantizer_special_values():
    inf, nan = np.float32(np.inf), np.float32(np.nan)
    g = np.zeros((6, 64), np.float32)
    g[0, 0] = nan; g[0, 1:] = np.arange(63)           # NaN first: min=max=NaN
    g[1] = np.arange(64); g[1, 5] = nan                # NaN later: skipped
    g[2, :] = 1.0; g[2, 3] = 0.0; g[2, 9] = -0.0      # +0 first among zeros
    g[3, :] = 1.0; g[3, 3] = -0.0; g[3, 9] = 0.0      # -0 first
    g[4, :] = 1.0; g[4, 7] = inf                      # inf max
    g[5, :] = 0.0; g[5, 1] = np.float32(1e-45)         # denormal range
    w, s, b = O.quantize(g)
    assert math.isnan(b[0]) and s[0] == 1.0 and not w[0].any()
    assert b[1] == 0.0 and s[1] == np.float32(63) / np.float32(15)
    assert w[1][5] & 15 == 0                           # NaN -> cvtt INT_MIN -> 0
    assert b[2] == 0.0 and not np.signbit(b[2])
    assert b[3] == 0.0 and np.signbit(b[3])
    assert s[4] == inf and b[4] == 1.0 and not w[4].any()
    # range 1e-45: 15/range overflows to inf; x86 cvtt(inf) = INT_MIN -> 0
    assert s[5] == np.float32(1e-45) / np.float32(15) and not w[5].any()


def test_to_i32_cvtt_semantics():
    L = O.lib()
    assert L.orc_to_i32(1.9) == 1 and L.orc_to_i32(-1.9) == -1
    assert L.orc_to_i32(float("nan")) == -2 ** 31
    assert L.orc_to_i32(2.0 ** 31) == -2 ** 31
    assert L.orc_to_i32(-(2.0 ** 31)) == -2 ** 31
    assert L.orc_to_i32(float("inf")) == -2 ** 31


def test_reduce16_is_the_halving_tree():
    a = np.array([1e8, 1, 1, 1, 1, 1, 1, 1, -1e8, 1, 1, 1, 1, 1, 1, 1], np.float32)
    got = O.lib().orc_reduce16(a.ctypes.data_as(C.c_void_p))
    v8 = a[:8] + a[8:]
    v4 = v8[:4] + v8[4:]
    v2 = v4[:2] + v4[2:]
    assert got == np.float32(v2[0] + v2[1]) == 14.0
    seq = np.float32(0)
    for v in a:
        seq = np.float32(seq + v)
    assert seq != got                    # a sequential sum would give another value


# --------------------------------------------------------------- attention

def _cache_planes(rng, n_kv, d, L, lmax=None):
    lmax = lmax or L
    gpd = d // 64
    x = rng.standard_normal((n_kv, lmax, d)).astype(np.float32)
    w, s, b = O.quantize(x)
    gph = lmax * gpd
    deq = O.dequantize(w, s, b).reshape(n_kv, lmax, d)
    return w, s, b, gph, deq


@pytest.mark.parametrize("d,n_q,n_kv,L", [(128, 4, 4, 37), (64, 8, 1, 33), (128, 8, 2, 64),
                                          (64, 2, 2, 5)])
def test_k_score_vs_f64(rng, d, n_q, n_kv, L):
    w, s, b, gph, deq = _cache_planes(rng, n_kv, d, L, L + 3)
    q = rng.standard_normal((n_q, d)).astype(np.float32)
    got = O.k_score(d, q, w, s, b, L, n_q, n_kv, gph)
    g = n_q // n_kv
    want = np.einsum("hd,htd->ht", q.astype(np.float64),
                     np.repeat(deq[:, :L].astype(np.float64), g, axis=0)) / math.sqrt(d)
    ok, err, _ = tol_close(got, want, atol=1e-5, rtol=1e-5)
    assert ok, err


@pytest.mark.parametrize("d", [64, 128])
def test_k_score_one_hot_is_exact(rng, d):
    L = 19
    w, s, b, gph, deq = _cache_planes(rng, 1, d, L)
    rs = np.float32(1.0) / np.float32(math.sqrt(d))
    for j in (0, 1, 15, 31, 32, 47, 63, d - 1):
        q = np.zeros((1, d), np.float32)
        q[0, j] = 1.0
        got = O.k_score(d, q, w, s, b, L, 1, 1, gph)[0]
        assert np.array_equal(got, (deq[0, :L, j] * rs).astype(np.float32)), j


def test_k_score_gqa_rows_replicate(rng):
    d, L = 128, 21
    w, s, b, gph, _ = _cache_planes(rng, 2, d, L)
    q1 = rng.standard_normal((2, d)).astype(np.float32)
    mha = O.k_score(d, q1, w, s, b, L, 2, 2, gph)
    q4 = np.repeat(q1, 4, axis=0)
    gqa = O.k_score(d, q4, w, s, b, L, 8, 2, gph)
    for h in range(8):
        assert np.array_equal(gqa[h], mha[h // 4])


@pytest.mark.parametrize("d,n_q,n_kv", [(128, 4, 4), (64, 8, 2)])
def test_v_sum_one_hot_and_zero(rng, d, n_q, n_kv):
    L = 23
    w, s, b, gph, deq = _cache_planes(rng, n_kv, d, L)
    g = n_q // n_kv
    for t in (0, 7, L - 1):
        wts = np.zeros((n_q, L), np.float32)
        wts[:, t] = 1.0
        got = O.v_sum(d, wts, w, s, b, L, n_q, n_kv, gph)
        assert np.array_equal(got, np.repeat(deq[:, t], g, axis=0))
    got = O.v_sum(d, np.zeros((n_q, L), np.float32), w, s, b, L, n_q, n_kv, gph)
    assert not got.any()


@pytest.mark.parametrize("d,n_q,n_kv,L", [(128, 4, 4, 40), (64, 8, 1, 33)])
def test_v_sum_vs_f64(rng, d, n_q, n_kv, L):
    w, s, b, gph, deq = _cache_planes(rng, n_kv, d, L)
    wts = rng.random((n_q, L)).astype(np.float32)
    got = O.v_sum(d, wts, w, s, b, L, n_q, n_kv, gph)
    want = np.einsum("ht,htd->hd", wts.astype(np.float64),
                     np.repeat(deq.astype(np.float64), n_q // n_kv, axis=0))
    ok, err, _ = tol_close(got, want, atol=1e-5, rtol=1e-5)
    assert ok, err


def test_softmax_rows(rng):
    sc = (rng.standard_normal((3, 50)) * 4).astype(np.float32)
    got = O.softmax_rows(sc)
    e = np.exp(sc.astype(np.float64) - sc.max(1, keepdims=True))
    ok, err, _ = tol_close(got, e / e.sum(1, keepdims=True), atol=1e-6, rtol=1e-5)
    assert ok, err


@pytest.mark.parametrize("d,n_q,n_kv,L", [(128, 4, 4, 37), (64, 8, 1, 33), (128, 8, 2, 64)])
def test_fused_matches_composition_and_f64(rng, d, n_q, n_kv, L):
    c = O.OracleCache(1, n_kv, d, L + 5)
    c.load_raw(rng.standard_normal((1, 2, n_kv, L, d)).astype(np.float32), L)
    q = rng.standard_normal((n_q, d)).astype(np.float32)
    fused = c.attention_fused(q, 0, n_q, n_kv)
    comp = c.attention_output(O.softmax_rows(c.attention_scores(q, 0, n_q, n_kv)), 0, n_q, n_kv)
    ok, err, _ = tol_close(fused, comp, atol=1e-5, rtol=1e-5)
    assert ok, err
    kw, ks, kb = c.read_planes(0, 0)
    vw, vs, vb = c.read_planes(0, 1)
    K = O.dequantize(kw, ks, kb).reshape(n_kv, -1, d)[:, :L].astype(np.float64)
    V = O.dequantize(vw, vs, vb).reshape(n_kv, -1, d)[:, :L].astype(np.float64)
    g = n_q // n_kv
    sc = np.einsum("hd,htd->ht", q.astype(np.float64), np.repeat(K, g, 0)) / math.sqrt(d)
    p = np.exp(sc - sc.max(1, keepdims=True))
    want = np.einsum("ht,htd->hd", p / p.sum(1, keepdims=True), np.repeat(V, g, 0))
    ok, err, _ = tol_close(fused, want, atol=1e-5, rtol=1e-5)
    assert ok, err


def test_fused_zero_query_is_mean_of_v(rng):
    d, L = 128, 50
    c = O.OracleCache(1, 2, d, L)
    c.load_raw(rng.standard_normal((1, 2, 2, L, d)).astype(np.float32), L)
    out = c.attention_fused(np.zeros((4, d), np.float32), 0, 4, 2)
    vw, vs, vb = c.read_planes(0, 1)
    V = O.dequantize(vw, vs, vb).reshape(2, L, d).astype(np.float64)
    ok, err, _ = tol_close(out, np.repeat(V.mean(1), 2, 0), atol=1e-5, rtol=1e-5)
    assert ok, err


def test_fused_empty_context_is_nan():
    # reference fused_attention.ea: sum = 0 -> 1/sum = inf -> o*inf = 0*inf = NaN
    c = O.OracleCache(1, 1, 64, 8)
    out = c.attention_fused(np.ones((1, 64), np.float32), 0, 1, 1)
    assert np.isnan(out).all()


@pytest.mark.skipif(not O.avx512_available(), reason="this CPU lacks AVX-512")
@pytest.mark.parametrize("d,n_q,n_kv,L", [(128, 32, 8, 700), (64, 8, 4, 300), (128, 4, 4, 1),
                                          (64, 16, 2, 65), (128, 6, 2, 0)])
def test_avx512_fused_attention_is_the_scalar_one(rng, d, n_q, n_kv, L):
    """The CPU baseline's AVX-512 form of the fused kernel (16-lane
    intrinsics) does the scalar restatement's arithmetic lane for lane:
    equal bit for bit, NaN for NaN (empty context)."""
    c = O.OracleCache(1, n_kv, d, max(L, 1) + 3)
    if L:
        c.load_raw((rng.standard_normal((1, 2, n_kv, L, d)) * 2).astype(np.float32), L)
    q = (rng.standard_normal((n_q, d)) * 1.5).astype(np.float32)
    a = c.attention_fused(q, 0, n_q, n_kv)
    b = c.attention_fused_avx512(q, 0, n_q, n_kv)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.skipif(not O.avx512_available(), reason="this CPU lacks AVX-512")
@pytest.mark.parametrize("d,n_q,n_kv,L", [(128, 8, 8, 300), (64, 4, 4, 77), (128, 32, 8, 129),
                                          (64, 32, 4, 64), (128, 7, 1, 33), (128, 3, 3, 0)])
def test_avx512_unfused_kernels_are_the_scalar_ones(rng, d, n_q, n_kv, L):
    """The CPU baseline's AVX-512 K-score and V-sum (16-lane intrinsics, the
    GQA loop flip, q heads in pairs, an odd head alone) against the scalar
    restatement: equal bit for bit, with signed and non-finite weights."""
    c = O.OracleCache(2, n_kv, d, max(L, 1) + 5)
    if L:
        c.load_raw((rng.standard_normal((2, 2, n_kv, L, d)) * 2).astype(np.float32), L)
    q = (rng.standard_normal((n_q, d)) * 1.5).astype(np.float32)
    for layer in (0, 1):
        a = c.attention_scores(q, layer, n_q, n_kv)
        b = c.attention_scores_avx512(q, layer, n_q, n_kv)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        w = rng.standard_normal((n_q, L)).astype(np.float32)
        if L > 3:
            w[0, 3] = np.nan
            w[-1, 1] = np.inf
        a = c.attention_output(w, layer, n_q, n_kv)
        b = c.attention_output_avx512(w, layer, n_q, n_kv)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ------------------------------------------------- dequantize range, validate

def test_dequantize_range_is_a_slice_of_the_closed_form(rng):
    w = rng.integers(0, 256, (50, 32), dtype=np.uint8)
    # scales and biases on a 1/16 grid: every n*s + b is exact in f32, so the
    # closed form needs no rounding
    s = (rng.integers(-128, 128, 50) / 16).astype(np.float32)
    b = (rng.integers(-128, 128, 50) / 16).astype(np.float32)
    # per group: dim j < 32 from the low nibble of byte j, dim j >= 32 from
    # the high nibble of byte j - 32
    lo, hi = (w & 15).astype(np.float64), (w >> 4).astype(np.float64)
    nib = np.concatenate([lo, hi], axis=1)
    want = (nib * s[:, None].astype(np.float64) + b[:, None]).astype(np.float32)
    for g0, n in [(0, 50), (7, 13), (49, 1), (20, 0)]:
        got = O.dequantize_range(w, s, b, g0, n)
        assert got.shape == (n, 64)
        assert np.array_equal(got, want[g0:g0 + n])


def _bits(u):
    return np.array([u], np.uint32).view(np.float32)[0]


def test_validate_codes_and_first_failure():
    n = 16
    ok_s, ok_b = np.full(n, 0.5, np.float32), np.full(n, -1.0, np.float32)
    assert O.validate(ok_s, ok_b, n) == 0
    cases = [
        # (group, scale, bias, code); NaN read from the bits, either sign
        (3, _bits(0x7fc00000), -1.0, 1),          # quiet NaN scale
        (3, _bits(0xffc00000), -1.0, 1),          # negative NaN scale
        (3, _bits(0x7f800001), -1.0, 1),          # signalling NaN scale
        (5, 0.5, _bits(0x7fc00000), 2),           # NaN bias
        (5, 0.5, _bits(0xffffffff), 2),           # NaN bias, all bits set
        (6, -1.0, -1.0, 3),                       # negative scale
        (6, -np.inf, -1.0, 3),                    # -inf scale: not NaN, negative
        (6, _bits(0x80000001), -1.0, 3),          # negative denormal scale
        (9, -0.0, -1.0, 0),                       # -0.0 is not < 0
        (9, np.inf, np.inf, 0),                   # +inf scale and bias pass
        (9, 0.5, -np.inf, 0),
        (2, _bits(0x7fc00000), _bits(0x7fc00000), 1),  # scale checked first
        (2, -1.0, _bits(0x7fc00000), 2),          # bias NaN before the sign
    ]
    for g, sv, bv, code in cases:
        s, b = ok_s.copy(), ok_b.copy()
        s[g], b[g] = sv, bv
        assert O.validate(s, b, n) == code, (g, sv, bv)
        assert O.validate(s, b, g) == 0           # groups before g only
    # the first failing group decides, not the lowest code
    s, b = ok_s.copy(), ok_b.copy()
    b[3] = np.nan
    s[5] = -2.0
    assert O.validate(s, b, n) == 2
    s, b = ok_s.copy(), ok_b.copy()
    s[2] = -2.0
    s[7] = np.nan
    assert O.validate(s, b, n) == 3


def test_validate_cache_covers_the_reference_group_range(rng):
    nl, nh, d, L, lmax = 2, 3, 64, 5, 8
    c = O.OracleCache(nl, nh, d, lmax)
    c.load_raw(rng.standard_normal((nl, 2, nh, L, d)).astype(np.float32), L)
    assert c.validate().tolist() == [0, 0, 0, 0]
    n = nh * d * L // 64                          # reference src/cli.c:49
    _, s, _ = c.plane_views(1, 0)
    s[n - 1] = -1.0                               # last checked group
    _, _, b = c.plane_views(0, 1)
    b[n] = np.nan                                 # first unchecked group
    assert c.validate().tolist() == [0, 0, 3, 0]
    c.free()


# ----------------------------------------------------------- ggml block type

@pytest.mark.parametrize("kind", ["normal", "scaled", "ints"])
def test_ggml_oracle_matches_reference_builds(rng, kind):
    """orc_ggml_*: the quantizer equals the reference's ggml_type.c (scalar
    build) bit for bit; dequantize and vec_dot equal its AVX-512 build bit for
    bit where the CPU runs it, and its scalar build (unfused n*d + m, one
    sequential sum) within the scores bar."""
    S, A = O.ref_lib(), O.ref_lib(avx512=True)
    if S is None:
        pytest.skip("oracle/_ref not built (needs the reference sources)")
    vp = lambda a: a.ctypes.data_as(C.c_void_p)
    x = _groups(rng, 40, kind).reshape(-1)
    blk = np.zeros((40, 40), np.uint8)
    S.eakv_quantize_row(vp(x), vp(blk), x.size)
    assert np.array_equal(O.ggml_quantize_row(x), blk)
    n, nrc = 640, 4
    vx = np.stack([O.ggml_quantize_row(_groups(rng, n // 64, kind).reshape(-1)).reshape(-1)
                   for _ in range(nrc)])
    vy = rng.standard_normal((nrc, n)).astype(np.float32)
    libs = [(S, False)] + ([(A, True)] if A is not None else [])
    for R, exact in libs:
        deq = np.zeros(x.size, np.float32)
        R.eakv_dequantize_row(vp(blk), vp(deq), x.size)
        dot = np.zeros(nrc, np.float32)
        R.eakv_vec_dot_q4_f32(n, vp(dot), 4, vp(vx), vx.shape[1], vp(vy), n * 4, nrc)
        od, ot = O.ggml_dequantize_row(blk), O.ggml_vec_dot(vx, vy)
        if exact:
            assert np.array_equal(od.view(np.uint32), deq.view(np.uint32))
            assert np.array_equal(ot.view(np.uint32), dot.view(np.uint32))
        else:
            ok, err, _ = tol_close(od, deq, 1e-4, 1e-5)
            assert ok, err
            # two f32 sums of the same n products in different orders: each
            # within n * 2^-24 * sum|terms| of the exact dot
            terms = np.stack([O.ggml_dequantize_row(r) for r in vx]).astype(np.float64) * vy
            bound = 2 * n * 2.0 ** -24 * np.abs(terms).sum(axis=1)
            assert np.all(np.abs(ot.astype(np.float64) - dot) <= bound)
