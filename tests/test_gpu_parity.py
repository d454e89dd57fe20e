"""GPU parity: libeakv.so (HIP, gfx950) against the CPU oracle on the same
seeded inputs, through the C ABI.

Bar: quantization (nibbles, scales, biases) and K-scores bit-exact; V-sum and
fused attention within |gpu - oracle| <= 1e-4 + 1e-5*|oracle|.
"""
import os
import sys

import numpy as np
import pytest

import oracle as O
from conftest import tol_close

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-4, 1e-5


@pytest.fixture(scope="module")
def E():
    import eakv_amd
    from eakv_amd import hipmem
    if hipmem.device_count() < 1:
        pytest.fail("no HIP device visible")
    return eakv_amd


def say(*a):
    print(*a, flush=True)


def special_data(rng, n_groups):
    """Groups with NaN / inf / signed zeros / constants / tiny ranges mixed in."""
    x = (rng.standard_normal((n_groups, 64)) *
         np.exp(rng.uniform(-4, 4, (n_groups, 1)))).astype(np.float32)
    k = np.arange(n_groups) % 12
    x[k == 1, 0] = np.nan
    x[k == 2, 17] = np.nan
    x[k == 3] = 1.0; x[k == 3, 5] = 0.0; x[k == 3, 40] = -0.0
    x[k == 4] = 1.0; x[k == 4, 5] = -0.0; x[k == 4, 40] = 0.0
    x[k == 5, 9] = np.inf
    x[k == 6, 33] = -np.inf
    x[k == 7] = 3.25
    x[k == 8] = 0.0; x[k == 8, 63] = np.float32(1e-45)
    x[k == 9] = np.float32(2.0 ** -130) * rng.integers(0, 8, (np.sum(k == 9), 64))
    x[k == 10] = -0.0
    x[k == 11] = rng.integers(-2, 3, (np.sum(k == 11), 64))
    return x


def planes_equal(a, b):
    return all(np.array_equal(np.ascontiguousarray(x).view(np.uint8),
                              np.ascontiguousarray(y).view(np.uint8)) for x, y in zip(a, b))


def pair(E, nl, nh, hd, lmax):
    return E.Cache(nl, nh, hd, lmax), O.OracleCache(nl, nh, hd, lmax)


# ------------------------------------------------------------- quantization

@pytest.mark.parametrize("nl,nh,hd,L,lmax,kind", [
    (1, 2, 128, 37, 40, "normal"), (2, 4, 64, 33, 33, "normal"),
    (1, 1, 64, 1, 5, "normal"), (1, 3, 128, 100, 128, "special"),
    (1, 2, 192, 10, 12, "normal"), (1, 2, 96, 7, 8, "normal"),
    (1, 8, 128, 2048, 2048, "special"), (3, 2, 64, 513, 600, "special")])
def test_bulk_quantize_bitexact(E, rng, nl, nh, hd, L, lmax, kind):
    say("bulk", nl, nh, hd, L, lmax, kind)
    n = nl * 2 * nh * L * hd
    if kind == "normal":
        data = rng.standard_normal(n).astype(np.float32)
    else:
        data = special_data(rng, n // 64).reshape(-1)
    g, o = pair(E, nl, nh, hd, lmax)
    g.load_raw(data, L)
    o.load_raw(data, L)
    assert g.seq_len == L
    for l in range(nl):
        for kv in range(2):
            assert planes_equal(g.read_planes(l, kv), o.read_planes(l, kv)), (l, kv)


@pytest.mark.parametrize("hd,n_tok", [(128, 1), (64, 1), (128, 5), (64, 70)])
def test_append_bitexact(E, rng, hd, n_tok):
    nl, nh, lmax = 2, 4, 80
    g, o = pair(E, nl, nh, hd, lmax)
    base = rng.standard_normal(nl * 2 * nh * 3 * hd).astype(np.float32)
    g.load_raw(base, 3)
    o.load_raw(base, 3)
    t = 3
    while t + n_tok <= lmax:
        for l in range(nl):
            for kv in range(2):
                x = special_data(rng, nh * n_tok * hd // 64).reshape(-1)
                assert g.append(x, l, kv, n_tok) == 0
                o.append(x, l, kv, n_tok)
        g.advance(n_tok)
        o.advance(n_tok)
        t += n_tok
        if t > 20:
            break
    for l in range(nl):
        for kv in range(2):
            assert planes_equal(g.read_planes(l, kv), o.read_planes(l, kv))


def test_append_device_and_batch(E, rng):
    from eakv_amd.hipmem import DeviceArray
    nl, nh, hd, lmax, nseq = 3, 2, 128, 16, 3
    gs = [E.Cache(nl, nh, hd, lmax) for _ in range(nseq)]
    os_ = [O.OracleCache(nl, nh, hd, lmax) for _ in range(nseq)]
    for i, (g, o) in enumerate(zip(gs, os_)):
        d = rng.standard_normal(nl * 2 * nh * (4 + i) * hd).astype(np.float32)
        dd = DeviceArray.from_host(d)
        assert E.lib().eakv_cache_load_raw_device(g.h, dd.ptr, 4 + i, None) == 0
        g.sync()
        o.load_raw(d, 4 + i)
    for step in range(3):
        x = rng.standard_normal((nseq, nl, 2, nh, 1, hd)).astype(np.float32)
        dx = DeviceArray.from_host(x)
        assert E.lib().eakv_append_batch_device(E.handles(gs), nseq, dx.ptr, 1, None) == 0
        gs[0].sync()
        for i in range(nseq):
            for l in range(nl):
                for kv in range(2):
                    os_[i].append(x[i, l, kv], l, kv, 1)
            os_[i].advance(1)
            gs[i].advance(1)
    # single (layer, kv) device append
    x = rng.standard_normal((nh, 2, hd)).astype(np.float32)
    dx = DeviceArray.from_host(x)
    assert E.lib().eakv_cache_append_device(gs[1].h, dx.ptr, 2, 1, 2, None) == 0
    gs[1].sync()
    os_[1].append(x, 2, 1, 2)
    for g, o in zip(gs, os_):
        for l in range(nl):
            for kv in range(2):
                assert planes_equal(g.read_planes(l, kv), o.read_planes(l, kv))


# ------------------------------------------------------------- attention

SHAPES = [  # (n_kv heads in cache, n_q, n_kv used, d, L, lmax)
    (8, 8, 8, 128, 37, 40), (4, 32, 4, 64, 300, 300), (8, 32, 8, 128, 513, 520),
    (2, 16, 2, 128, 1000, 1024), (4, 4, 4, 64, 1, 4), (4, 8, 2, 128, 257, 260),
    (1, 8, 1, 64, 1025, 1030), (2, 64, 2, 128, 100, 100),
    (8, 32, 8, 128, 4097, 4100), (4, 16, 4, 64, 2049, 2050), (2, 4, 2, 128, 3000, 3000),
    (2, 6, 2, 64, 700, 704), (2, 10, 2, 128, 777, 780), (1, 7, 1, 64, 300, 300)]


def loaded(E, rng, nh, d, L, lmax, nl=2):
    g, o = pair(E, nl, nh, d, lmax)
    data = (rng.standard_normal(nl * 2 * nh * L * d) * 1.5).astype(np.float32)
    g.load_raw(data, L)
    o.load_raw(data, L)
    return g, o


@pytest.mark.parametrize("nh,n_q,n_kv,d,L,lmax", SHAPES)
def test_k_score_bitexact(E, rng, nh, n_q, n_kv, d, L, lmax):
    say("kscore", nh, n_q, n_kv, d, L)
    g, o = loaded(E, rng, nh, d, L, lmax)
    q = rng.standard_normal((n_q, d)).astype(np.float32)
    for layer in (0, 1):
        a = g.attention_scores(q, layer, n_q, n_kv)
        b = o.attention_scores(q, layer, n_q, n_kv)
        assert a.shape == (n_q, L)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), \
            np.abs(a - b).max()


@pytest.mark.parametrize("nh,n_q,n_kv,d,L,lmax", SHAPES)
def test_v_sum_parity(E, rng, nh, n_q, n_kv, d, L, lmax):
    say("vsum", nh, n_q, n_kv, d, L)
    g, o = loaded(E, rng, nh, d, L, lmax)
    q = rng.standard_normal((n_q, d)).astype(np.float32)
    w = O.softmax_rows(o.attention_scores(q, 1, n_q, n_kv))
    a = g.attention_output(w, 1, n_q, n_kv)
    b = o.attention_output(w, 1, n_q, n_kv)
    ok, err, nbad = tol_close(a, b, ATOL, RTOL)
    assert ok, (err, nbad)
    # Unnormalised weights: a plain f32 sum of seq_len terms, whose rounding
    # (oracle: one sequential chain; GPU: split chains) grows with the sum of
    # |terms|.  Both are held to 4e-7 * sum|w*v| + 1e-4 of the exact f64 value.
    w2 = rng.random((n_q, L)).astype(np.float32)
    vw, vs, vb = o.read_planes(1, 1)
    Vd = O.dequantize(vw, vs, vb).reshape(nh, lmax, d)[:n_kv, :L].astype(np.float64)
    Vd = np.repeat(Vd, n_q // n_kv, axis=0)
    exact = np.einsum("ht,htd->hd", w2.astype(np.float64), Vd)
    mag = np.einsum("ht,htd->hd", w2.astype(np.float64), np.abs(Vd))
    for got in (g.attention_output(w2, 1, n_q, n_kv), o.attention_output(w2, 1, n_q, n_kv)):
        err = np.abs(got - exact)
        assert np.all(err <= 1e-4 + 4e-7 * mag), (err.max(), (err / mag).max())


@pytest.mark.parametrize("nh,n_q,n_kv,d,L,lmax", [
    (8, 32, 8, 128, 3000, 3000), (4, 32, 4, 64, 1000, 1024), (2, 2, 2, 128, 77, 80),
    (2, 12, 2, 128, 513, 520)])
def test_v_sum_signed_and_nonfinite_weights(E, rng, nh, n_q, n_kv, d, L, lmax):
    """Weights of either sign (the V-sum takes any weights, not only softmax
    rows): within 1e-4 + 4e-7 * sum|w*v| of the exact f64 sum, as the
    reference's single fma chain.  A NaN weight in a head's row makes that
    head's output NaN, as in the reference's chain; the other heads are
    unaffected."""
    say("vsum-signed", nh, n_q, n_kv, d, L)
    g, o = loaded(E, rng, nh, d, L, lmax)
    w = (rng.standard_normal((n_q, L)) * np.exp(rng.uniform(-3, 3, (n_q, 1)))).astype(np.float32)
    vw, vs, vb = o.read_planes(1, 1)
    Vd = O.dequantize(vw, vs, vb).reshape(nh, lmax, d)[:n_kv, :L].astype(np.float64)
    Vd = np.repeat(Vd, n_q // n_kv, axis=0)
    exact = np.einsum("ht,htd->hd", w.astype(np.float64), Vd)
    mag = np.einsum("ht,htd->hd", np.abs(w.astype(np.float64)), np.abs(Vd))
    for got in (g.attention_output(w, 1, n_q, n_kv), o.attention_output(w, 1, n_q, n_kv)):
        err = np.abs(got - exact)
        assert np.all(err <= 1e-4 + 4e-7 * mag), (err.max(), (err / mag).max())
    w[1, L // 2] = np.nan
    got = g.attention_output(w, 1, n_q, n_kv)
    assert np.isnan(got[1]).all()
    assert np.isnan(o.attention_output(w, 1, n_q, n_kv)[1]).all()
    keep = [h for h in range(n_q) if h != 1]
    err = np.abs(got[keep] - exact[keep])
    assert np.all(err <= 1e-4 + 4e-7 * mag[keep]), err.max()


@pytest.mark.parametrize("nh,n_q,n_kv,d,L,lmax", [
    (2, 32, 2, 128, 1500, 1500), (1, 16, 1, 64, 2100, 2100), (2, 24, 2, 128, 700, 704),
    (2, 20, 2, 64, 333, 340), (1, 11, 1, 128, 500, 500), (4, 48, 4, 128, 1025, 1030)])
def test_large_groups_fused_and_v_sum(E, rng, nh, n_q, n_kv, d, L, lmax):
    """More than 8 q heads per kv head (MQA and wide GQA): the matrix-core
    programs split the group into virtual kv heads of at most 8 q heads that
    read the same kv head (16 -> 2 x 8, 24 -> 3 x 8, 10 -> 2 x 5, 12 -> 2 x 6,
    11 -> 11 x 1).  Fused attention and the V-sum against the oracle."""
    say("large-groups", nh, n_q, n_kv, d, L)
    g, o = loaded(E, rng, nh, d, L, lmax)
    q = (rng.standard_normal((n_q, d)) * 2).astype(np.float32)
    ok, err, nbad = tol_close(g.attention_fused(q, 1, n_q, n_kv),
                              o.attention_fused(q, 1, n_q, n_kv), ATOL, RTOL)
    assert ok, (err, nbad)
    w = O.softmax_rows(o.attention_scores(q, 1, n_q, n_kv))
    ok, err, nbad = tol_close(g.attention_output(w, 1, n_q, n_kv),
                              o.attention_output(w, 1, n_q, n_kv), ATOL, RTOL)
    assert ok, (err, nbad)


@pytest.mark.parametrize("nh,n_q,n_kv,d,L", [
    (8, 64, 8, 128, 40000), (2, 16, 2, 64, 20000), (2, 12, 2, 128, 9000),
    (4, 16, 4, 128, 30000)])
def test_fused_repeat_bits_eight_heads(E, rng, nh, n_q, n_kv, d, L):
    """Every wave of the matrix-core program sums a fixed set of tiles in a
    fixed order, so a call repeated on the same inputs gives the same bits:
    fused attention (against the oracle too) and the V-sum, at 5-8 q heads
    per kv head (two quads per wave) and at 4 (one quad per wave), over
    contexts long enough that every wave takes many tiles."""
    say("repeat-bits", nh, n_q, n_kv, d, L)
    g, o = loaded(E, rng, nh, d, L, L, nl=1)
    q = (rng.standard_normal((n_q, d)) * 2).astype(np.float32)
    a = g.attention_fused(q, 0, n_q, n_kv)
    ok, err, nbad = tol_close(a, o.attention_fused(q, 0, n_q, n_kv), ATOL, RTOL)
    assert ok, (err, nbad)
    for _ in range(3):
        assert np.array_equal(g.attention_fused(q, 0, n_q, n_kv).view(np.uint32),
                              a.view(np.uint32))
    w = rng.random((n_q, L)).astype(np.float32)
    b = g.attention_output(w, 0, n_q, n_kv)
    for _ in range(3):
        assert np.array_equal(g.attention_output(w, 0, n_q, n_kv).view(np.uint32),
                              b.view(np.uint32))


@pytest.mark.parametrize("nh,n_q,n_kv,d,L,lmax", SHAPES)
def test_fused_parity(E, rng, nh, n_q, n_kv, d, L, lmax):
    say("fused", nh, n_q, n_kv, d, L)
    g, o = loaded(E, rng, nh, d, L, lmax)
    q = (rng.standard_normal((n_q, d)) * 2).astype(np.float32)
    a = g.attention_fused(q, 1, n_q, n_kv)
    b = o.attention_fused(q, 1, n_q, n_kv)
    ok, err, nbad = tol_close(a, b, ATOL, RTOL)
    assert ok, (err, nbad)


@pytest.mark.parametrize("d,n_q,L", [(128, 16, 100), (64, 8, 4097), (128, 4, 31)])
def test_fused_ignores_stale_nonfinite_tail(E, rng, d, n_q, L):
    """Tokens past seq_len that hold non-finite data (appended without
    advancing) must not reach the result: a tile that covers them gives them
    weight exactly 0."""
    nh, lmax = 4, L + 64
    g, o = pair(E, 1, nh, d, lmax)
    data = rng.standard_normal((1, 2, nh, L, d)).astype(np.float32)
    g.load_raw(data, L)
    o.load_raw(data, L)
    bad = np.full((nh, 40, d), np.nan, np.float32)
    bad[:, ::3] = np.inf
    bad[:, 1::3, :5] = -np.inf
    for kv in (0, 1):
        g.append(bad, 0, kv, 40)       # at positions L..L+39, seq_len stays L
        o.append(bad, 0, kv, 40)
    assert g.seq_len == L
    q = rng.standard_normal((n_q, d)).astype(np.float32)
    a = g.attention_fused(q, 0, n_q, nh)
    b = o.attention_fused(q, 0, n_q, nh)
    assert np.isfinite(a).all()
    ok, err, nbad = tol_close(a, b, ATOL, RTOL)
    assert ok, (err, nbad)


def exact_attention(o, q, layer, n_q, n_kv, L):
    """Attention over the quantized cache in f64: K and V = nibble*scale + bias
    exactly, softmax(q.K/sqrt(d)) V with the exact max."""
    nh, d, lmax = o.n_heads, o.head_dim, o.max_seq_len
    kv = []
    for k in (0, 1):
        w, s, b = o.read_planes(layer, k)
        n = np.concatenate([w & 15, w >> 4], axis=1).astype(np.float64)
        x = n * s.astype(np.float64)[:, None] + b.astype(np.float64)[:, None]
        kv.append(x.reshape(nh, lmax, d)[:, :L])
    K, V = kv
    qpk = n_q // n_kv
    out = np.zeros((n_q, d))
    for h in range(n_q):
        sc = K[h // qpk] @ q[h].astype(np.float64) / np.sqrt(d)
        p = np.exp(sc - sc.max())
        out[h] = p @ V[h // qpk] / p.sum()
    return out


def slope_case(E, rng, d, n_q, n_kv, L, slope, center):
    """Keys along one direction per kv head, growing with the token index
    (times `slope`, from -L/2 if `center`), and queries along it: scores that
    rise (slope > 0) or fall (< 0) by about `slope` per token."""
    u = rng.standard_normal((n_kv, d))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    t = np.arange(L, dtype=np.float64) - (L / 2 if center else 0)
    K = (slope * t)[None, :, None] * u[:, None, :] + 0.1 * rng.standard_normal((n_kv, L, d))
    V = rng.standard_normal((n_kv, L, d))
    data = np.stack([K, V])[None].astype(np.float32)
    g, o = pair(E, 1, n_kv, d, L + 8)
    g.load_raw(data, L)
    o.load_raw(data, L)
    q = (np.repeat(u, n_q // n_kv, axis=0) * np.sqrt(d) +
         0.3 * rng.standard_normal((n_q, d))).astype(np.float32)
    sc = o.attention_scores(q, 0, n_q, n_kv)
    assert abs(float(sc[:, -1].mean() - sc[:, 0].mean())) > 0.5 * abs(slope) * L
    return g, o, q, float(np.abs(sc).max())


@pytest.mark.parametrize("d,n_q,n_kv,L,slope", [
    (128, 32, 8, 600, 0.2), (128, 64, 8, 600, 0.25), (128, 64, 8, 96, 1.5),
    (64, 8, 8, 1500, 0.05), (128, 16, 4, 700, -0.2), (64, 32, 4, 90, 1.4),
    (128, 64, 8, 20000, 0.007), (64, 64, 8, 16400, -0.008)])
def test_fused_rising_and_falling_scores(E, rng, d, n_q, n_kv, L, slope):
    """Scores within about +-150: rising ones move the running max again and
    again (every tile at the steep slopes, in every quad of q heads); falling
    ones put the max in the first tile and drive the later weights to 0.  The
    long contexts run two-quad waves (8 q heads per wave), asserted."""
    say("fused-slope", d, n_q, n_kv, L, slope)
    g, o, q, smax = slope_case(E, rng, d, n_q, n_kv, L, slope, center=True)
    assert smax < 160
    if L > 10000:
        assert E.fused_plan([g], n_q, n_kv)["quads"] == 2
    a = g.attention_fused(q, 0, n_q, n_kv)
    b = o.attention_fused(q, 0, n_q, n_kv)
    assert np.isfinite(a).all()
    ok, err, nbad = tol_close(a, b, ATOL, RTOL)
    assert ok, (err, nbad)


@pytest.mark.parametrize("d,n_q,n_kv,L,slope", [(128, 64, 8, 2000, 1.5),
                                               (128, 32, 8, 3000, 0.25)])
def test_fused_huge_scores_as_accurate_as_reference(E, rng, d, n_q, n_kv, L, slope):
    """Scores in the hundreds and thousands: one f32 ulp of the largest score
    (6.1e-5 at 788, 2.4e-4 at 3203) moves its token's weight by that much
    relative, and so the outputs by more than the 1e-4 bar; two f32 orders
    of the score arithmetic (the reference's fma chain, the fused kernel's
    exact integer dots recombined in f32) cannot agree within the bar, nor
    either of them meet it against the exact f64 attention over the same
    quantized cache.  The premise is asserted (ulp(max|score|) * max|output|
    above the bar), and the fused kernel is held to the exact result: no less
    accurate than the reference algorithm at the largest error and in the
    mean square, and value by value within the reference's largest error
    plus the bar."""
    say("fused-huge", d, n_q, n_kv, L, slope)
    g, o, q, smax = slope_case(E, rng, d, n_q, n_kv, L, slope, center=False)
    assert smax > 700
    exact = exact_attention(o, q, 0, n_q, n_kv, L)
    assert float(np.spacing(np.float32(smax))) * float(np.abs(exact).max()) > ATOL
    got = g.attention_fused(q, 0, n_q, n_kv).astype(np.float64)
    ref = o.attention_fused(q, 0, n_q, n_kv).astype(np.float64)
    e_gpu = float(np.abs(got - exact).max())
    e_ref = float(np.abs(ref - exact).max())
    r_gpu = float(np.sqrt(np.mean((got - exact) ** 2)))
    r_ref = float(np.sqrt(np.mean((ref - exact) ** 2)))
    say("  max|score|", smax, "error vs exact (max, rms): gpu", e_gpu, r_gpu,
        "reference algorithm", e_ref, r_ref, "gpu vs reference", float(np.abs(got - ref).max()))
    assert e_gpu <= e_ref
    assert r_gpu <= r_ref
    assert np.all(np.abs(got - exact) <= e_ref + ATOL + RTOL * np.abs(exact))


@pytest.mark.parametrize("d,n_q,n_kv,L,where", [(128, 32, 8, 700, "k"), (128, 16, 2, 300, "v"),
                                                (64, 8, 4, 500, "k"), (128, 64, 8, 450, "v"),
                                                (128, 64, 8, 20000, "k"), (64, 64, 8, 16400, "v")])
def test_fused_nonfinite_cache_values_propagate(E, rng, d, n_q, n_kv, L, where):
    """A NaN as the first value of a 64-value group quantizes to a NaN scale
    and bias (the strict min/max scan keeps it).  In K it makes that token's
    score NaN and so every output of the kv head's q heads; in V it makes the
    group's 64 output dims NaN.  The NaN pattern equals the oracle's and the
    other values match it."""
    say("fused-nan", d, n_q, n_kv, L, where)
    data = rng.standard_normal((1, 2, n_kv, L, d)).astype(np.float32)
    data[0, 0 if where == "k" else 1, 1, L // 3, 0] = np.nan
    g, o = pair(E, 1, n_kv, d, L + 4)
    g.load_raw(data, L)
    o.load_raw(data, L)
    q = rng.standard_normal((n_q, d)).astype(np.float32)
    if L > 10000:                               # two-quad waves
        assert E.fused_plan([g], n_q, n_kv)["quads"] == 2
    a = g.attention_fused(q, 0, n_q, n_kv)
    b = o.attention_fused(q, 0, n_q, n_kv)
    nan = np.isnan(b)
    assert nan.any() and not nan.all()
    assert np.array_equal(np.isnan(a), nan)
    ok, err, nbad = tol_close(a[~nan], b[~nan], ATOL, RTOL)
    assert ok, (err, nbad)


def test_fused_batch_device(E, rng):
    from eakv_amd.hipmem import DeviceArray
    nl, nh, d, n_q, lmax = 2, 4, 128, 16, 1100
    lens = [1, 511, 512, 513, 1100, 37]
    gs, os_ = [], []
    for L in lens:
        g, o = loaded(E, rng, nh, d, L, lmax, nl)
        gs.append(g)
        os_.append(o)
    q = rng.standard_normal((len(lens), n_q, d)).astype(np.float32)
    dq = DeviceArray.from_host(q)
    dout = DeviceArray((len(lens), n_q, d))
    assert E.lib().eakv_attention_fused_batch_device(E.handles(gs), len(gs), 1, dq.ptr,
                                                     n_q, nh, dout.ptr, None) == 0
    gs[0].sync()
    out = dout.download()
    for i, o in enumerate(os_):
        ok, err, nbad = tol_close(out[i], o.attention_fused(q[i], 1, n_q, nh), ATOL, RTOL)
        assert ok, (lens[i], err, nbad)


@pytest.mark.parametrize("d,lens,lmax", [
    (64, [0, 5, 4600, 300], 4608), (128, [0, 5, 4600, 300], 4608),
    (64, [0, 5, 1000, 300], 1024), (128, [300, 0, 1000, 1], 1024)])
def test_fused_batch_long_short_and_empty(E, rng, d, lens, lmax):
    """A batch of long, short and empty sequences.  With 4600 tokens the
    longest splits into more than 16 chunks (the 8-part merge launch); with
    1000 the grid is smaller than the device and the launch merges its own
    chunks (counters in the first cache).  Each sequence merges only its own
    chunks, the empty one gives NaN, as the reference's 0 * (1/0), and a
    second call (the counters back at zero) gives the same bits."""
    from eakv_amd.hipmem import DeviceArray
    nl, nh, n_q = 1, 2, 8
    gs, os_ = [], []
    for L in lens:
        g, o = pair(E, nl, nh, d, lmax) if L == 0 else loaded(E, rng, nh, d, L, lmax, nl)
        gs.append(g)
        os_.append(o)
    q = rng.standard_normal((len(lens), n_q, d)).astype(np.float32)
    dq = DeviceArray.from_host(q)
    dout = DeviceArray((len(lens), n_q, d))
    assert E.lib().eakv_attention_fused_batch_device(E.handles(gs), len(gs), 0, dq.ptr,
                                                     n_q, nh, dout.ptr, None) == 0
    gs[0].sync()
    out = dout.download()
    for i, L in enumerate(lens):
        if L == 0:
            assert np.isnan(out[i]).all()
            continue
        ok, err, nbad = tol_close(out[i], os_[i].attention_fused(q[i], 0, n_q, nh), ATOL, RTOL)
        assert ok, (L, err, nbad)
    from eakv_amd.hipmem import synchronize
    dout.zero()
    synchronize()
    assert E.lib().eakv_attention_fused_batch_device(E.handles(gs), len(gs), 0, dq.ptr,
                                                     n_q, nh, dout.ptr, None) == 0
    gs[0].sync()
    again = dout.download()
    assert np.array_equal(again.view(np.uint32), out.view(np.uint32))


def test_workspace_ordered_across_caller_streams(E, rng):
    """Device calls on two caller streams, back to back, share the cache's
    workspace (the fused chunk partials, the V-sum partials): each call waits
    for the previous one through an event, so every result matches the
    oracle; a host call and freeing the cache afterwards wait for them too."""
    from eakv_amd.hipmem import DeviceArray, Stream
    nh, d, n_q, L = 8, 128, 32, 8192
    g, o = loaded(E, rng, nh, d, L, L, 1)
    sa, sb = Stream(), Stream()
    qs = [rng.standard_normal((n_q, d)).astype(np.float32) for _ in range(4)]
    dq = [DeviceArray.from_host(q) for q in qs]
    dout = [DeviceArray((n_q, d)) for _ in qs]
    for i in range(len(qs)):
        st = (sa, sb)[i % 2].s
        assert E.lib().eakv_attention_fused_batch_device(E.handles([g]), 1, 0, dq[i].ptr,
                                                         n_q, nh, dout[i].ptr, st) == 0
    ws = [rng.random((n_q, L)).astype(np.float32) for _ in range(2)]
    dw = [DeviceArray.from_host(w) for w in ws]
    dvo = [DeviceArray((n_q, d)) for _ in ws]
    for i in range(2):
        assert E.lib().eakv_attention_output_device(g.h, dw[i].ptr, 0, n_q, nh, dvo[i].ptr,
                                                    (sb, sa)[i].s) == 0
    # a host call on the cache's own stream right behind them
    host = g.attention_fused(qs[0], 0, n_q, nh)
    sa.synchronize()
    sb.synchronize()
    for i, q in enumerate(qs):
        ok, err, nbad = tol_close(dout[i].download(), o.attention_fused(q, 0, n_q, nh),
                                  ATOL, RTOL)
        assert ok, (i, err, nbad)
    assert np.array_equal(host, dout[0].download())
    for i, w in enumerate(ws):
        assert np.array_equal(dvo[i].download(), g.attention_output(w, 0, n_q, nh)), i
    # the last workspace use on a caller's stream, then free
    assert E.lib().eakv_attention_output_device(g.h, dw[0].ptr, 0, n_q, nh, dvo[1].ptr,
                                                sa.s) == 0
    g.free()
    sa.synchronize()
    assert np.array_equal(dvo[1].download(), dvo[0].download())


def test_device_calls_equal_host_calls(E, rng):
    from eakv_amd.hipmem import DeviceArray
    g, _ = loaded(E, rng, 4, 128, 200, 256)
    q = rng.standard_normal((16, 128)).astype(np.float32)
    dq, ds = DeviceArray.from_host(q), DeviceArray((16, 200))
    assert E.lib().eakv_attention_scores_device(g.h, dq.ptr, 0, 16, 4, ds.ptr, None) == 0
    g.sync()
    assert np.array_equal(ds.download(), g.attention_scores(q, 0, 16, 4))
    w = rng.random((16, 200)).astype(np.float32)
    dw, do = DeviceArray.from_host(w), DeviceArray((16, 128))
    assert E.lib().eakv_attention_output_device(g.h, dw.ptr, 0, 16, 4, do.ptr, None) == 0
    g.sync()
    assert np.array_equal(do.download(), g.attention_output(w, 0, 16, 4))


def test_empty_cache(E):
    g, o = pair(E, 1, 2, 64, 8)
    q = np.ones((2, 64), np.float32)
    assert g.attention_scores(q, 0, 2, 2).shape == (2, 0)
    out = g.attention_output(np.zeros((2, 0), np.float32), 0, 2, 2)
    assert np.array_equal(out, o.attention_output(np.zeros((2, 0), np.float32), 0, 2, 2))
    assert not out.any()
    assert np.isnan(g.attention_fused(q, 0, 2, 2)).all()


@pytest.mark.parametrize("args", [(0, 3, 2), (0, 4, 3), (2, 4, 4), (0, 16, 8), (-1, 4, 4)])
def test_attention_rejects_invalid(E, rng, args):
    layer, n_q, n_kv = args
    g, _ = loaded(E, rng, 4, 64, 10, 10)
    with pytest.raises(E.EakvError) as e:
        g.attention_scores(np.ones((n_q, 64), np.float32), layer, n_q, n_kv)
    assert e.value.code == E.EAKV_ERR_INVALID


def test_head_dim_other_than_64_128_rejected(E, rng):
    g = E.Cache(1, 2, 192, 8)
    g.load_raw(rng.standard_normal(2 * 2 * 8 * 192).astype(np.float32), 8)
    with pytest.raises(E.EakvError):
        g.attention_scores(np.ones((2, 192), np.float32), 0, 2, 2)


def test_save_bytes_match_oracle(E, rng, tmp_path):
    for (nl, nh, hd, L, lmax) in [(2, 4, 128, 32, 32), (1, 3, 64, 10, 16)]:
        g, o = pair(E, nl, nh, hd, lmax)
        data = rng.standard_normal(nl * 2 * nh * L * hd).astype(np.float32)
        g.load_raw(data, L)
        o.load_raw(data, L)
        pg, po = tmp_path / "g.eakv", tmp_path / "o.eakv"
        g.save(str(pg))
        o.save(str(po))
        assert pg.read_bytes() == po.read_bytes()
        h = E.Cache.load(str(po))
        q = rng.standard_normal((nh, hd)).astype(np.float32)
        assert np.array_equal(h.attention_scores(q, 0, nh, nh), o.attention_scores(q, 0, nh, nh))


@pytest.mark.parametrize("d,n_q,n_kv,L", [(128, 32, 8, 5000), (64, 32, 4, 3000),
                                          (128, 32, 32, 2100), (128, 64, 8, 2500)])
def test_fused_parity_config_distributions(E, rng, d, n_q, n_kv, L):
    """Channel scales log-uniform in [0.5, 4] with two x10 outlier channels per
    head (K), and 1% +-20 outliers (V): the magnitudes of the benchmark
    configurations, at a context the oracle finishes quickly."""
    say("fused-dist", d, n_q, n_kv, L)
    nl = 1
    ch = np.exp(rng.uniform(np.log(0.5), np.log(4.0), (n_kv, d))).astype(np.float32)
    for h in range(n_kv):
        ch[h, rng.choice(d, 2, replace=False)] *= 10
    K = rng.standard_normal((n_kv, L, d)).astype(np.float32) * ch[:, None, :]
    V = rng.standard_normal((n_kv, L, d)).astype(np.float32)
    out_mask = rng.random(V.shape) < 0.01
    V[out_mask] = np.where(rng.random(out_mask.sum()) < 0.5, -20.0, 20.0)
    data = np.stack([K, V])[None].astype(np.float32)
    g, o = pair(E, nl, n_kv, d, L + 8)
    g.load_raw(data, L)
    o.load_raw(data, L)
    q = rng.standard_normal((n_q, d)).astype(np.float32)
    a = g.attention_fused(q, 0, n_q, n_kv)
    b = o.attention_fused(q, 0, n_q, n_kv)
    ok, err, nbad = tol_close(a, b, ATOL, RTOL)
    assert ok, (err, nbad)
    sa = g.attention_scores(q, 0, n_q, n_kv)
    assert np.array_equal(sa, o.attention_scores(q, 0, n_q, n_kv))


# ------------------------------------------------- dequantize range, validate

@pytest.mark.parametrize("nh,d,L,lmax", [(2, 128, 37, 40), (3, 64, 100, 128), (1, 64, 1, 1)])
def test_dequantize_range_bitexact(E, rng, nh, d, L, lmax):
    """GPU dequantization of plane ranges equals the oracle's bit for bit
    (fma(nibble, scale, bias)), host and device forms, including ranges at
    the plane's ends and ranges over never-written groups."""
    say("dequantize", nh, d, L, lmax)
    g, o = loaded(E, rng, nh, d, L, lmax)
    ng = nh * lmax * d // 64
    for layer, kv in [(0, 0), (1, 1)]:
        w, s, b = o.read_planes(layer, kv)
        for g0, n in [(0, ng), (0, 1), (ng - 1, 1), (ng // 3, ng // 2), (5 % ng, 0)]:
            got = g.dequantize_range(layer, kv, g0, n)
            assert np.array_equal(got, O.dequantize_range(w, s, b, g0, n)), (layer, kv, g0, n)
    from eakv_amd.hipmem import DeviceArray
    d_out = DeviceArray((ng, 64))
    assert E.lib().eakv_dequantize_range_device(g.h, 1, 0, 0, ng, d_out.ptr, None) == 0
    g.sync()
    w, s, b = o.read_planes(1, 0)
    assert np.array_equal(d_out.download(), O.dequantize_range(w, s, b, 0, ng))
    L_ = E.lib()
    for args in [(2, 0, 0, 1), (0, 2, 0, 1), (0, 0, -1, 1), (0, 0, ng, 1), (0, 0, 0, ng + 1)]:
        assert L_.eakv_dequantize_range_device(g.h, *args, d_out.ptr, None) == E.EAKV_ERR_INVALID
    g.free()
    o.free()


def test_validate_matches_oracle(E, rng, tmp_path):
    """Corrupt values planted in an oracle cache travel through an .eakv file
    to the GPU; eakv_validate reports the reference's code per block (first
    failing group of the first n_kv*d*seq_len/64 groups), as the oracle does
    on the same file (a file's caches have max_seq_len = seq_len, so the
    plane layout differs from the cache that wrote it), before and after a
    restore shortens the checked range."""
    nl, nh, d, L, lmax = 4, 3, 128, 50, 64
    o = O.OracleCache(nl, nh, d, lmax)
    o.load_raw(rng.standard_normal((nl, 2, nh, L, d)).astype(np.float32), L)
    n = nh * d * L // 64
    plant = {(0, 1): ("s", 7, np.float32(np.nan)),             # 1: NaN scale
             (1, 0): ("b", n - 1, np.float32(np.nan)),         # 2: NaN bias, last group
             (2, 0): ("s", 0, np.float32(-3.0)),               # 3: negative scale
             (2, 1): ("b", n, np.float32(np.nan)),             # beyond the range: ok
             (3, 1): ("s", 10, np.float32(-np.inf))}           # 3: -inf scale
    for (layer, kv), (which, gi, v) in plant.items():
        _, s, b = o.plane_views(layer, kv)
        (s if which == "s" else b)[gi] = v
    _, s, b = o.plane_views(3, 1)
    b[4] = np.float32(np.nan)                                  # earlier group wins: 2
    assert o.validate().tolist() == [0, 1, 2, 0, 3, 0, 0, 2]
    path = tmp_path / "planted.eakv"
    o.save(str(path))
    g = E.Cache.load(str(path))
    o2 = O.OracleCache.load(str(path))
    want = o2.validate()
    assert want.tolist() == [0, 1, 2, 0, 3, 2, 0, 2]        # (2,1)'s group is in range now
    assert g.validate().tolist() == want.tolist()
    for sl in (40, 1, 0):
        g.restore(sl)
        o2.restore(sl)
        assert g.validate().tolist() == o2.validate().tolist(), sl
    g.free()
    o.free()
    o2.free()


def test_validate_nan_input_gives_nan_bias(E, rng):
    """A group whose first value is NaN quantizes to bias NaN (the min scan
    starts from element 0): validate says 2 on the GPU and in the oracle."""
    nl, nh, d, L = 1, 2, 64, 8
    data = rng.standard_normal((nl, 2, nh, L, d)).astype(np.float32)
    data[0, 1, 1, 3, 0] = np.nan
    g, o = pair(E, nl, nh, d, L)
    g.load_raw(data, L)
    o.load_raw(data, L)
    assert o.validate().tolist() == [0, 2]
    assert g.validate().tolist() == [0, 2]
    g.clear()
    assert g.validate().tolist() == [0, 0]                     # no groups checked
    g.free()
    o.free()


# -------------------------------------------------------- ggml block type

@pytest.mark.parametrize("nb,nrc,off", [(1, 1, 0), (333, 5, 0), (4096, 2, 4), (17, 64, 4)])
def test_ggml_rows_bitexact(E, rng, nb, nrc, off):
    """eakv_ggml_* against the oracle's restatement of ggml_type.c, bit for
    bit: quantize (scalar-path min/max), dequantize and vec_dot (AVX-512
    path arithmetic), with 4-byte (not 16-byte) aligned buffers when off = 4,
    a shared f32 row (by = 0) and several rows per call."""
    from eakv_amd.hipmem import DeviceArray
    say("ggml", nb, nrc, off)
    L = E.lib()
    x = (rng.standard_normal(nb * 64) * np.exp(rng.uniform(-5, 5))).astype(np.float32)
    x[rng.integers(0, x.size, 3)] = 0.0
    pad = off // 4
    dx = DeviceArray.from_host(np.concatenate([np.zeros(pad, np.float32), x]))
    db = DeviceArray((nb * 40 + off,), np.uint8)
    assert L.eakv_ggml_quantize_row_device(dx.ptr + off, db.ptr + off, x.size, None) == 0
    dd = DeviceArray((x.size + pad,))
    assert L.eakv_ggml_dequantize_row_device(db.ptr + off, dd.ptr + off, x.size, None) == 0
    E.hipmem.synchronize()
    blocks = db.download()[off:].reshape(nb, 40)
    assert np.array_equal(blocks, O.ggml_quantize_row(x))
    assert np.array_equal(dd.download()[pad:].view(np.uint32),
                          O.ggml_dequantize_row(blocks).view(np.uint32))
    n = nb * 64
    vx = np.stack([O.ggml_quantize_row(rng.standard_normal(n).astype(np.float32)).reshape(-1)
                   for _ in range(nrc)])
    vy = rng.standard_normal((nrc, n)).astype(np.float32)
    dvx, dvy = DeviceArray.from_host(vx), DeviceArray.from_host(vy)
    ds = DeviceArray((nrc,))
    assert L.eakv_ggml_vec_dot_device(n, ds.ptr, 4, dvx.ptr, vx.shape[1], dvy.ptr, n * 4, nrc,
                                      None) == 0
    ds0 = DeviceArray((nrc,))
    assert L.eakv_ggml_vec_dot_device(n, ds0.ptr, 4, dvx.ptr, vx.shape[1], dvy.ptr, 0, nrc,
                                      None) == 0
    E.hipmem.synchronize()
    assert np.array_equal(ds.download().view(np.uint32), O.ggml_vec_dot(vx, vy).view(np.uint32))
    shared = O.ggml_vec_dot(vx, np.repeat(vy[:1], nrc, axis=0))
    assert np.array_equal(ds0.download().view(np.uint32), shared.view(np.uint32))


def test_ggml_rejects_bad_arguments(E):
    from eakv_amd.hipmem import DeviceArray
    L = E.lib()
    d = DeviceArray((1024,))
    assert L.eakv_ggml_quantize_row_device(d.ptr, d.ptr + 2048, 100, None) == E.EAKV_ERR_INVALID
    assert L.eakv_ggml_quantize_row_device(d.ptr + 2, d.ptr + 2048, 64, None) == E.EAKV_ERR_INVALID
    assert L.eakv_ggml_dequantize_row_device(d.ptr, d.ptr + 1, 64, None) == E.EAKV_ERR_INVALID
    assert L.eakv_ggml_vec_dot_device(64, d.ptr, 2, d.ptr, 40, d.ptr, 256, 2,
                                      None) == E.EAKV_ERR_INVALID
    assert L.eakv_ggml_quantize_row_device(None, None, 0, None) == 0


# ----------------------------------------------------------------- full size

@pytest.mark.parametrize("n_kv,n_q,L", [(8, 32, 32768), (2, 16, 131072)])
def test_fused_full_size_matches_oracle(E, n_kv, n_q, L):
    """The benchmark's context lengths: one sequence of the 32Q/8KV 32K
    workload, and 131072 tokens at 8 q heads per kv head (the 64Q/8KV
    workload's ratio and length, 2 of its 8 kv heads), against the oracle."""
    say("fused-full", n_kv, n_q, L)
    rng = np.random.default_rng(L + n_kv)
    data = rng.standard_normal((1, 2, n_kv, L, 128), dtype=np.float32)
    g, o = pair(E, 1, n_kv, 128, L)
    g.load_raw(data, L)
    o.load_raw(data, L)
    del data
    q = rng.standard_normal((n_q, 128), dtype=np.float32)
    ok, err, nbad = tol_close(g.attention_fused(q, 0, n_q, n_kv),
                              o.attention_fused(q, 0, n_q, n_kv), ATOL, RTOL)
    assert ok, (err, nbad)
    g.free()
    o.free()


def test_fused_full_size_zero_query_is_mean_of_v(E):
    """q = 0 gives every token the same score, so the output is the mean of
    the dequantized V rows over all 131072 tokens (f64 reference from the
    cache's own planes)."""
    n_kv, n_q, L, d = 2, 16, 131072, 128
    rng = np.random.default_rng(7)
    data = (rng.standard_normal((1, 2, n_kv, L, d), dtype=np.float32) * 3).astype(np.float32)
    g = E.Cache(1, n_kv, d, L)
    g.load_raw(data, L)
    del data
    out = g.attention_fused(np.zeros((n_q, d), np.float32), 0, n_q, n_kv)
    vw, vs, vb = g.read_planes(0, 1)
    V = O.dequantize(vw, vs, vb).reshape(n_kv, L, d).astype(np.float64)
    want = np.repeat(V.mean(axis=1), n_q // n_kv, axis=0)
    ok, err, nbad = tol_close(out, want, ATOL, RTOL)
    assert ok, (err, nbad)
    g.free()
