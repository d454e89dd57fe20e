"""GPU parity at the benchmark workloads' own shapes and on the routes the
smaller cases do not reach, through the C ABI against the CPU oracle.

- The unfused API path (scores -> row softmax -> output) at the shapes of the
  five workloads: 8Q/8KV d128 2048 tokens, 32Q/4KV d64 4096 tokens (22
  layers), 32Q/32KV d128 8192 tokens, 32Q/8KV d128 32768 tokens, and the
  MHA d64 V-sum over several 256-token chunks.
- The 80-layer, 64Q/8KV, 131136-token geometry of the 70B-shape workload:
  a cache of 13.4 GB whose last layer block lies beyond 4 GiB of the base.
- Caches whose (layer, kv) block exceeds 1 GiB (the kernels' 32-bit buffer
  offsets no longer cover a layer): the VALU programs.
- The chunk merge for more than 16 chunks under NaN and moving maxima.
- Batched calls ordered after work enqueued on the other caches' streams.

Bars as everywhere: quantized planes and K-scores bit-exact; V-sum and fused
outputs within |gpu - oracle| <= 1e-4 + 1e-5*|oracle|.
"""
import ctypes as C
import os

import numpy as np
import pytest

import oracle as O
from conftest import check_against_reference, tol_close

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-4, 1e-5
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def E():
    import eakv_amd
    from eakv_amd import hipmem
    if hipmem.device_count() < 1:
        pytest.fail("no HIP device visible")
    return eakv_amd


def say(*a):
    print(*a, flush=True)


def pair(E, nl, nh, hd, lmax):
    return E.Cache(nl, nh, hd, lmax), O.OracleCache(nl, nh, hd, lmax)


def n_cu():
    lib = C.CDLL(os.path.join(ROOT, "eakv_amd", "libeakv_synth.so"))
    lib.eakv_synth_cu_count.restype = C.c_int
    return lib.eakv_synth_cu_count() or 256


def mfma_chunks(L, units, qpk, d):
    """Chunks per (sequence, kv head) of the fused matrix-core program: the
    launch rule of fused.hip's mfma_blocks_per_unit (chunks of at least 512
    tokens, 256 when that leaves fewer blocks than CUs; resident blocks per
    CU: 2 for up to 4 q heads per kv head, else 1 at d=128, 2 at d=64)."""
    per_cu = 2 if qpk <= 4 else (1 if d == 128 else 2)
    cu = n_cu()
    slots = cu * per_cu
    nb = 1 if units >= slots else slots // units
    coarse = -(-L // 512)
    cap = -(-L // 256) if units * coarse < cu else coarse
    return max(1, min(nb, cap))


def unfused_check(g, o, q, layer, n_q, n_kv, rng, signed=True):
    """Scores bit-exact; softmax rows of the oracle's scores through both
    V-sums within the bar; signed, unnormalised weights within the bound of
    a plain f32 sum against the exact f64 value."""
    sg = g.attention_scores(q, layer, n_q, n_kv)
    so = o.attention_scores(q, layer, n_q, n_kv)
    assert np.array_equal(sg.view(np.uint32), so.view(np.uint32)), np.abs(sg - so).max()
    w = O.softmax_rows(so)
    ok, err, nbad = tol_close(g.attention_output(w, layer, n_q, n_kv),
                              o.attention_output(w, layer, n_q, n_kv), ATOL, RTOL)
    assert ok, (err, nbad)
    if not signed:
        return
    L = sg.shape[1]
    d = q.shape[1]
    w2 = (rng.standard_normal((n_q, L)) * np.exp(rng.uniform(-3, 0, (n_q, 1)))).astype(np.float32)
    vw, vs, vb = o.read_planes(layer, 1)
    nh, lmax = o.n_heads, o.max_seq_len
    Vd = O.dequantize(vw, vs, vb).reshape(nh, lmax, d)[:n_kv, :L].astype(np.float64)
    qpk = n_q // n_kv
    for got in (g.attention_output(w2, layer, n_q, n_kv), o.attention_output(w2, layer, n_q, n_kv)):
        for h in range(n_q):
            ex = w2[h].astype(np.float64) @ Vd[h // qpk]
            mag = np.abs(w2[h].astype(np.float64)) @ np.abs(Vd[h // qpk])
            err = np.abs(got[h] - ex)
            assert np.all(err <= 1e-4 + 4e-7 * mag), (h, err.max())
    # a NaN weight poisons its head only, as in the reference's fma chain
    w2[n_q - 1, L // 2] = np.nan
    got = g.attention_output(w2, layer, n_q, n_kv)
    assert np.isnan(got[n_q - 1]).all()
    assert np.isfinite(got[: n_q - 1]).all()


# ------------------------------------------------------- unfused at workloads

@pytest.mark.parametrize("name,nl,nh,n_q,d,L,layer", [
    ("8q8kv-d128-2048", 1, 8, 8, 128, 2048, 0),
    ("32q4kv-d64-4096-22layers", 22, 4, 32, 64, 4096, 21),
    ("32q32kv-d128-8192", 1, 32, 32, 128, 8192, 0),
    ("32q8kv-d128-32768", 1, 8, 32, 128, 32768, 0),
    ("mha-d64-1500", 1, 4, 4, 64, 1500, 0),
    ("mha-d128-5000", 2, 2, 2, 128, 5000, 1),
    ("mha-d128-40000", 1, 2, 2, 128, 40000, 0),
    ("mha-d64-70000", 1, 2, 2, 64, 70000, 0),
])
def test_unfused_at_workload_shapes(E, rng, name, nl, nh, n_q, d, L, layer):
    """The reference API's unfused step at the benchmark shapes.  The MHA
    V-sums cover 512-token chunks at d128 and 1024-token chunks at d64: 4
    (2048 tokens), 16 (8192), 2 (d64 1500), 10 (5000), 79 (40000) and 69
    (d64 70000) chunk partials, added by the last block of each kv head in
    batches of 16, so the partials, the counters and the fixed-order sum are
    all exercised, on every call of unfused_check again."""
    say("unfused", name)
    data = (rng.standard_normal(nl * 2 * nh * L * d) * 1.5).astype(np.float32)
    g, o = pair(E, nl, nh, d, L)
    g.load_raw(data, L)
    o.load_raw(data, L)
    del data
    q = rng.standard_normal((n_q, d)).astype(np.float32)
    unfused_check(g, o, q, layer, n_q, nh, rng)
    g.free()
    o.free()


@pytest.mark.parametrize("name,nh,n_q,d,L", [
    ("8q8kv-d128-2048", 8, 8, 128, 2048), ("32q32kv-d128-8192", 32, 32, 128, 8192),
    ("mha-d64-1500", 4, 4, 64, 1500)])
def test_fused_mha_at_workload_shapes(E, rng, name, nh, n_q, d, L):
    say("fused-mha", name)
    data = rng.standard_normal(2 * nh * L * d).astype(np.float32)
    g, o = pair(E, 1, nh, d, L)
    g.load_raw(data, L)
    o.load_raw(data, L)
    q = (rng.standard_normal((n_q, d)) * 2).astype(np.float32)
    ok, err, nbad = tol_close(g.attention_fused(q, 0, n_q, nh),
                              o.attention_fused(q, 0, n_q, nh), ATOL, RTOL)
    assert ok, (err, nbad)


# ------------------------------------------------------------ 70B geometry

def chan_outlier(rng, n_kv, L, d):
    """K or V of the 70B-shape workload: N(0,1) times per-channel scales
    log-uniform in [0.25, 8], 1% of the values replaced by +-20."""
    ch = np.exp(rng.uniform(np.log(0.25), np.log(8.0), (n_kv, 1, d))).astype(np.float32)
    x = rng.standard_normal((n_kv, L, d), dtype=np.float32) * ch
    m = rng.random(x.shape, dtype=np.float32) < 0.01
    x[m] = np.where(rng.random(int(m.sum())) < 0.5, -20.0, 20.0).astype(np.float32)
    return x


def exact_attention(o, q, layer, n_q, n_kv, L):
    """softmax(q.K/sqrt(d)) V in f64 over the oracle cache's quantized planes
    (K and V = nibble*scale + bias exactly, the exact max and sum)."""
    nh, d, lmax = o.n_heads, o.head_dim, o.max_seq_len
    kv = []
    for k in (0, 1):
        w, s, b = o.read_planes(layer, k)
        n = np.concatenate([w & 15, w >> 4], axis=1).astype(np.float64)
        x = n * s.astype(np.float64)[:, None] + b.astype(np.float64)[:, None]
        kv.append(x.reshape(nh, lmax, d)[:n_kv, :L])
        del w, s, b, n, x
    K, V = kv
    qpk = n_q // n_kv
    out = np.zeros((n_q, d))
    for h in range(n_q):
        sc = K[h // qpk] @ q[h].astype(np.float64) / np.sqrt(d)
        p = np.exp(sc - sc.max())
        out[h] = p @ V[h // qpk] / p.sum()
    return out


def fused_against_exact(g, o, q, layer_g, n_q, n_kv, L, expect_exception=None):
    """Fused attention against the reference algorithm (the oracle's fused
    call, its AVX-512 form where the host has one) at the bar of 1e-4 abs /
    1e-5 rel, with the exception asserted by check_against_reference: over
    long contexts with sharp softmax rows the reference's single f32 sum of
    the weights (fused_attention.ea:280-359: sum = sum + w, token after
    token) drops the terms below half an ulp of the running sum (at 131072
    tokens of the 70B-shape data it is up to 0.03% low, which moves outputs
    of magnitude 18 by 5e-3); where the GPU misses the bar against the
    reference it must be closer than the reference to the exact f64
    attention, it must meet the bar against exact everywhere and lie no
    farther from the reference than the reference from exact, plus the bar.
    expect_exception: True / False asserts which of the two held."""
    exact = exact_attention(o, q, 0, n_q, n_kv, L)
    got = g.attention_fused(q, layer_g, n_q, n_kv)
    ref = o.attention_fused_avx512(q, 0, n_q, n_kv) if O.avx512_available() \
        else o.attention_fused(q, 0, n_q, n_kv)
    mode, e_gr, e_re, e_ge, n_ex, ref_bar = check_against_reference(got, ref, exact, ATOL, RTOL)
    say("  fused:", mode, "bar; gpu-reference", e_gr, "reference-exact", e_re,
        f"({ref_bar:.3f} of the bar)", "gpu-exact", e_ge, "values excused", n_ex)
    if expect_exception is not None:
        assert (mode == "exact") == expect_exception, mode


def test_70b_geometry_last_layer(E):
    """An 80-layer cache of 8 kv heads, head_dim 128 and max_seq_len 131136
    (13.4 GB): layer 79's blocks start 13.3 GB past the base.  Layer 79 is
    filled through the host append at the full 131072-token context with the
    workload's distribution; its planes must equal a 1-layer oracle cache fed
    the same data, bit for bit, K-scores must be bit-exact and the V-sum of
    the oracle's softmax rows within the bar.  Fused attention is held to the
    exact result (fused_against_exact: the reference algorithm itself misses
    the bar here)."""
    nl, nkv, d, lmax, L, n_q = 80, 8, 128, 131136, 131072, 64
    rng = np.random.default_rng(0xEA4B + 5)
    say("70b-geometry: create", nl, nkv, d, lmax)
    g = E.Cache(nl, nkv, d, lmax)
    o = O.OracleCache(1, nkv, d, lmax)
    for kv in (0, 1):
        x = chan_outlier(rng, nkv, L, d)
        say("70b-geometry: append layer 79 kv", kv)
        g.append(x, 79, kv, L)
        o.append(x, 0, kv, L)
        del x
    g.advance(L)
    o.advance(L)
    for kv in (0, 1):
        a, b = g.read_planes(79, kv), o.read_planes(0, kv)
        for x, y in zip(a, b):
            assert np.array_equal(np.ascontiguousarray(x).view(np.uint8),
                                  np.ascontiguousarray(y).view(np.uint8)), kv
        del a
    q = rng.standard_normal((n_q, d), dtype=np.float32)
    say("70b-geometry: scores")
    sg = g.attention_scores(q, 79, n_q, nkv)
    so = o.attention_scores(q, 0, n_q, nkv)
    assert np.array_equal(sg.view(np.uint32), so.view(np.uint32)), np.abs(sg - so).max()
    w = O.softmax_rows(so)
    del sg, so
    say("70b-geometry: output")
    ok, err, nbad = tol_close(g.attention_output(w, 79, n_q, nkv),
                              o.attention_output(w, 0, n_q, nkv), ATOL, RTOL)
    assert ok, (err, nbad)
    del w
    say("70b-geometry: fused")
    fused_against_exact(g, o, q, 79, n_q, nkv, L, expect_exception=True)
    # layer 0 was never written: zero planes, zero scores
    assert not g.attention_scores(q, 0, n_q, nkv).any()
    g.free()
    o.free()


def test_32k_workload_distribution_fused(E):
    """One sequence of the 32Q/8KV d128 32768-token workload with its K
    distribution (channel scales log-uniform in [0.5, 4], two x10 channels
    per head) and V ~ N(0,1): fused attention against the exact result and
    the reference algorithm's error beside it."""
    nkv, d, L, n_q = 8, 128, 32768, 32
    rng = np.random.default_rng(0xEA4B + 4)
    ch = np.exp(rng.uniform(np.log(0.5), np.log(4.0), (nkv, 1, d))).astype(np.float32)
    for h in range(nkv):
        ch[h, 0, rng.choice(d, 2, replace=False)] *= 10
    K = rng.standard_normal((nkv, L, d), dtype=np.float32) * ch
    V = rng.standard_normal((nkv, L, d), dtype=np.float32)
    g, o = pair(E, 1, nkv, d, L)
    for kv, x in ((0, K), (1, V)):
        g.append(x, 0, kv, L)
        o.append(x, 0, kv, L)
    del K, V
    g.advance(L)
    o.advance(L)
    q = rng.standard_normal((n_q, d), dtype=np.float32)
    say("32k-distribution: fused")
    fused_against_exact(g, o, q, 0, n_q, nkv, L)
    g.free()
    o.free()


# ------------------------------------------------------ blocks beyond 1 GiB

@pytest.mark.parametrize("nkv,n_q,d,lmax,L", [(2, 16, 128, 7_000_000, 3000),
                                              (4, 4, 64, 7_000_000, 1700)])
def test_blocks_beyond_1gib(E, rng, nkv, n_q, d, lmax, L):
    """A max_seq_len of 7M tokens makes each (layer, kv) block larger than
    1 GiB, past what the matrix-core programs address with 32-bit buffer
    offsets, so fused attention and the V-sum take the VALU programs.  A short
    context against an oracle cache of the same data."""
    say("big-block", nkv, n_q, d, lmax, L)
    data = rng.standard_normal(2 * nkv * L * d).astype(np.float32)
    g = E.Cache(1, nkv, d, lmax)
    o = O.OracleCache(1, nkv, d, L)
    g.load_raw(data, L)
    o.load_raw(data, L)
    q = (rng.standard_normal((n_q, d)) * 2).astype(np.float32)
    ok, err, nbad = tol_close(g.attention_fused(q, 0, n_q, nkv),
                              o.attention_fused(q, 0, n_q, nkv), ATOL, RTOL)
    assert ok, (err, nbad)
    unfused_check(g, o, q, 0, n_q, nkv, rng, signed=False)
    g.free()


# -------------------------------------------- long contexts: 8-part merge

def tile_tokens(L, units, qpk, d):
    """Tokens per tile of the fused matrix-core program (fused.hip's
    tile_tokens): 64 where waves serve two quads (5-8 q heads per kv head)
    and each of the unit's 8 waves per chunk gets at least 4 tiles of 64,
    else 32."""
    mc = mfma_chunks(L, units, qpk, d)
    return 64 if qpk > 4 and -(-L // 64) >= 4 * mc * 8 else 32


# ------------------------------------------ 64-token tiles (two-quad waves)

@pytest.mark.parametrize("d,n_q,n_kv,L,case", [
    (128, 64, 8, 65536 + 37, "random"), (128, 48, 8, 70000, "nan-v"),
    (128, 64, 8, 66000, "slope"), (64, 128, 16, 65600, "random")])
def test_64_token_tiles(E, rng, d, n_q, n_kv, L, case):
    """Long contexts at 6-8 q heads per kv head run 64-token tiles (one
    16x16x64 V product and one recombination per 64 tokens).  Fused
    attention against the oracle with a ragged last tile, a NaN V value,
    scores that rise along the context (the running max moves), and the
    V-sum mode with signed weights (the V-sum's grid has the same chunks,
    so it runs 64-token tiles too)."""
    assert tile_tokens(L, n_kv, n_q // n_kv, d) == 64
    say("tt64", d, n_q, n_kv, L, case)
    if case == "slope":
        u = rng.standard_normal((n_kv, d))
        u /= np.linalg.norm(u, axis=1, keepdims=True)
        t = np.arange(L, dtype=np.float64) - L / 2
        K = (0.0015 * t)[None, :, None] * u[:, None, :] + 0.1 * rng.standard_normal((n_kv, L, d))
        data = np.stack([K, rng.standard_normal((n_kv, L, d))])[None].astype(np.float32)
        q = (np.repeat(u, n_q // n_kv, axis=0) * np.sqrt(d) +
             0.3 * rng.standard_normal((n_q, d))).astype(np.float32)
    else:
        data = rng.standard_normal((1, 2, n_kv, L, d)).astype(np.float32)
        q = rng.standard_normal((n_q, d)).astype(np.float32)
    if case == "nan-v":
        # the first value of a group (the quantizer's scan carries a NaN
        # only from there): that group's 64 dims of kv head 3 turn NaN
        data[0, 1, 3, L - 5, 64] = np.nan
    g, o = pair(E, 1, n_kv, d, L + 8)
    g.load_raw(data, L)
    o.load_raw(data, L)
    a = g.attention_fused(q, 0, n_q, n_kv)
    b = o.attention_fused(q, 0, n_q, n_kv)
    nan = np.isnan(b)
    assert nan.any() == (case == "nan-v")
    assert np.array_equal(np.isnan(a), nan)
    ok, err, nbad = tol_close(a[~nan], b[~nan], ATOL, RTOL)
    assert ok, (err, nbad)
    if case == "random":
        unfused_check(g, o, q, 0, n_q, n_kv, rng, signed=True)
    g.free()


@pytest.mark.parametrize("d,n_q,n_kv,L,where", [(128, 8, 2, 8192, "k"), (128, 16, 2, 4600, "v"),
                                                (64, 8, 2, 6000, "v")])
def test_long_context_nonfinite_values(E, rng, d, n_q, n_kv, L, where):
    """A NaN first value of a group in K (every output of the kv head's q heads
    NaN) or V (that group's 64 dims NaN) with more than 16 chunks per
    sequence, so the chunk merge is the 8-part one."""
    assert mfma_chunks(L, n_kv, n_q // n_kv, d) > 16
    say("long-nan", d, n_q, n_kv, L, where)
    data = rng.standard_normal((1, 2, n_kv, L, d)).astype(np.float32)
    data[0, 0 if where == "k" else 1, 1, (2 * L) // 3, 0] = np.nan
    g, o = pair(E, 1, n_kv, d, L + 4)
    g.load_raw(data, L)
    o.load_raw(data, L)
    q = rng.standard_normal((n_q, d)).astype(np.float32)
    a = g.attention_fused(q, 0, n_q, n_kv)
    b = o.attention_fused(q, 0, n_q, n_kv)
    nan = np.isnan(b)
    assert nan.any() and not nan.all()
    assert np.array_equal(np.isnan(a), nan)
    ok, err, nbad = tol_close(a[~nan], b[~nan], ATOL, RTOL)
    assert ok, (err, nbad)


@pytest.mark.parametrize("d,n_q,n_kv,L,slope", [(128, 8, 2, 8192, 0.01), (128, 16, 2, 4608, -0.02),
                                                (64, 8, 2, 6000, 0.015)])
def test_long_context_moving_max(E, rng, d, n_q, n_kv, L, slope):
    """Scores rising (the running max moves in chunk after chunk) or falling
    over a context of more than 16 chunks: the 8-part merge rescales every
    part to the common max."""
    assert mfma_chunks(L, n_kv, n_q // n_kv, d) > 16
    say("long-slope", d, n_q, n_kv, L, slope)
    u = rng.standard_normal((n_kv, d))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    t = np.arange(L, dtype=np.float64) - L / 2
    K = (slope * t)[None, :, None] * u[:, None, :] + 0.1 * rng.standard_normal((n_kv, L, d))
    V = rng.standard_normal((n_kv, L, d))
    data = np.stack([K, V])[None].astype(np.float32)
    g, o = pair(E, 1, n_kv, d, L + 8)
    g.load_raw(data, L)
    o.load_raw(data, L)
    q = (np.repeat(u, n_q // n_kv, axis=0) * np.sqrt(d) +
         0.3 * rng.standard_normal((n_q, d))).astype(np.float32)
    sc = o.attention_scores(q, 0, n_q, n_kv)
    assert np.abs(sc).max() < 160
    assert abs(float(sc[:, -1].mean() - sc[:, 0].mean())) > 0.5 * abs(slope) * L
    a = g.attention_fused(q, 0, n_q, n_kv)
    assert np.isfinite(a).all()
    ok, err, nbad = tol_close(a, o.attention_fused(q, 0, n_q, n_kv), ATOL, RTOL)
    assert ok, (err, nbad)


# ------------------------------------------------- batched calls and streams

def test_batch_fused_waits_for_other_caches_streams(E, rng):
    """Appends enqueued with a NULL stream on caches 1 and 3 run on those
    caches' own streams; a batched fused call right behind them, on caches[0]'s
    stream, must see the appended tokens."""
    from eakv_amd.hipmem import DeviceArray
    nl, nh, d, n_q, L0, n_new = 1, 2, 128, 8, 1000, 4000
    gs, os_ = [], []
    for _ in range(4):
        data = rng.standard_normal(nl * 2 * nh * L0 * d).astype(np.float32)
        g, o = pair(E, nl, nh, d, L0 + n_new)
        g.load_raw(data, L0)
        o.load_raw(data, L0)
        gs.append(g)
        os_.append(o)
    keep = []
    for i in (1, 3):
        for kv in (0, 1):
            x = rng.standard_normal((nh, n_new, d)).astype(np.float32)
            dx = DeviceArray.from_host(x)
            keep.append(dx)
            assert E.lib().eakv_cache_append_device(gs[i].h, dx.ptr, 0, kv, n_new, None) == 0
            os_[i].append(x, 0, kv, n_new)
        gs[i].advance(n_new)
        os_[i].advance(n_new)
    q = rng.standard_normal((4, n_q, d)).astype(np.float32)
    dq = DeviceArray.from_host(q)
    dout = DeviceArray((4, n_q, d))
    say("batch-order: fused")
    assert E.lib().eakv_attention_fused_batch_device(E.handles(gs), 4, 0, dq.ptr, n_q, nh,
                                                     dout.ptr, None) == 0
    gs[0].sync()
    out = dout.download()
    for i, o in enumerate(os_):
        ok, err, nbad = tol_close(out[i], o.attention_fused(q[i], 0, n_q, nh), ATOL, RTOL)
        assert ok, (i, err, nbad)


def test_batch_append_orders_later_calls_on_each_cache(E, rng):
    """A batched append (NULL stream: caches[0]'s) writes every cache; host
    calls on the other caches, which run on their own streams, come after
    it."""
    from eakv_amd.hipmem import DeviceArray
    nl, nh, d, n_q, L0, n_new, n = 2, 4, 64, 16, 500, 3000, 3
    gs, os_ = [], []
    for _ in range(n):
        data = rng.standard_normal(nl * 2 * nh * L0 * d).astype(np.float32)
        g, o = pair(E, nl, nh, d, L0 + n_new)
        g.load_raw(data, L0)
        o.load_raw(data, L0)
        gs.append(g)
        os_.append(o)
    x = rng.standard_normal((n, nl, 2, nh, n_new, d)).astype(np.float32)
    dx = DeviceArray.from_host(x)
    say("batch-order: append")
    assert E.lib().eakv_append_batch_device(E.handles(gs), n, dx.ptr, n_new, None) == 0
    for i in range(n):
        gs[i].advance(n_new)
        for l in range(nl):
            for kv in (0, 1):
                os_[i].append(x[i, l, kv], l, kv, n_new)
        os_[i].advance(n_new)
    q = rng.standard_normal((n_q, d)).astype(np.float32)
    for i in (2, 1):
        a = gs[i].attention_scores(q, 1, n_q, nh)
        b = os_[i].attention_scores(q, 1, n_q, nh)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), i


# ------------------------------------------------------------ .eakv files

@pytest.mark.parametrize("nl,nh,d,L,lmax", [(2, 4, 128, 32, 32), (3, 2, 128, 7, 20),
                                            (1, 3, 64, 10, 10)])
def test_gpu_file_layout_restated(E, rng, tmp_path, nl, nh, d, L, lmax):
    """The GPU library's .eakv bytes against the format restated from the
    reference's packed header struct (tests/eakv_format.py), not against the
    oracle's writer: header fields, index table, 64-byte blocks holding each
    head's first seq_len tokens."""
    import eakv_format as F
    g = E.Cache(nl, nh, d, lmax)
    g.load_raw(rng.standard_normal(nl * 2 * nh * L * d).astype(np.float32), L)
    p = tmp_path / "g.eakv"
    g.save(str(p))
    data = p.read_bytes()
    h, offs, n_groups = F.parse(data)
    assert (h["magic"], h["version"], h["quant_scheme"], h["group_size"]) == (b"EAKV", 1, 0, 64)
    assert (h["n_layers"], h["n_heads"], h["head_dim"], h["seq_len"], h["max_seq_len"]) == \
        (nl, nh, d, L, L)
    start = F.align64(F.HEADER_SIZE + 16 * nl)
    blk = F.align64(40 * n_groups)
    assert offs == [start + i * blk for i in range(2 * nl)]
    assert len(data) == start + 2 * nl * blk
    gpd = d // 64
    for i, off in enumerate(offs):
        w, s, b = g.read_planes(i // 2, i % 2)
        rows = lambda a, k: np.ascontiguousarray(
            a.reshape(nh, lmax * gpd, k)[:, :L * gpd]).tobytes()
        assert F.block(data, off, n_groups) == (rows(w, 32), rows(s.view(np.uint8), 4),
                                                rows(b.view(np.uint8), 4))


def test_gpu_loads_independently_built_file(E, rng, tmp_path):
    """Blocks in reverse order with gaps: the GPU loader follows the table;
    bad magic, version and a truncated block are format errors."""
    import eakv_format as F
    nl, nh, d, L = 2, 3, 128, 9
    ng = nh * d * L // 64
    blocks = [(rng.integers(0, 256, (ng, 32), dtype=np.uint8).tobytes(),
               rng.random(ng).astype(np.float32).tobytes(),
               rng.standard_normal(ng).astype(np.float32).tobytes()) for _ in range(2 * nl)]
    p = tmp_path / "x.eakv"
    p.write_bytes(F.build(nl, nh, d, L, blocks, order=reversed(range(2 * nl)), gap=192))
    g = E.Cache.load(str(p))
    assert (g.n_layers, g.n_heads, g.head_dim, g.seq_len, g.max_seq_len) == (nl, nh, d, L, L)
    for i in range(2 * nl):
        w, s, b = g.read_planes(i // 2, i % 2)
        assert (w.tobytes(), s.tobytes(), b.tobytes()) == blocks[i]
    for kw, cut in (({"magic": b"EAKW"}, 0), ({"version": 2}, 0), ({}, 100)):
        data = F.build(nl, nh, d, L, blocks, **kw)
        p.write_bytes(data[:len(data) - cut])
        with pytest.raises(E.EakvError) as e:
            E.Cache.load(str(p))
        assert e.value.code == E.EAKV_ERR_FORMAT


def test_bench_softmax_is_row_softmax(E, rng):
    """The caller's row softmax the benchmark times for the unfused workloads
    (libeakv_synth.so) against the oracle's, at every row length it uses
    (register-resident up to 16384 values, three passes beyond)."""
    from eakv_amd.hipmem import DeviceArray
    lib = C.CDLL(os.path.join(ROOT, "eakv_amd", "libeakv_synth.so"))
    lib.eakv_synth_softmax.restype = C.c_int
    lib.eakv_synth_softmax.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]
    for L in (1, 2048, 3000, 8192, 16384, 20000):
        s = (rng.standard_normal((5, L)) * 4).astype(np.float32)
        ds, dw = DeviceArray.from_host(s), DeviceArray((5, L))
        assert lib.eakv_synth_softmax(ds.ptr, dw.ptr, 5, L, None) == 0
        got = dw.download()
        # two f32 summation orders of up to 20000 weights: 1e-4 relative
        ok, err, nbad = tol_close(got, O.softmax_rows(s), 1e-7, 1e-4)
        assert ok, (L, err, nbad)
        assert abs(float(got.astype(np.float64).sum()) - 5.0) < 1e-3
