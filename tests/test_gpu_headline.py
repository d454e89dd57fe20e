"""The headline launch exactly as the benchmark times it, against the CPU
oracle through the C ABI.

The 32Q/8KV d128 32K-context workload's step: 8 sequences whose caches hold
32767 tokens, one token appended to each by one batched append, then one
eakv_attention_fused_batch_device call over all 8 caches (32 q heads, 8 kv
heads, 32768 tokens each).  On MI355X's 256 CUs that launch has 64 units
(sequence, kv head) of 8 chunks, merges its chunks inside the launch and
walks 32 tiles of 32 tokens per wave; the plan is read back from the library
(eakv_attention_fused_plan) and asserted, so the test checks the launch the
benchmark runs and not a neighbour of it.  The allocation-free form of the
same call (chunks merged by a second launch) must give the same bits.

Each sequence is compared with the reference algorithm (the oracle's fused
call, the AVX-512 restatement of fused_attention.ea:190-373 where the host
has AVX-512) at 1e-4 abs / 1e-5 rel, with the long-context exception
asserted by check_against_reference (the reference's f32 weight sum against
the exact f64 attention over the same quantized cache).

A second case runs single-quad waves through at least 16 tiles each at
other shapes (16 kv heads, ragged contexts, d=64), with the chunks merged in
the launch.
"""
import ctypes as C
import os
from concurrent.futures import ThreadPoolExecutor

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


def n_cu():
    lib = C.CDLL(os.path.join(ROOT, "eakv_amd", "libeakv_synth.so"))
    lib.eakv_synth_cu_count.restype = C.c_int
    return lib.eakv_synth_cu_count() or 256


def chan_k(rng, n_kv, L, d):
    """K of the 32Q/8KV workload: N(0,1) times per-channel scales log-uniform
    in [0.5, 4], two channels per head x10."""
    ch = np.exp(rng.uniform(np.log(0.5), np.log(4.0), (n_kv, 1, d))).astype(np.float32)
    for h in range(n_kv):
        ch[h, 0, rng.choice(d, 2, replace=False)] *= 10
    return rng.standard_normal((n_kv, L, d), dtype=np.float32) * ch


def exact_attention(o, q, n_q, n_kv, L):
    """softmax(q.K/sqrt(d)) V in f64 over layer 0 of the oracle cache's
    quantized planes (K and V = nibble*scale + bias exactly)."""
    nh, d, lmax = o.n_heads, o.head_dim, o.max_seq_len
    kv = []
    for k in (0, 1):
        w, s, b = o.read_planes(0, k)
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


# worker threads for the per-sequence CPU work (numpy's generators and the
# oracle library release the GIL)
POOL = 8


def build_batch(E, seed, n_seq, n_kv, d, lens, lmax, kdist):
    """n_seq one-layer caches (GPU and oracle) of lens[i] tokens each, every
    sequence seeded separately; K from kdist, V ~ N(0,1).  The inputs are
    drawn and the oracle caches filled on worker threads, the GPU caches
    loaded in order as their inputs arrive."""
    def make(i):
        rng = np.random.default_rng(seed + 1000 * i)
        L = lens[i]
        data = np.empty((2, n_kv, L, d), np.float32)
        data[0] = kdist(rng, n_kv, L, d)
        data[1] = rng.standard_normal((n_kv, L, d), dtype=np.float32)
        o = O.OracleCache(1, n_kv, d, lmax)
        o.load_raw(data, L)
        return data, o

    gs, os_ = [], []
    with ThreadPoolExecutor(POOL) as ex:
        for i, (data, o) in enumerate(ex.map(make, range(n_seq))):
            g = E.Cache(1, n_kv, d, lmax)
            g.load_raw(data, lens[i])
            del data
            gs.append(g)
            os_.append(o)
            say("  filled sequence", i, "tokens", lens[i])
    return gs, os_


def batch_call(E, fn, gs, q, n_q, n_kv):
    from eakv_amd.hipmem import DeviceArray
    dq = DeviceArray.from_host(q)
    dout = DeviceArray(q.shape)
    say("  call", fn, "n_seq", len(gs))
    assert getattr(E.lib(), fn)(E.handles(gs), len(gs), 0, dq.ptr, n_q, n_kv, dout.ptr,
                                None) == 0, E.last_error()
    gs[0].sync()
    out = dout.download()
    dq.free()
    dout.free()
    return out


def compare_sequences(os_, q, out, n_q, n_kv, lens):
    """Every sequence against the reference algorithm and the exact result
    (computed on worker threads), checked in order."""
    def refs(i):
        o = os_[i]
        ref = o.attention_fused_avx512(q[i], 0, n_q, n_kv) if O.avx512_available() \
            else o.attention_fused(q[i], 0, n_q, n_kv)
        return ref, exact_attention(o, q[i], n_q, n_kv, lens[i])

    modes = []
    with ThreadPoolExecutor(POOL) as ex:
        for i, (ref, exact) in enumerate(ex.map(refs, range(len(os_)))):
            mode, e_gr, e_re, e_ge, n_ex, ref_bar = check_against_reference(
                out[i], ref, exact, ATOL, RTOL)
            say(f"  sequence {i}: {mode} bar; gpu-reference {e_gr:.3g}, reference-exact "
                f"{e_re:.3g} ({ref_bar:.3f} of the bar), gpu-exact {e_ge:.3g}, "
                f"{n_ex} values excused")
            modes.append(mode)
    return modes


def test_headline_launch_as_benchmarked(E):
    """8 caches x 8 kv heads x 32768 tokens, 32 q heads, d=128: the
    benchmark's batched append of token 32768 and its one fused launch, with
    the launch plan asserted, both entry points, every sequence checked."""
    n_seq, n_kv, n_q, d, L0 = 8, 8, 32, 128, 32767
    lmax = L0 + 1 + 64                      # the benchmark's max_seq_len
    say("headline: build", n_seq, "caches of", L0, "tokens")
    gs, os_ = build_batch(E, 0xEA4B + 4, n_seq, n_kv, d, [L0] * n_seq, lmax, chan_k)
    from eakv_amd.hipmem import DeviceArray
    rng = np.random.default_rng(0xEA4B + 44)
    tok = rng.standard_normal((n_seq, 1, 2, n_kv, 1, d), dtype=np.float32)
    dtok = DeviceArray.from_host(tok)
    say("headline: batched append of one token")
    assert E.lib().eakv_append_batch_device(E.handles(gs), n_seq, dtok.ptr, 1, None) == 0
    for i in range(n_seq):
        gs[i].advance(1)
        for kv in (0, 1):
            os_[i].append(tok[i, 0, kv], 0, kv, 1)
        os_[i].advance(1)
    L = L0 + 1

    plan = E.fused_plan(gs, n_q, n_kv)
    say("headline: plan", plan)
    cu = n_cu()
    chunks = 2 * cu // (n_seq * n_kv)        # two one-quad blocks per CU, 64 units
    assert plan["mfma"] == 1 and plan["quads"] == 1 and plan["split"] == 1
    assert plan["waves_per_block"] == 4 and plan["tile_tokens"] == 32
    assert plan["chunks"] == chunks
    assert plan["merge_levels"] == 1
    assert plan["tiles_per_wave"] == -(-(L // 32) // (chunks * 4))
    if cu == 256:
        assert (plan["chunks"], plan["tiles_per_wave"]) == (8, 32)
    na_plan = E.fused_plan(gs, n_q, n_kv, noalloc=True)
    assert na_plan["merge_levels"] == 0
    assert {k: v for k, v in na_plan.items() if k != "merge_levels"} == \
        {k: v for k, v in plan.items() if k != "merge_levels"}

    q = rng.standard_normal((n_seq, n_q, d), dtype=np.float32)
    out = batch_call(E, "eakv_attention_fused_batch_device", gs, q, n_q, n_kv)
    out_na = batch_call(E, "eakv_attention_fused_batch_device_noalloc", gs, q, n_q, n_kv)
    # the in-launch merge restates the merge launch's arithmetic and order
    assert np.array_equal(out.view(np.uint32), out_na.view(np.uint32))
    # a second call of the workspace form: the counters were left at zero
    out2 = batch_call(E, "eakv_attention_fused_batch_device", gs, q, n_q, n_kv)
    assert np.array_equal(out.view(np.uint32), out2.view(np.uint32))
    compare_sequences(os_, q, out, n_q, n_kv, [L] * n_seq)
    # the appended token is in the launch: K-scores of its position,
    # bit-exact against the oracle for one sequence
    s_g = gs[5].attention_scores(q[5], 0, n_q, n_kv)
    s_o = os_[5].attention_scores(q[5], 0, n_q, n_kv)
    assert np.array_equal(s_g.view(np.uint32), s_o.view(np.uint32))
    dtok.free()
    for g in gs:
        g.free()


@pytest.mark.parametrize("d,n_kv,n_q,lens", [
    (128, 16, 64, [18000, 17001, 12345, 18000]),
    (64, 16, 32, [30000, 29999, 4097, 1])])
def test_single_quad_waves_many_tiles(E, d, n_kv, n_q, lens):
    """Single-quad waves (up to 4 q heads per kv head) through at least 16
    tiles each, chunks merged in the launch, ragged contexts in one batch
    (the shorter sequences' waves run out of tiles early and their blocks
    still count on the unit counters)."""
    n_seq = len(lens)
    say("many-tiles: build", d, n_kv, n_q, lens)
    gs, os_ = build_batch(E, 0xEA4B + 77 + d, n_seq, n_kv, d, lens, max(lens) + 8, chan_k)
    plan = E.fused_plan(gs, n_q, n_kv)
    say("many-tiles: plan", plan)
    assert plan["mfma"] == 1 and plan["quads"] == 1
    assert plan["merge_levels"] == 1
    assert plan["tiles_per_wave"] >= 16
    rng = np.random.default_rng(0xEA4B + 78 + d)
    q = rng.standard_normal((n_seq, n_q, d), dtype=np.float32)
    out = batch_call(E, "eakv_attention_fused_batch_device", gs, q, n_q, n_kv)
    out_na = batch_call(E, "eakv_attention_fused_batch_device_noalloc", gs, q, n_q, n_kv)
    assert np.array_equal(out.view(np.uint32), out_na.view(np.uint32))
    compare_sequences(os_, q, out, n_q, n_kv, lens)
    for g in gs:
        g.free()


def chan_outlier_kv(rng, L, d):
    """One kv head's K or V of the 70B-shape workload: N(0,1) times
    per-channel scales log-uniform in [0.25, 8], 1% of the values +-20."""
    ch = np.exp(rng.uniform(np.log(0.25), np.log(8.0), (1, d))).astype(np.float32)
    x = rng.standard_normal((L, d), dtype=np.float32) * ch
    m = rng.random(x.shape, dtype=np.float32) < 0.01
    x[m] = np.where(rng.random(int(m.sum())) < 0.5, -20.0, 20.0).astype(np.float32)
    return x


def exact_attention_by_head(o, q, n_q, n_kv, L):
    """exact_attention with one worker per kv head."""
    d, lmax = o.head_dim, o.max_seq_len
    planes = [o.read_planes(0, k) for k in (0, 1)]
    gph = lmax * d // 64
    qpk = n_q // n_kv

    def head(kv):
        KV = []
        for w, s, b in planes:
            sl = slice(kv * gph, kv * gph + L * d // 64)
            n = np.concatenate([w[sl] & 15, w[sl] >> 4], axis=1).astype(np.float64)
            KV.append((n * s[sl].astype(np.float64)[:, None] +
                       b[sl].astype(np.float64)[:, None]).reshape(L, d))
        K, V = KV
        res = []
        for h in range(kv * qpk, (kv + 1) * qpk):
            sc = K @ q[h].astype(np.float64) / np.sqrt(d)
            p = np.exp(sc - sc.max())
            res.append(p @ V / p.sum())
        return res

    with ThreadPoolExecutor(POOL) as ex:
        return np.array([r for rs in ex.map(head, range(n_kv)) for r in rs])


def test_70b_shape_launch(E):
    """One layer of the 70B-shape workload: 64 q heads / 8 kv heads, d=128,
    131072 tokens, its K and V distribution.  On 256 CUs the launch runs
    two-quad waves over 64-token tiles, 32 chunks per kv head, merged by a
    second launch (merge_parts_kernel: 8 parts of 4 chunks, then the
    parts); the allocation-free form and the host-pointer call must give the
    same bits, and the result meets the reference bar, with the exception
    checked value by value.  The V-sum of the oracle's softmax rows runs the
    same chunks in V-sum mode against the oracle."""
    n_kv, n_q, d, L = 8, 64, 128, 131072
    lmax = L + 64
    say("70b-shape: build")

    def make(kv):
        rng = np.random.default_rng(0xEA4B + 5 + 100 * kv)
        return chan_outlier_kv(rng, L, d), chan_outlier_kv(rng, L, d)

    data = np.empty((2, n_kv, L, d), np.float32)
    with ThreadPoolExecutor(POOL) as ex:
        for kv, (k, v) in enumerate(ex.map(make, range(n_kv))):
            data[0, kv], data[1, kv] = k, v
    g, o = E.Cache(1, n_kv, d, lmax), O.OracleCache(1, n_kv, d, lmax)
    g.load_raw(data, L)
    o.load_raw(data, L)
    del data
    plan = E.fused_plan([g], n_q, n_kv)
    say("70b-shape: plan", plan)
    assert plan["mfma"] == 1 and plan["quads"] == 2 and plan["tile_tokens"] == 64
    assert plan["waves_per_block"] == 8 and plan["split"] == 1
    if n_cu() == 256:
        assert plan["chunks"] == 32 and plan["merge_levels"] == 0
    rng = np.random.default_rng(0xEA4B + 55)
    q = rng.standard_normal((1, n_q, d), dtype=np.float32)
    out = batch_call(E, "eakv_attention_fused_batch_device", [g], q, n_q, n_kv)
    out_na = batch_call(E, "eakv_attention_fused_batch_device_noalloc", [g], q, n_q, n_kv)
    assert np.array_equal(out.view(np.uint32), out_na.view(np.uint32))
    out2 = g.attention_fused(q[0], 0, n_q, n_kv)
    assert np.array_equal(out[0].view(np.uint32), out2.view(np.uint32))
    ref = o.attention_fused_avx512(q[0], 0, n_q, n_kv) if O.avx512_available() \
        else o.attention_fused(q[0], 0, n_q, n_kv)
    exact = exact_attention_by_head(o, q[0], n_q, n_kv, L)
    mode, e_gr, e_re, e_ge, n_ex, ref_bar = check_against_reference(out[0], ref, exact, ATOL,
                                                                    RTOL)
    say(f"70b-shape: {mode} bar; gpu-reference {e_gr:.3g}, reference-exact {e_re:.3g} "
        f"({ref_bar:.3f} of the bar), gpu-exact {e_ge:.3g}, {n_ex} values excused")
    say("70b-shape: V-sum")
    avx = O.avx512_available()
    w = O.softmax_rows(o.attention_scores_avx512(q[0], 0, n_q, n_kv) if avx
                       else o.attention_scores(q[0], 0, n_q, n_kv))
    want = o.attention_output_avx512(w, 0, n_q, n_kv) if avx \
        else o.attention_output(w, 0, n_q, n_kv)
    ok, err, nbad = tol_close(g.attention_output(w, 0, n_q, n_kv), want, ATOL, RTOL)
    assert ok, (err, nbad)
    g.free()
    o.free()
