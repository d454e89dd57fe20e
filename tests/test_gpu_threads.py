"""The reference's threading contract, "All functions are thread-safe for
distinct caches" (reference include/eakv.h:3), through the host-pointer C
API on the GPU.

Two threads each drive a cache of their own at the same time (ctypes releases
the GIL for the library's calls, so the calls overlap): load_raw, appends of
every layer, advance, K-scores, the caller's softmax and the V-sum, the fused
call, checkpoint and restore, round after round.  Each thread checks its
results against an oracle cache of its own: planes and K-scores bit-exact,
V-sum and fused outputs within 1e-4 abs / 1e-5 rel.  A third thread keeps the
device's shared stream busy with device-pointer calls on a third cache,
which the host-pointer calls of the other two must not wait for.
"""
import threading
import time

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


def drive(E, name, nl, nh, d, n_q, L0, n_new, rounds, seed, start, log):
    rng = np.random.default_rng(seed)
    lmax = L0 + rounds * n_new
    g, o = E.Cache(nl, nh, d, lmax), O.OracleCache(nl, nh, d, lmax)
    data = rng.standard_normal(nl * 2 * nh * L0 * d).astype(np.float32)
    start.wait()
    g.load_raw(data, L0)
    o.load_raw(data, L0)
    del data
    for r in range(rounds):
        for l in range(nl):
            for kv in (0, 1):
                x = rng.standard_normal((nh, n_new, d)).astype(np.float32)
                g.append(x, l, kv, n_new)
                o.append(x, l, kv, n_new)
        g.advance(n_new)
        o.advance(n_new)
        layer = r % nl
        for kv in (0, 1):
            a, b = g.read_planes(layer, kv), o.read_planes(layer, kv)
            assert all(np.array_equal(np.ascontiguousarray(x).view(np.uint8),
                                      np.ascontiguousarray(y).view(np.uint8))
                       for x, y in zip(a, b)), (name, r, kv)
        q = rng.standard_normal((n_q, d)).astype(np.float32)
        sg = g.attention_scores(q, layer, n_q, nh)
        so = o.attention_scores(q, layer, n_q, nh)
        assert np.array_equal(sg.view(np.uint32), so.view(np.uint32)), (name, r)
        w = O.softmax_rows(so)
        ok, err, nbad = tol_close(g.attention_output(w, layer, n_q, nh),
                                  o.attention_output(w, layer, n_q, nh), ATOL, RTOL)
        assert ok, (name, r, "output", err, nbad)
        ok, err, nbad = tol_close(g.attention_fused(q, layer, n_q, nh),
                                  o.attention_fused(q, layer, n_q, nh), ATOL, RTOL)
        assert ok, (name, r, "fused", err, nbad)
        # rewind half a round and append again (the next round overwrites)
        cp = g.checkpoint()
        assert cp == o.checkpoint()
        g.restore(cp - n_new // 2)
        o.restore(cp - n_new // 2)
        log.append((name, r))
    g.free()
    o.free()


def busy_shared_stream(E, stop, count):
    """Device-pointer fused calls on a third cache, on the shared stream, until
    stop is set (each waited for, so the queue stays short)."""
    from eakv_amd.hipmem import DeviceArray
    nh, d, n_q, L = 8, 128, 32, 60000
    c = E.Cache(1, nh, d, L)
    rng = np.random.default_rng(7)
    c.load_raw(rng.standard_normal(2 * nh * L * d).astype(np.float32), L)
    dq = DeviceArray.from_host(rng.standard_normal((1, n_q, d)).astype(np.float32))
    dout = DeviceArray((1, n_q, d))
    h = E.handles([c])
    while not stop.is_set():
        for _ in range(20):
            assert E.lib().eakv_attention_fused_batch_device(h, 1, 0, dq.ptr, n_q, nh,
                                                             dout.ptr, None) == 0
        c.sync()
        count[0] += 20
    dq.free()
    dout.free()
    c.free()


def test_distinct_caches_from_concurrent_threads(E):
    specs = [("gqa-d128", 2, 8, 128, 32, 20000, 3000, 4, 101),
             ("mha-d64", 3, 4, 64, 4, 30000, 2000, 4, 202)]
    start = threading.Barrier(len(specs))
    stop = threading.Event()
    count = [0]
    errors, log = [], []

    def run(spec):
        try:
            drive(E, *spec, start, log)
        except BaseException as e:      # re-raised in the main thread
            errors.append((spec[0], e))

    busy = threading.Thread(target=busy_shared_stream, args=(E, stop, count))
    busy.start()
    threads = [threading.Thread(target=run, args=(s,)) for s in specs]
    t0 = time.perf_counter()
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    stop.set()
    busy.join()
    say("threads: rounds", log, "in", round(time.perf_counter() - t0, 2), "s; fused calls "
        "on the shared stream meanwhile:", count[0])
    if errors:
        raise errors[0][1]
    assert sorted(log) == sorted((s[0], r) for s in specs for r in range(s[7]))


def keep_stream_busy(E, stream, n_calls=40):
    """Queue n_calls fused calls of a 60000-token cache on `stream` (NULL:
    the shared stream) and return what must be freed once it has drained."""
    from eakv_amd.hipmem import DeviceArray
    nh, d, n_q, L = 8, 128, 32, 60000
    c = E.Cache(1, nh, d, L)
    rng = np.random.default_rng(5)
    c.load_raw(rng.standard_normal(2 * nh * L * d).astype(np.float32), L)
    dq = DeviceArray.from_host(rng.standard_normal((1, n_q, d)).astype(np.float32))
    dout = DeviceArray((1, n_q, d))
    h = E.handles([c])
    for _ in range(n_calls):
        assert E.lib().eakv_attention_fused_batch_device(h, 1, 0, dq.ptr, n_q, nh, dout.ptr,
                                                         stream) == 0
    return [c, dq, dout]


def test_device_scores_on_caller_stream_after_shared_append(E):
    """A NULL-stream append queued behind a busy shared stream, then K-scores
    of the same cache on a caller's stream with no wait of the caller's: the
    library orders the scores after the append on the device, and they are
    bit-exact against the oracle with the appended tokens.  (Whether an
    unordered launch would overlap here depends on how the runtime maps the
    streams to hardware queues; the results are checked either way.)"""
    from eakv_amd.hipmem import DeviceArray, Stream
    nh, d, n_q, L0, n_new = 8, 128, 8, 3000, 5000
    rng = np.random.default_rng(21)
    g, o = E.Cache(1, nh, d, L0 + n_new), O.OracleCache(1, nh, d, L0 + n_new)
    data = rng.standard_normal(2 * nh * L0 * d).astype(np.float32)
    g.load_raw(data, L0)
    o.load_raw(data, L0)
    # every buffer allocated and uploaded before the queue fills
    x = rng.standard_normal((nh, n_new, d)).astype(np.float32)
    dx = DeviceArray.from_host(x)
    s = Stream()
    q = rng.standard_normal((n_q, d)).astype(np.float32)
    dq = DeviceArray.from_host(q)
    dsc = DeviceArray((n_q, L0 + n_new))
    busy = keep_stream_busy(E, None)
    assert E.lib().eakv_cache_append_device(g.h, dx.ptr, 0, 0, n_new, None) == 0
    o.append(x, 0, 0, n_new)
    g.advance(n_new)
    o.advance(n_new)
    assert E.lib().eakv_attention_scores_device(g.h, dq.ptr, 0, n_q, nh, dsc.ptr, s.s) == 0
    s.synchronize()
    got = dsc.download()
    want = o.attention_scores(q, 0, n_q, nh)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    g.sync()
    for a in [dx, dq, dsc] + busy:
        a.free()
    g.free()
    o.free()


def test_host_call_after_device_append_on_caller_stream(E):
    """An append on a caller's stream queued behind other work there, then a
    host-pointer K-score call on the cache: the library orders the host call
    after the append on the device (no host wait: the call's staging is sized
    beforehand), and its scores are bit-exact against the oracle with the
    appended tokens."""
    from eakv_amd.hipmem import DeviceArray, Stream
    nh, d, n_q, L0, n_new = 8, 128, 8, 3000, 5000
    rng = np.random.default_rng(22)
    g, o = E.Cache(1, nh, d, L0 + n_new), O.OracleCache(1, nh, d, L0 + n_new)
    data = rng.standard_normal(2 * nh * L0 * d).astype(np.float32)
    g.load_raw(data, L0)
    o.load_raw(data, L0)
    s = Stream()
    x = rng.standard_normal((nh, n_new, d)).astype(np.float32)
    dx = DeviceArray.from_host(x)
    q = rng.standard_normal((n_q, d)).astype(np.float32)
    # size the host call's staging for the full context now, so that the call
    # below allocates nothing (a reallocation would wait on the host)
    g.advance(n_new)
    g.attention_scores(q, 0, n_q, nh)
    g.restore(L0)
    busy = keep_stream_busy(E, s.s)
    assert E.lib().eakv_cache_append_device(g.h, dx.ptr, 0, 0, n_new, s.s) == 0
    o.append(x, 0, 0, n_new)
    g.advance(n_new)
    o.advance(n_new)
    a = g.attention_scores(q, 0, n_q, nh)
    b = o.attention_scores(q, 0, n_q, nh)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    s.synchronize()
    for x_ in [dx] + busy:
        x_.free()
    g.free()
    o.free()


@pytest.mark.parametrize("explicit", [False, True])
def test_host_call_after_device_append_on_shared_stream(E, explicit):
    """A device-pointer append on the shared stream (NULL, or the stream
    eakv_cache_stream returns, named explicitly) is pending work of the
    cache: the next host-pointer call, which runs on the cache's own stream,
    waits for it on the device and sees the appended tokens."""
    from eakv_amd.hipmem import DeviceArray
    nh, d, n_q, L0, n_new = 8, 128, 32, 3000, 20000
    rng = np.random.default_rng(11 + explicit)
    g, o = E.Cache(1, nh, d, L0 + n_new), O.OracleCache(1, nh, d, L0 + n_new)
    data = rng.standard_normal(2 * nh * L0 * d).astype(np.float32)
    g.load_raw(data, L0)
    o.load_raw(data, L0)
    st = g.stream if explicit else None
    keep = []
    for kv in (0, 1):
        x = rng.standard_normal((nh, n_new, d)).astype(np.float32)
        dx = DeviceArray.from_host(x)
        keep.append(dx)
        assert E.lib().eakv_cache_append_device(g.h, dx.ptr, 0, kv, n_new, st) == 0
        o.append(x, 0, kv, n_new)
    g.advance(n_new)
    o.advance(n_new)
    q = rng.standard_normal((n_q, d)).astype(np.float32)
    a = g.attention_scores(q, 0, n_q, nh)
    b = o.attention_scores(q, 0, n_q, nh)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    g.free()
    o.free()
