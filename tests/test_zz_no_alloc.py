"""The allocation-free batched fused call (partials in the library's static
device scratch) against the workspace form of the same call, through the C
ABI: identical outputs, bit for bit, on two calls in a row (the second over
a smaller batch), and a launch too large for the scratch rejected before
anything runs."""
import numpy as np
import pytest

import oracle as O
from conftest import tol_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def E():
    import eakv_amd
    from eakv_amd import hipmem
    if hipmem.device_count() < 1:
        pytest.fail("no HIP device visible")
    return eakv_amd


def say(*a):
    print(*a, flush=True)


def caches(E, rng, nl, nh, d, lens, lmax):
    gs, os_ = [], []
    for L in lens:
        g = E.Cache(nl, nh, d, lmax)
        o = O.OracleCache(nl, nh, d, lmax)
        if L:
            data = rng.standard_normal(nl * 2 * nh * L * d).astype(np.float32)
            g.load_raw(data, L)
            o.load_raw(data, L)
        gs.append(g)
        os_.append(o)
    return gs, os_


def both(E, gs, layer, q, n_q, n_kv):
    """(workspace form, allocation-free form) outputs of one batch."""
    from eakv_amd.hipmem import DeviceArray
    n, d = q.shape[0], q.shape[2]
    dq = DeviceArray.from_host(q)
    outs = []
    for fn in ("eakv_attention_fused_batch_device", "eakv_attention_fused_batch_device_noalloc"):
        dout = DeviceArray((n, n_q, d))
        say("  call", fn, "n_seq", n, "n_q", n_q, "n_kv", n_kv)
        assert getattr(E.lib(), fn)(E.handles(gs), n, layer, dq.ptr, n_q, n_kv, dout.ptr,
                                    None) == 0, E.last_error()
        gs[0].sync()
        outs.append(dout.download())
    return outs


@pytest.mark.parametrize("d,nh,n_q", [(128, 8, 32), (64, 4, 32), (128, 2, 16)])
def test_noalloc_equals_workspace_form(E, rng, d, nh, n_q):
    say("noalloc", d, nh, n_q)
    gs, os_ = caches(E, rng, 2, nh, d, [3000, 5000, 1, 4600], 5000)
    q = rng.standard_normal((4, n_q, d)).astype(np.float32)
    ws, na = both(E, gs, 1, q, n_q, nh)
    assert np.array_equal(ws.view(np.uint32), na.view(np.uint32))
    for i, o in enumerate(os_):
        ok, err, nbad = tol_close(na[i], o.attention_fused(q[i], 1, n_q, nh))
        assert ok, (i, err, nbad)
    # a second call right behind, over a smaller batch: fewer sequences,
    # shorter contexts, fewer q heads
    for g in gs[:2]:
        g.restore(700)
    n_q2 = n_q // 2
    q2 = rng.standard_normal((2, n_q2, d)).astype(np.float32)
    ws, na = both(E, gs[:2], 0, q2, n_q2, nh // 2 if nh > 2 else 1)
    assert np.array_equal(ws.view(np.uint32), na.view(np.uint32))
    for i in range(2):
        os_[i].restore(700)
        ok, err, nbad = tol_close(na[i], os_[i].attention_fused(q2[i], 0, n_q2,
                                                                nh // 2 if nh > 2 else 1))
        assert ok, (i, err, nbad)


def test_noalloc_rejects_launch_beyond_scratch(E):
    """32 caches of 128 kv heads with 8 q heads each: 4096 (cache, kv head)
    units of one chunk, 32 * 1024 * (128 + 2) * 4 = 17.0 MB of partials,
    above the 16 MiB scratch; the call reports EAKV_ERR_INVALID and launches
    nothing (the queries are never read)."""
    from eakv_amd.hipmem import DeviceArray
    gs = [E.Cache(1, 128, 128, 16) for _ in range(32)]
    for g in gs:
        g.advance(16)
    dq = DeviceArray((32, 1024, 128))
    dout = DeviceArray((32, 1024, 128))
    rc = E.lib().eakv_attention_fused_batch_device_noalloc(E.handles(gs), 32, 0, dq.ptr, 1024,
                                                          128, dout.ptr, None)
    assert rc == E.EAKV_ERR_INVALID
    assert b"scratch" in E.lib().eakv_last_error_message()


def test_noalloc_after_null_stream_batch_append(E, rng):
    """A batched append on the shared stream (NULL) writes caches c0, c1 and
    c2.  The allocation-free call over [c1, c2] on a caller's stream right
    behind it must run after it (the append is pending work of every cache
    it names, not of c0 alone), and so must the workspace form on another
    caller's stream and a host-pointer call on c2 (the cache's own stream)."""
    from eakv_amd.hipmem import DeviceArray, Stream
    nh, d, n_q, n_new = 4, 128, 16, 6000
    gs, os_ = caches(E, rng, 1, nh, d, [2000, 3000, 2500], 2000 + 3000 + n_new)
    x = rng.standard_normal((3, 1, 2, nh, n_new, d)).astype(np.float32)
    dx = DeviceArray.from_host(x)
    say("race: batched append on the shared stream")
    assert E.lib().eakv_append_batch_device(E.handles(gs), 3, dx.ptr, n_new, None) == 0
    for i in range(3):
        gs[i].advance(n_new)
        for kv in (0, 1):
            os_[i].append(x[i, 0, kv], 0, kv, n_new)
        os_[i].advance(n_new)
    q = rng.standard_normal((2, n_q, d)).astype(np.float32)
    dq = DeviceArray.from_host(q)
    outs = []
    for fn in ("eakv_attention_fused_batch_device_noalloc", "eakv_attention_fused_batch_device"):
        st = Stream()
        dout = DeviceArray((2, n_q, d))
        say("race:", fn, "on a caller's stream")
        assert getattr(E.lib(), fn)(E.handles(gs[1:]), 2, 0, dq.ptr, n_q, nh, dout.ptr,
                                    st.s) == 0, E.last_error()
        st.synchronize()
        outs.append(dout.download())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    for i in range(2):
        ok, err, nbad = tol_close(outs[0][i], os_[i + 1].attention_fused(q[i], 0, n_q, nh))
        assert ok, (i, err, nbad)
    # another append on the shared stream, then a host-pointer call on c2
    x2 = rng.standard_normal((3, 1, 2, nh, 500, d)).astype(np.float32)
    dx2 = DeviceArray.from_host(x2)
    assert E.lib().eakv_append_batch_device(E.handles(gs), 3, dx2.ptr, 500, None) == 0
    gs[2].advance(500)
    for kv in (0, 1):
        os_[2].append(x2[2, 0, kv], 0, kv, 500)
    os_[2].advance(500)
    a = gs[2].attention_scores(q[1], 0, n_q, nh)
    b = os_[2].attention_scores(q[1], 0, n_q, nh)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
