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
