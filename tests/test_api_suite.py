"""The reference's own C tests, re-expressed once and run against both
backends: the CPU oracle (always) and libeakv.so on the GPU (-m gpu).

Sources: reference tests/test_cache.c, test_append.c, test_checkpoint.c,
test_attention_c.c, test_io_c.c, test_e2e.c.  Inputs are the same closed
forms those files use; tolerances are theirs.
"""
import os

import numpy as np
import pytest

import oracle as O

BACKENDS = ["oracle", pytest.param("hip", marks=pytest.mark.gpu)]

INVALID, IO, FORMAT = -4, -1, -2


class Api:
    def __init__(self, name):
        self.name = name
        if name == "oracle":
            self.Cache = O.OracleCache
            self.Err = O.OracleError
        else:
            import eakv_amd
            self.Cache = eakv_amd.Cache
            self.Err = eakv_amd.EakvError

    def create(self, *a):
        try:
            return self.Cache(*a)
        except (ValueError, self.Err):
            return None

    def rc(self, fn, *a):
        try:
            return fn(*a)
        except self.Err as e:
            return e.code


@pytest.fixture(params=BACKENDS)
def api(request):
    return Api(request.param)


def ramp(n, mod, div, off):
    """(i % mod)/div - off, the reference tests' closed-form inputs."""
    i = np.arange(n, dtype=np.int64)
    return ((i % mod).astype(np.float32) / np.float32(div) - np.float32(off)).astype(np.float32)


# ---- tests/test_cache.c:4-49

def test_create_and_getters(api):
    c = api.create(2, 8, 128, 64)
    assert c is not None
    assert (c.seq_len, c.n_layers, c.n_heads, c.head_dim, c.max_seq_len) == (0, 2, 8, 128, 64)
    c.free()


def test_create_rejects_bad_params(api):
    assert api.create(0, 8, 128, 64) is None
    assert api.create(2, 0, 128, 64) is None
    assert api.create(2, 8, 128, 0) is None
    assert api.create(2, 3, 100, 64) is None        # 300 % 64 != 0


def test_load_raw_sets_seq_len(api):
    nl, nh, hd, sl = 1, 2, 128, 64
    c = api.create(nl, nh, hd, sl)
    assert c.load_raw(ramp(nl * 2 * nh * sl * hd, 1000, 100, 5), sl) == 0
    assert c.seq_len == sl
    assert c.compression_ratio == np.float32(40.0 / 256.0)


def test_load_raw_rejects_oversized(api):
    c = api.create(1, 2, 128, 32)
    assert api.rc(c.load_raw, np.zeros(1, np.float32), 64) == INVALID
    assert api.rc(c.load_raw, np.zeros(1, np.float32), 0) == INVALID


# ---- tests/test_append.c:40-211

def _extract(bulk, nl, nh, hd, sl, layer, kv, t0, n):
    b = bulk.reshape(nl, 2, nh, sl, hd)
    return np.ascontiguousarray(b[layer, kv, :, t0:t0 + n, :])


@pytest.mark.parametrize("nl,nh,hd,sl", [(1, 4, 64, 32), (1, 4, 128, 16), (2, 8, 128, 8)])
def test_append_matches_bulk(api, nl, nh, hd, sl):
    data = ramp(nl * 2 * nh * sl * hd, 2000, 200, 5)
    bulk = api.create(nl, nh, hd, sl)
    bulk.load_raw(data, sl)
    incr = api.create(nl, nh, hd, sl)
    for t in range(sl):
        for l in range(nl):
            for kv in range(2):
                assert incr.append(_extract(data, nl, nh, hd, sl, l, kv, t, 1), l, kv, 1) == 0
        incr.advance(1)
    for l in range(nl):
        for kv in range(2):
            for a, b in zip(bulk.read_planes(l, kv), incr.read_planes(l, kv)):
                assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
    q = np.full((nh, hd), 0.1, np.float32)
    s1, s2 = bulk.attention_scores(q, 0, nh, nh), incr.attention_scores(q, 0, nh, nh)
    assert np.abs(s1 - s2).max() < 1e-5
    w = np.full((nh, sl), 1.0 / sl, np.float32)
    o1, o2 = bulk.attention_output(w, 0, nh, nh), incr.attention_output(w, 0, nh, nh)
    assert np.abs(o1 - o2).max() < 1e-5


def test_batch_append_matches_bulk(api):
    nl, nh, hd, sl = 1, 4, 64, 32
    data = ramp(nl * 2 * nh * sl * hd, 2000, 200, 5)
    bulk = api.create(nl, nh, hd, sl)
    bulk.load_raw(data, sl)
    batch = api.create(nl, nh, hd, sl)
    for t in range(0, sl, 8):
        n = min(8, sl - t)
        for kv in range(2):
            batch.append(_extract(data, nl, nh, hd, sl, 0, kv, t, n), 0, kv, n)
        batch.advance(n)
    q = np.full((nh, hd), 0.1, np.float32)
    assert np.abs(bulk.attention_scores(q, 0, nh, nh) -
                  batch.attention_scores(q, 0, nh, nh)).max() < 1e-5


def test_clear_and_reuse(api):
    nl, nh, hd, sl = 1, 4, 64, 16
    c = api.create(nl, nh, hd, sl)
    data = ramp(nl * 2 * nh * sl * hd, 2000, 200, 5)
    c.load_raw(data, sl)
    assert c.seq_len == sl
    c.clear()
    assert c.seq_len == 0
    c.load_raw(data, sl)
    assert c.seq_len == sl


def test_append_overflow(api):
    nl, nh, hd, sl = 1, 4, 64, 8
    c = api.create(nl, nh, hd, sl)
    c.load_raw(ramp(nl * 2 * nh * sl * hd, 2000, 200, 5), sl)
    assert api.rc(c.advance, 1) == INVALID
    assert api.rc(c.append, np.zeros(nh * hd, np.float32), 0, 0, 1) == INVALID


def test_append_bad_params(api):
    c = api.create(2, 4, 64, 16)
    tok = np.zeros(4 * 64, np.float32)
    assert api.rc(c.append, tok, 5, 0, 1) == INVALID
    assert api.rc(c.append, tok, 0, 2, 1) == INVALID
    assert api.rc(c.append, tok, 0, 0, 0) == INVALID
    assert api.rc(c.append, tok, -1, 0, 1) == INVALID


# ---- tests/test_checkpoint.c:7-72

def test_checkpoint_restore(api):
    c = api.create(2, 2, 64, 256)
    assert c.checkpoint() == 0
    c.load_raw(np.zeros(2 * 2 * 128 * 16, np.float32), 16)
    assert c.checkpoint() == 16
    assert c.restore(8) == 0 and c.seq_len == 8
    assert c.restore(0) == 0 and c.seq_len == 0


def test_restore_bounds(api):
    c = api.create(2, 2, 64, 256)
    c.load_raw(np.zeros(2 * 2 * 128 * 8, np.float32), 8)
    assert api.rc(c.restore, 16) == INVALID and c.seq_len == 8
    assert api.rc(c.restore, -1) == INVALID and c.seq_len == 8


def test_append_after_restore(api):
    c = api.create(2, 2, 64, 256)
    c.load_raw(np.zeros(2 * 2 * 128 * 16, np.float32), 16)
    c.restore(8)
    a = np.zeros(128 * 4, np.float32)
    for l in range(2):
        c.append(a, l, 0, 4)
        c.append(a, l, 1, 4)
    c.advance(4)
    assert c.seq_len == 12


# ---- tests/test_attention_c.c:10-80

def test_mha_scores_and_output_finite(api):
    nl, nh, hd, sl = 1, 4, 128, 32
    c = api.create(nl, nh, hd, sl)
    c.load_raw(ramp(nl * 2 * nh * sl * hd, 256, 50, 2.5), sl)
    assert np.isfinite(c.attention_scores(np.ones((4, 128), np.float32), 0, 4, 4)).all()
    w = np.full((4, 32), 1.0 / 32, np.float32)
    assert np.isfinite(c.attention_output(w, 0, 4, 4)).all()


def test_scores_deterministic(api):
    nl, nh, hd, sl = 1, 2, 128, 16
    data = ramp(nl * 2 * nh * sl * hd, 256, 50, 2.5)
    c1, c2 = api.create(nl, nh, hd, sl), api.create(nl, nh, hd, sl)
    c1.load_raw(data, sl)
    c2.load_raw(data, sl)
    q = np.full((2, 128), 0.5, np.float32)
    assert np.abs(c1.attention_scores(q, 0, 2, 2) - c2.attention_scores(q, 0, 2, 2)).max() <= 1e-6


# ---- tests/test_io_c.c:6-65 and tests/test_e2e.c:6-57

def test_save_load_roundtrip(api, tmp_path):
    nl, nh, hd, sl = 2, 4, 128, 32
    c = api.create(nl, nh, hd, sl)
    c.load_raw(ramp(nl * 2 * nh * sl * hd, 1000, 100, 5), sl)
    p = str(tmp_path / "rt.eakv")
    assert c.save(p) == 0
    d = api.Cache.load(p)
    assert (d.seq_len, d.n_layers, d.n_heads, d.head_dim) == (sl, nl, nh, hd)
    q = np.ones((4, 128), np.float32)
    assert np.abs(c.attention_scores(q, 0, 4, 4) - d.attention_scores(q, 0, 4, 4)).max() <= 1e-6


def test_load_nonexistent(api, tmp_path):
    with pytest.raises(api.Err) as e:
        api.Cache.load(str(tmp_path / "does_not_exist.eakv"))
    assert e.value.code == IO


def test_load_bad_magic(api, tmp_path):
    p = tmp_path / "bad.eakv"
    p.write_bytes(b"NOPE" + bytes(508))
    with pytest.raises(api.Err) as e:
        api.Cache.load(str(p))
    assert e.value.code == FORMAT


def test_full_pipeline(api, tmp_path):
    nl, nh, hd, sl = 4, 8, 128, 256
    c = api.create(nl, nh, hd, sl)
    assert c.load_raw(ramp(nl * 2 * nh * sl * hd, 2000, 200, 5), sl) == 0
    q = np.full((8, 128), 0.1, np.float32)
    for l in range(nl):
        assert np.isfinite(c.attention_scores(q, l, 8, 8)).all()
        w = np.full((8, 256), 1.0 / 256, np.float32)
        assert np.isfinite(c.attention_output(w, l, 8, 8)).all()
    p = str(tmp_path / "e2e.eakv")
    assert c.save(p) == 0
    d = api.Cache.load(p)
    assert d.seq_len == sl and d.n_layers == nl
    assert np.abs(c.attention_scores(q, 0, 8, 8) - d.attention_scores(q, 0, 8, 8)).max() <= 1e-6
