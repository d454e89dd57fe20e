"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
and, for the ggml block type, tests/golden/make_ggml_golden.py).

The fixtures hold seeded inputs and the expected quantized planes, K-scores,
softmax weights, V-sums and fused outputs.  The CPU tests pin the oracle to
them (bit for bit) and to the reference's own src/ggml_type.c quantizer where
oracle/_ref is built; the gpu tests run the same inputs through the HIP path
(libeakv.so): quantization and K-scores bit-exact, V-sum and fused attention
within |err| <= 1e-4 + 1e-5*|want|.
"""
import hashlib
import json
import os

import numpy as np
import pytest

from conftest import tol_close

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ATTN = ["mha_d128_L37", "gqa8_d64_L33", "gqa4_d128_L64"]


def load(name):
    with np.load(os.path.join(GOLD, name + ".npz")) as z:
        return {k: z[k] for k in z.files}


def bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


def test_manifest_sha256():
    manifest = json.load(open(os.path.join(GOLD, "manifest.json")))
    assert sorted(manifest) == sorted([n + ".npz" for n in ["special_groups", "ggml_rows"] + ATTN])
    for fname, digest in manifest.items():
        got = hashlib.sha256(open(os.path.join(GOLD, fname), "rb").read()).hexdigest()
        assert got == digest, fname


# ------------------------------------------------------------------ oracle

def test_oracle_special_groups():
    import oracle as O
    g = load("special_groups")
    w, s, b = O.quantize(g["x"])
    assert np.array_equal(w, g["w"])
    assert np.array_equal(bits(s), bits(g["s"])) and np.array_equal(bits(b), bits(g["b"]))
    assert np.array_equal(bits(O.dequantize(w, s, b)), bits(g["deq"]))
    # closed forms: constant group -> scale 1, bias = value, nibbles 0
    assert g["s"][0] == 1.0 and g["b"][0] == np.float32(3.25) and not g["w"][0].any()
    # 0..63 -> scale 63/15, bias 0, min -> 0 and max -> 15
    assert g["s"][1] == np.float32(63.0) / np.float32(15.0) and g["b"][1] == 0.0
    assert (g["w"][1][0] & 15) == 0 and (g["w"][1][31] >> 4) == 15


def test_oracle_special_groups_match_reference_ggml():
    import oracle as O
    if O.ref_lib() is None:
        pytest.skip("oracle/_ref not built (needs the reference sources)")
    from golden.make_golden import ref_check
    g = load("special_groups")
    ref_check(g["x"], g["w"], g["s"], g["b"])


@pytest.mark.parametrize("name", ATTN)
def test_oracle_reproduces_fixture(name):
    import oracle as O
    f = load(name)
    n_kv, n_q, d, L = (int(v) for v in f["shape"])
    with O.OracleCache(1, n_kv, d, L) as c:
        c.load_raw(f["data"], L)
        for kv, p in ((0, "k"), (1, "v")):
            w, s, b = c.read_planes(0, kv)
            assert np.array_equal(w, f[p + "_w"])
            assert np.array_equal(bits(s), bits(f[p + "_s"]))
            assert np.array_equal(bits(b), bits(f[p + "_b"]))
        sc = c.attention_scores(f["q"], 0, n_q, n_kv)
        assert np.array_equal(bits(sc), bits(f["scores"]))
        assert np.array_equal(bits(O.softmax_rows(sc)), bits(f["weights"]))
        out = c.attention_output(f["weights"], 0, n_q, n_kv)
        assert np.array_equal(bits(out), bits(f["output"]))
        fused = c.attention_fused(f["q"], 0, n_q, n_kv)
        assert np.array_equal(bits(fused), bits(f["fused"]))


@pytest.mark.parametrize("name", ATTN)
def test_fixture_against_f64(name):
    """The expected scores and outputs agree with an f64 evaluation of the
    dequantized cache (pins the fixture independently of the oracle's f32
    operation order)."""
    import oracle as O
    f = load(name)
    n_kv, n_q, d, L = (int(v) for v in f["shape"])
    g = n_q // n_kv
    kd = O.dequantize(f["k_w"], f["k_s"], f["k_b"]).astype(np.float64).reshape(n_kv, L, d)
    vd = O.dequantize(f["v_w"], f["v_s"], f["v_b"]).astype(np.float64).reshape(n_kv, L, d)
    q = f["q"].astype(np.float64)
    sc = np.stack([kd[h // g] @ q[h] for h in range(n_q)]) / np.sqrt(d)
    ok, err, _ = tol_close(f["scores"], sc, atol=2e-5, rtol=2e-6)
    assert ok, err
    w = np.exp(sc - sc.max(axis=1, keepdims=True))
    w /= w.sum(axis=1, keepdims=True)
    out = np.stack([w[h] @ vd[h // g] for h in range(n_q)])
    ok, err, _ = tol_close(f["fused"], out)
    assert ok, err
    ok, err, _ = tol_close(f["output"], out)
    assert ok, err


# -------------------------------------------------------------------- HIP

@pytest.mark.gpu
def test_gpu_special_groups_bit_exact():
    import eakv_amd as E
    g = load("special_groups")
    data = np.stack([g["x"], g["x"]])[None, :, None]          # [1][2][1][8][64]
    with E.Cache(1, 1, 64, 8) as c:
        c.load_raw(data, 8)
        for kv in (0, 1):
            w, s, b = c.read_planes(0, kv)
            assert np.array_equal(w, g["w"])
            assert np.array_equal(bits(s), bits(g["s"]))
            assert np.array_equal(bits(b), bits(g["b"]))


@pytest.mark.gpu
@pytest.mark.parametrize("name", ATTN)
def test_gpu_fixture_parity(name):
    import eakv_amd as E
    f = load(name)
    n_kv, n_q, d, L = (int(v) for v in f["shape"])
    with E.Cache(1, n_kv, d, L) as c:
        c.load_raw(f["data"], L)
        for kv, p in ((0, "k"), (1, "v")):
            w, s, b = c.read_planes(0, kv)
            assert np.array_equal(w, f[p + "_w"])
            assert np.array_equal(bits(s), bits(f[p + "_s"]))
            assert np.array_equal(bits(b), bits(f[p + "_b"]))
        sc = c.attention_scores(f["q"], 0, n_q, n_kv)
        assert np.array_equal(bits(sc), bits(f["scores"]))
        out = c.attention_output(f["weights"], 0, n_q, n_kv)
        ok, err, nbad = tol_close(out, f["output"])
        assert ok, (err, nbad)
        fused = c.attention_fused(f["q"], 0, n_q, n_kv)
        ok, err, nbad = tol_close(fused, f["fused"])
        assert ok, (err, nbad)


# ------------------------------------------------------- ggml block type

def test_oracle_reproduces_ggml_fixture():
    """The fixture's values come from the reference's ggml_type.c (scalar
    quantizer, AVX-512 dequantize and vec_dot); the oracle matches them."""
    import oracle as O
    g = load("ggml_rows")
    assert np.array_equal(O.ggml_quantize_row(g["x"]), g["blocks"])
    assert np.array_equal(bits(O.ggml_dequantize_row(g["blocks"])), bits(g["deq"]))
    assert np.array_equal(bits(O.ggml_vec_dot(g["dot_x"], g["dot_y"])), bits(g["dot"]))
    # closed forms: a constant block stores d = 0 (no range check, unlike the
    # cache quantizer's scale 1), m = the value, nibbles 0
    blk = g["blocks"][0]
    assert blk[32:36].view(np.float32)[0] == 0.0 and not blk[:32].any()
    assert blk[36:40].view(np.float32)[0] == np.float32(3.25)
    # 0..63: d = 63/15, m = 0, element 0 -> 0 and element 63 -> 15
    blk = g["blocks"][1]
    assert blk[32:36].view(np.float32)[0] == np.float32(63.0) / np.float32(15.0)
    assert (blk[0] & 15) == 0 and (blk[31] >> 4) == 15


@pytest.mark.gpu
def test_gpu_ggml_fixture_bit_exact():
    import eakv_amd as E
    from eakv_amd.hipmem import DeviceArray
    g = load("ggml_rows")
    L = E.lib()
    dx = DeviceArray.from_host(g["x"])
    db = DeviceArray((g["blocks"].size,), np.uint8)
    assert L.eakv_ggml_quantize_row_device(dx.ptr, db.ptr, g["x"].size, None) == 0
    dd = DeviceArray((g["x"].size,))
    assert L.eakv_ggml_dequantize_row_device(db.ptr, dd.ptr, g["x"].size, None) == 0
    dvx, dvy = DeviceArray.from_host(g["dot_x"]), DeviceArray.from_host(g["dot_y"])
    ds = DeviceArray((3,))
    n = g["dot_y"].shape[1]
    assert L.eakv_ggml_vec_dot_device(n, ds.ptr, 4, dvx.ptr, g["dot_x"].shape[1], dvy.ptr,
                                      n * 4, 3, None) == 0
    assert np.array_equal(db.download().reshape(-1, 40), g["blocks"])
    assert np.array_equal(bits(dd.download()), bits(g["deq"]))
    assert np.array_equal(bits(ds.download()), bits(g["dot"]))
