"""Write the golden fixtures under tests/golden/ (run from the repo root:
`python tests/golden/make_golden.py`).

Every expected value comes from the oracle (oracle/eakv_oracle.c, the C
restatement of the reference kernels).  Before anything is written, the
quantization of every fixture is cross-checked against the reference's own
src/ggml_type.c (`eakv_quantize_row`, built by `make -C oracle ref` into
oracle/_ref/): nibbles and biases must match bit for bit everywhere, scales
wherever the group's range is non-zero (ggml_type.c:48-50 stores 0 for a
constant group where quantize_simd.ea:33-38 stores 1.0).

Fixtures (.npz, no pickles; sha256 of each in manifest.json):
  special_groups  8 single-group special cases (constant, ramps, exact
                  half-ticks, min last / max first, two-valued, tiny and
                  huge ranges)
  mha_d128_L37    1 layer, 2 q / 2 kv heads, d=128, 37 tokens (odd tail)
  gqa8_d64_L33    1 layer, 16 q / 2 kv heads (8:1), d=64, 33 tokens
  gqa4_d128_L64   1 layer, 8 q / 2 kv heads (4:1), d=128, 64 tokens
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402


def special_groups():
    g = np.zeros((8, 64), np.float32)
    g[0] = 3.25                                           # constant
    g[1] = np.arange(64, dtype=np.float32)                # 0..63: scale 4.2
    g[2] = -np.arange(64, dtype=np.float32) / 8.0         # descending
    s = np.float32(0.75)                                  # x = min + k*scale (ticks)
    g[3] = np.float32(-2.0) + (np.arange(64) % 16).astype(np.float32) * s / 2
    g[4] = np.linspace(1.0, -1.0, 64, dtype=np.float32)   # max first, min last
    g[5] = np.where(np.arange(64) % 2 == 0, -1.0, 1.0)    # two values
    g[6] = np.arange(64, dtype=np.float32) * np.float32(1e-30)   # tiny range
    g[7] = (np.arange(64, dtype=np.float32) - 31.5) * np.float32(1e30)  # huge range
    return g


def ref_check(x, w, s, b):
    """Cross-check (w, s, b) against the reference's eakv_quantize_row."""
    R = O.ref_lib()
    if R is None:
        raise SystemExit("oracle/_ref/libggml_ref.so missing: run `make -C oracle ref`")
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    n = x.size // 64
    blk = np.zeros(n * 40, np.uint8)      # block_q4_1_eakv: u8 qs[32], f32 d, f32 m
    R.eakv_quantize_row(O._p(x), O._p(blk), x.size)
    blk = blk.reshape(n, 40)
    rq = blk[:, 0:32]
    rd = blk[:, 32:36].copy().view(np.float32).ravel()
    rm = blk[:, 36:40].copy().view(np.float32).ravel()
    assert np.array_equal(rq, w), "nibbles differ from ggml_type.c"
    assert np.array_equal(rm.view(np.uint32), b.view(np.uint32)), "biases differ"
    nz = rd != 0
    assert np.array_equal(rd[nz].view(np.uint32), s[nz].view(np.uint32)), "scales differ"
    assert np.all(s[~nz] == 1.0)


def attention_case(seed, n_kv, n_q, d, L):
    rng = np.random.default_rng(seed)
    data = rng.standard_normal((1, 2, n_kv, L, d), dtype=np.float32)
    q = rng.standard_normal((n_q, d), dtype=np.float32)
    with O.OracleCache(1, n_kv, d, L) as c:
        c.load_raw(data, L)
        kw, ks, kb = c.read_planes(0, 0)
        vw, vs, vb = c.read_planes(0, 1)
        scores = c.attention_scores(q, 0, n_q, n_kv)
        weights = O.softmax_rows(scores)
        out = c.attention_output(weights, 0, n_q, n_kv)
        fused = c.attention_fused(q, 0, n_q, n_kv)
    # groups are stored per head at stride L*gpd (max_seq_len == L here)
    ref_check(data[0, 0], kw, ks, kb)
    ref_check(data[0, 1], vw, vs, vb)
    return dict(data=data, q=q, k_w=kw, k_s=ks, k_b=kb, v_w=vw, v_s=vs, v_b=vb,
                scores=scores, weights=weights, output=out, fused=fused,
                shape=np.array([n_kv, n_q, d, L], np.int32))


def main():
    os.makedirs(HERE, exist_ok=True)
    fixtures = {}
    g = special_groups()
    w, s, b = O.quantize(g)
    ref_check(g, w, s, b)
    fixtures["special_groups"] = dict(x=g, w=w, s=s, b=b, deq=O.dequantize(w, s, b))
    fixtures["mha_d128_L37"] = attention_case(0xEA4B01, 2, 2, 128, 37)
    fixtures["gqa8_d64_L33"] = attention_case(0xEA4B02, 2, 16, 64, 33)
    fixtures["gqa4_d128_L64"] = attention_case(0xEA4B03, 2, 8, 128, 64)
    manifest = {}
    for name, arrs in fixtures.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez(path, **arrs)
        manifest[name + ".npz"] = hashlib.sha256(open(path, "rb").read()).hexdigest()
        print(f"wrote {path} ({os.path.getsize(path)} B)")
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
        f.write("\n")


if __name__ == "__main__":
    main()
