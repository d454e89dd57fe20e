"""Write tests/golden/ggml_rows.npz (run from the repo root after
`make -C oracle ref`: `python tests/golden/make_ggml_golden.py`).

Every expected value comes from the reference's own src/ggml_type.c, built by
`make -C oracle ref`, and is cross-checked against the oracle, bit for bit,
before anything is written.  The quantized blocks come from its scalar build
(oracle/_ref/libggml_ref.so): the strict min/max scan keeps the first of +0 /
-0, where the AVX-512 reduction (ggml_type.c:31-40) may return the other
sign, and that is the only difference between the two builds checked here.
The dequantized values and dot products come from the AVX-512 build
(oracle/_ref/libggml_ref_avx512.so, which needs an AVX-512 CPU): fused
n*d + m and 16 lane accumulators.

Arrays:
  x         f32[24*64]  rows to quantize: 24 blocks of finite special and
                        random cases
  blocks    u8[24, 40]  eakv_quantize_row(x), scalar build
  deq       f32[24*64]  eakv_dequantize_row(blocks)
  dot_x     u8[3, 320]  three rows of 8 blocks (n = 512)
  dot_y     f32[3, 512] the f32 rows they are dotted with
  dot       f32[3]      eakv_vec_dot_q4_f32(512, ..., nrc = 3)
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


def blocks_in():
    rng = np.random.default_rng(0xEA4B40)
    g = np.zeros((24, 64), np.float32)
    g[0] = 3.25                                           # constant: d = 0
    g[1] = np.arange(64, dtype=np.float32)
    g[2] = -np.arange(64, dtype=np.float32) / 8.0
    g[3] = np.linspace(1.0, -1.0, 64, dtype=np.float32)   # max first, min last
    g[4] = np.where(np.arange(64) % 2 == 0, -1.0, 1.0)
    g[5] = np.arange(64, dtype=np.float32) * np.float32(1e-30)
    g[6] = (np.arange(64, dtype=np.float32) - 31.5) * np.float32(1e30)
    g[7] = rng.standard_normal(64)
    g[7][0], g[7][9] = 0.0, -0.0                          # signed zeros, +0 first
    g[8] = np.abs(rng.standard_normal(64))
    g[8][0], g[8][5] = -0.0, 0.0                          # min is a zero, -0 first
    g[9] = -np.abs(rng.standard_normal(64))
    g[9][3], g[9][0] = 0.0, -0.0                          # max is a zero, -0 first
    s = np.float32(0.75)                                  # exact half ticks
    g[10] = np.float32(-2.0) + (np.arange(64) % 16).astype(np.float32) * s / 2
    g[11:] = (rng.standard_normal((13, 64)) *
              np.exp(rng.uniform(-8, 8, (13, 1)))).astype(np.float32)
    return g.reshape(-1)


def main():
    R = O.ref_lib(avx512=True)
    S = O.ref_lib()
    if R is None or S is None:
        raise SystemExit("needs oracle/_ref (make -C oracle ref) and an AVX-512 CPU")
    x = blocks_in()
    nb = x.size // 64
    blocks = np.zeros((nb, 40), np.uint8)
    S.eakv_quantize_row(O._p(x), O._p(blocks), x.size)
    avx = np.zeros_like(blocks)
    R.eakv_quantize_row(O._p(x), O._p(avx), x.size)
    diff = np.nonzero((blocks != avx).any(axis=1))[0]
    for i in diff:                        # only the sign of a zero minimum
        assert np.array_equal(blocks[i, :39], avx[i, :39]), i
        m_s, m_a = blocks[i, 36:40].view(np.float32)[0], avx[i, 36:40].view(np.float32)[0]
        assert m_s == 0.0 and m_a == 0.0, i
    print(f"blocks where the AVX-512 build keeps the other zero: {diff.tolist()}")
    assert np.array_equal(blocks, O.ggml_quantize_row(x)), "oracle quantizer differs"
    deq = np.zeros(x.size, np.float32)
    R.eakv_dequantize_row(O._p(blocks), O._p(deq), x.size)
    assert np.array_equal(deq.view(np.uint32), O.ggml_dequantize_row(blocks).view(np.uint32))

    rng = np.random.default_rng(0xEA4B41)
    n, nrc = 512, 3
    dot_x = np.stack([O.ggml_quantize_row(rng.standard_normal(n).astype(np.float32)).reshape(-1)
                      for _ in range(nrc)])
    dot_y = rng.standard_normal((nrc, n)).astype(np.float32)
    dot = np.zeros(nrc, np.float32)
    R.eakv_vec_dot_q4_f32(n, O._p(dot), 4, O._p(dot_x), dot_x.shape[1], O._p(dot_y), n * 4, nrc)
    one = np.zeros(1, np.float32)
    R.eakv_vec_dot_q4_f32(n, O._p(one), 0, O._p(dot_x), 0, O._p(dot_y), 0, 1)
    assert one[0] == dot[0], "nrc = 1 and nrc = 3 paths differ"
    assert np.array_equal(dot.view(np.uint32), O.ggml_vec_dot(dot_x, dot_y).view(np.uint32))

    path = os.path.join(HERE, "ggml_rows.npz")
    np.savez(path, x=x, blocks=blocks, deq=deq, dot_x=dot_x, dot_y=dot_y, dot=dot)
    mpath = os.path.join(HERE, "manifest.json")
    manifest = json.load(open(mpath))
    manifest["ggml_rows.npz"] = hashlib.sha256(open(path, "rb").read()).hexdigest()
    with open(mpath, "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"wrote {path} ({os.path.getsize(path)} B)")


if __name__ == "__main__":
    main()
