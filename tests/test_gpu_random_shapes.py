"""A seeded sweep of launch shapes against the CPU oracle.

Each case draws a shape from its own seed: head_dim 64 or 128, 1-8 kv heads,
1-16 q heads per kv head (groups above 8 run as virtual kv heads, odd groups
pad their quads), 1-8 sequences of 1-4000 tokens each (ragged, a one-token
sequence included now and then), and a cache max_seq_len a little above the
longest.  The launch plan follows from the shape (one or two quads, 32- or
64-token tiles, chunks merged in the launch or by a second launch); every
case checks

- the batched fused call (eakv_attention_fused_batch_device) against the
  reference algorithm per sequence (fused_attention.ea:190-373 as restated
  by the oracle) at 1e-4 abs / 1e-5 rel, with the long-context exception
  asserted by check_against_reference;
- its allocation-free form, bit for bit;
- on the first sequence, the unfused K-score bit for bit
  (fused_k_score*.ea as restated by the oracle) and the V-sum on the
  oracle's softmax rows within the same bar.
"""
import numpy as np
import pytest

import oracle as O
from conftest import tol_close
from test_gpu_headline import (E, batch_call, build_batch, compare_sequences,  # noqa: F401
                               say)

pytestmark = pytest.mark.gpu

N_CASES = 24


def draw(case):
    rng = np.random.default_rng(0xEA4B5EED + case)
    d = int(rng.choice([64, 128]))
    n_kv = int(rng.choice([1, 2, 3, 4, 8]))
    qpk = int(rng.choice([1, 2, 3, 4, 5, 6, 8, 11, 16]))
    n_seq = int(rng.choice([1, 2, 3, 5, 8]))
    lens = [int(x) for x in rng.integers(1, 4001, n_seq)]
    if n_seq > 1 and case % 3 == 0:
        lens[int(rng.integers(0, n_seq))] = 1
    lmax = max(lens) + int(rng.integers(0, 70))
    return d, n_kv, qpk, n_seq, lens, lmax


def normal_k(rng, n_kv, L, d):
    return rng.standard_normal((n_kv, L, d), dtype=np.float32) * np.float32(1.5)


@pytest.mark.parametrize("case", range(N_CASES))
def test_random_shape(E, case):  # noqa: F811
    d, n_kv, qpk, n_seq, lens, lmax = draw(case)
    n_q = n_kv * qpk
    say(f"random case {case}: d {d} n_kv {n_kv} q/kv {qpk} seqs {n_seq} lens {lens} "
        f"lmax {lmax}")
    gs, os_ = build_batch(E, 0xEA4B + 500 + case, n_seq, n_kv, d, lens, lmax, normal_k)
    plan = E.fused_plan(gs, n_q, n_kv)
    say("  plan", plan)
    rng = np.random.default_rng(0xEA4B + 600 + case)
    q = rng.standard_normal((n_seq, n_q, d), dtype=np.float32)
    out = batch_call(E, "eakv_attention_fused_batch_device", gs, q, n_q, n_kv)
    out_na = batch_call(E, "eakv_attention_fused_batch_device_noalloc", gs, q, n_q, n_kv)
    assert np.array_equal(out.view(np.uint32), out_na.view(np.uint32))
    compare_sequences(os_, q, out, n_q, n_kv, lens)

    g, o = gs[0], os_[0]
    sg = g.attention_scores(q[0], 0, n_q, n_kv)
    so = o.attention_scores(q[0], 0, n_q, n_kv)
    say("  K-score: max diff", float(np.abs(sg - so).max()) if sg.size else 0.0)
    assert np.array_equal(sg.view(np.uint32), so.view(np.uint32))
    w = O.softmax_rows(so)
    want = o.attention_output_avx512(w, 0, n_q, n_kv) if O.avx512_available() \
        else o.attention_output(w, 0, n_q, n_kv)
    ok, err, nbad = tol_close(g.attention_output(w, 0, n_q, n_kv), want, 1e-4, 1e-5)
    say("  V-sum: max err", err)
    assert ok, (err, nbad)
    for x in gs:
        x.free()
    for x in os_:
        x.free()
