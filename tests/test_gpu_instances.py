"""Every instantiation of the fused matrix-core kernel against the oracle.

mfma_kernel<D, HH, false, TT> exists for head_dim D in {64, 128}, one or two
quads of q heads per wave (HH) and 32- or 64-token tiles (TT, two quads
only).  Which one a call runs follows from the launch plan (q heads per kv
head, the grid against the chip's resident blocks, tiles per wave); each
case below picks a shape whose plan, read back from the library
(eakv_attention_fused_plan) and asserted, is the instantiation named, so
every compiled form of the kernel meets the reference bar
(fused_attention.ea:190-373) at least once, with both entry points giving
the same bits.  The same six forms in V-sum mode (the unfused output call
for 2-8 q heads per kv head) are held to the oracle's V-sum.  The 70B-shape
and headline launches (test_gpu_headline) cover d=128 with two quads and
64-token tiles, and d=128 with one quad, at their own shapes.
"""
import numpy as np
import pytest

from test_gpu_headline import (E, batch_call, build_batch, chan_k,  # noqa: F401
                               compare_sequences, n_cu, say)

pytestmark = pytest.mark.gpu


# (d, q heads, kv heads, contexts of the batch, expected quads, tile tokens):
# the plan's arithmetic on 256 CUs, asserted below
CASES = [
    # one quad (4 q heads per kv head), d=64, 16 kv heads x 2 sequences
    (64, 64, 16, [9000, 7777], 1, 32),
    # two quads, d=128, one sequence: 32 chunks per kv head, 32-token
    # tiles (fewer than 4 tiles of 64 per wave), merged by a second launch
    (128, 64, 8, [20000], 2, 32),
    # two quads, d=64, one sequence: 40 chunks per kv head, 32-token tiles
    (64, 64, 8, [20000], 2, 32),
    # two quads, d=64, 8 sequences: 8 chunks per unit, 64-token tiles,
    # merged in the launch; one sequence shorter than the others
    (64, 64, 8, [16400] * 7 + [9001], 2, 64),
    # two quads, d=128, 4 sequences: 8 chunks per unit, 64-token tiles
    (128, 64, 8, [16400, 16400, 16400, 16399], 2, 64),
    # the same launch with ragged contexts: one token, a third of the tiles
    (128, 64, 8, [16400, 1, 5555, 16399], 2, 64),
]


@pytest.mark.parametrize("d,n_q,n_kv,lens,quads,tile", CASES)
def test_fused_instantiation(E, d, n_q, n_kv, lens, quads, tile):  # noqa: F811
    n_seq = len(lens)
    say("instance: build", d, n_q, n_kv, lens)
    gs, os_ = build_batch(E, 0xEA4B + 300 + d + n_seq, n_seq, n_kv, d, lens, max(lens) + 8,
                          chan_k)
    plan = E.fused_plan(gs, n_q, n_kv)
    say("instance: plan", plan)
    assert plan["mfma"] == 1 and plan["split"] == 1
    if n_cu() == 256:
        assert (plan["quads"], plan["tile_tokens"]) == (quads, tile)
        assert plan["waves_per_block"] == (4 if quads == 1 else 8)
    rng = np.random.default_rng(0xEA4B + 301 + d)
    q = rng.standard_normal((n_seq, n_q, d), dtype=np.float32)
    out = batch_call(E, "eakv_attention_fused_batch_device", gs, q, n_q, n_kv)
    out_na = batch_call(E, "eakv_attention_fused_batch_device_noalloc", gs, q, n_q, n_kv)
    assert np.array_equal(out.view(np.uint32), out_na.view(np.uint32))
    compare_sequences(os_, q, out, n_q, n_kv, lens)
    for g in gs:
        g.free()


# The unfused V-sum's matrix-core program (mfma_kernel<D, HH, true, TT>, 2-8
# q heads per kv head) is planned by the same rules as a one-sequence fused
# call on the same cache (virtual heads, chunks, tile size), so that call's
# plan names the instantiation the V-sum runs.
VS_CASES = [
    (128, 32, 8, 9000, 1, 32),
    (64, 32, 8, 9000, 1, 32),
    (128, 64, 8, 20000, 2, 32),
    (64, 64, 8, 16400, 2, 32),
    (128, 128, 16, 32800, 2, 64),
    (64, 256, 32, 32800, 2, 64),
]


@pytest.mark.parametrize("d,n_q,n_kv,L,quads,tile", VS_CASES)
def test_vsum_instantiation(E, d, n_q, n_kv, L, quads, tile):  # noqa: F811
    import oracle as O
    from conftest import tol_close
    say("vsum instance: build", d, n_q, n_kv, L)
    gs, os_ = build_batch(E, 0xEA4B + 400 + d + n_kv, 1, n_kv, d, [L], L + 8, chan_k)
    g, o = gs[0], os_[0]
    plan = E.fused_plan([g], n_q, n_kv)
    say("vsum instance: plan", plan)
    assert plan["mfma"] == 1 and plan["split"] == 1
    if n_cu() == 256:
        assert (plan["quads"], plan["tile_tokens"]) == (quads, tile)
    rng = np.random.default_rng(0xEA4B + 401 + d)
    q = rng.standard_normal((n_q, d), dtype=np.float32)
    avx = O.avx512_available()
    w = O.softmax_rows(o.attention_scores_avx512(q, 0, n_q, n_kv) if avx
                       else o.attention_scores(q, 0, n_q, n_kv))
    want = o.attention_output_avx512(w, 0, n_q, n_kv) if avx \
        else o.attention_output(w, 0, n_q, n_kv)
    ok, err, nbad = tol_close(g.attention_output(w, 0, n_q, n_kv), want, 1e-4, 1e-5)
    say("vsum instance: max err", err)
    assert ok, (err, nbad)
    g.free()
    o.free()
