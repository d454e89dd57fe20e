"""Every instantiation of the fused matrix-core kernel against the oracle.

mfma_kernel<D, HH, false, TT> exists for head_dim D in {64, 128}, one or two
quads of q heads per wave (HH) and 32- or 64-token tiles (TT, two quads
only).  Which one a call runs follows from the launch plan (q heads per kv
head, the grid against the chip's resident blocks, tiles per wave); each
case below picks a shape whose plan, read back from the library
(eakv_attention_fused_plan) and asserted, is the instantiation named, so
every compiled form of the kernel meets the reference bar
(fused_attention.ea:190-373) at least once, with both entry points giving
the same bits.  The 70B-shape and headline launches (test_gpu_headline)
cover d=128 with two quads and 64-token tiles, and d=128 with one quad, at
their own shapes.
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
