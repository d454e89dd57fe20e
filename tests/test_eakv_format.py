"""The .eakv format of the oracle's save and load, pinned by the reference's
packed header struct restated in tests/eakv_format.py (src/io.c:11-28,
:40-160) rather than by the oracle's own offsets.  The GPU library's files
are compared with these in tests/test_gpu_configs.py."""
import numpy as np
import pytest

import eakv_format as F
import oracle as O


def planes_rows(o, layer, kv, seq_len):
    """The first seq_len tokens of every head of one plane, [head][pos][group]."""
    w, s, b = o.read_planes(layer, kv)
    nh, lmax, gpd = o.n_heads, o.max_seq_len, o.head_dim // 64
    w = w.reshape(nh, lmax * gpd, 32)[:, :seq_len * gpd]
    s = s.reshape(nh, lmax * gpd)[:, :seq_len * gpd]
    b = b.reshape(nh, lmax * gpd)[:, :seq_len * gpd]
    return (np.ascontiguousarray(w).tobytes(), np.ascontiguousarray(s).tobytes(),
            np.ascontiguousarray(b).tobytes())


@pytest.mark.parametrize("nl,nh,d,L,lmax", [(2, 4, 128, 32, 32), (1, 3, 64, 10, 10),
                                            (3, 2, 128, 7, 20), (1, 1, 64, 0, 4)])
def test_oracle_file_layout(tmp_path, nl, nh, d, L, lmax):
    rng = np.random.default_rng(nl * 1000 + L)
    o = O.OracleCache(nl, nh, d, lmax)
    if L:
        o.load_raw(rng.standard_normal(nl * 2 * nh * L * d).astype(np.float32), L)
    p = tmp_path / "o.eakv"
    o.save(str(p))
    data = p.read_bytes()
    h, offs, n_groups = F.parse(data)
    assert h["magic"] == b"EAKV" and h["version"] == 1 and h["quant_scheme"] == 0
    assert h["group_size"] == 64 and h["orig_dtype"] == 0 and h["compression"] == 0
    assert (h["n_layers"], h["n_heads"], h["head_dim"]) == (nl, nh, d)
    assert h["seq_len"] == L and h["max_seq_len"] == L     # written as seq_len (io.c:65)
    assert h["model_hash"] == bytes(32) and h["tokenizer_hash"] == bytes(32)
    assert h["checksum"] == 0
    assert data[F.HEADER.size:F.HEADER_SIZE] == bytes(F.HEADER_SIZE - F.HEADER.size)
    assert n_groups == nh * d * L // 64
    start = F.align64(F.HEADER_SIZE + 16 * nl)
    blk = F.align64(40 * n_groups)
    assert offs == [start + i * blk for i in range(2 * nl)]
    assert all(x % 64 == 0 for x in offs)
    assert data[F.HEADER_SIZE + 16 * nl:start] == bytes(start - F.HEADER_SIZE - 16 * nl)
    assert len(data) == start + 2 * nl * blk
    for i, off in enumerate(offs):
        assert F.block(data, off, n_groups) == planes_rows(o, i // 2, i % 2, L)
        assert data[off + 40 * n_groups:off + blk] == bytes(blk - 40 * n_groups)


def test_oracle_loads_independently_built_file(tmp_path):
    """A file written by the restated format, blocks in reverse order with
    gaps between them: load follows the index table."""
    rng = np.random.default_rng(3)
    nl, nh, d, L = 2, 3, 128, 9
    ng = nh * d * L // 64
    blocks = []
    for _ in range(2 * nl):
        w = rng.integers(0, 256, (ng, 32), dtype=np.uint8)
        s = rng.random(ng).astype(np.float32)
        b = rng.standard_normal(ng).astype(np.float32)
        blocks.append((w.tobytes(), s.tobytes(), b.tobytes()))
    p = tmp_path / "x.eakv"
    p.write_bytes(F.build(nl, nh, d, L, blocks, order=reversed(range(2 * nl)), gap=192))
    o = O.OracleCache.load(str(p))
    assert (o.n_layers, o.n_heads, o.head_dim, o.seq_len, o.max_seq_len) == (nl, nh, d, L, L)
    for i in range(2 * nl):
        assert planes_rows(o, i // 2, i % 2, L) == blocks[i]


@pytest.mark.parametrize("what", ["magic", "version", "truncated"])
def test_oracle_rejects_bad_files(tmp_path, what):
    rng = np.random.default_rng(4)
    ng = 2 * 64 * 4 // 64
    blocks = [(rng.integers(0, 256, ng * 32, dtype=np.uint8).tobytes(),
               bytes(4 * ng), bytes(4 * ng))] * 2
    kw = {"magic": {"magic": b"EAKW"}, "version": {"version": 2}, "truncated": {}}[what]
    data = F.build(1, 2, 64, 4, blocks, **kw)
    if what == "truncated":
        data = data[:-100]
    p = tmp_path / "bad.eakv"
    p.write_bytes(data)
    with pytest.raises(O.OracleError) as e:
        O.OracleCache.load(str(p))
    assert e.value.code == -2                                # EAKV_ERR_FORMAT
