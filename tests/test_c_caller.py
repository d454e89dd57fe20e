"""A compiled C caller of the drop-in (tests/c_api/drop_in_caller.c): it
includes only include/eakv.h, links eakv_amd/libeakv.so and runs the
reference's call pattern (create, per-token append of every layer and K/V,
advance, scores, caller softmax, output, checkpoint/restore, save/load, error
codes).  On a GPU its results are compared with the CPU oracle on the inputs
it wrote."""
import os
import subprocess

import numpy as np
import pytest

import eakv_format as F
import oracle as O
from conftest import tol_close

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "c_api", "drop_in_caller.c")
BIN = os.path.join(ROOT, "tests", "c_api", "drop_in_caller")


def test_public_header_compiles_as_c11():
    """include/eakv.h alone, strict C11 with warnings as errors: what the
    reference's C callers compile against."""
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-pedantic",
                        "-fsyntax-only", "-I", os.path.join(ROOT, "include"), SRC],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("hd", [64, 128])
def test_c_caller_against_oracle(tmp_path, hd):
    assert os.path.exists(BIN), "build first: make -C tests/c_api"
    out, ef = tmp_path / "res.bin", tmp_path / "c.eakv"
    print("c-caller", hd, flush=True)
    r = subprocess.run([BIN, str(hd), str(out), str(ef)], capture_output=True, text=True,
                       timeout=120)
    print(r.stdout[-3000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout
    raw = out.read_bytes()
    nl, nh, d, sl, nq = np.frombuffer(raw[:20], np.int32)
    f = np.frombuffer(raw[20:], np.float32)
    n = nl * 2 * nh * sl * d
    data, f = f[:n], f[n:]
    q, f = f[:nq * d].reshape(nq, d), f[nq * d:]
    scores, f = f[:nq * sl].reshape(nq, sl), f[nq * sl:]
    w, f = f[:nq * sl].reshape(nq, sl), f[nq * sl:]
    output = f[:nq * d].reshape(nq, d)
    o = O.OracleCache(int(nl), int(nh), int(d), int(sl))
    o.load_raw(data, int(sl))
    so = o.attention_scores(q, int(nl) - 1, int(nq), int(nh))
    assert np.array_equal(scores.view(np.uint32), so.view(np.uint32))
    ok, err, nbad = tol_close(output, o.attention_output(w, int(nl) - 1, int(nq), int(nh)))
    assert ok, (err, nbad)
    # the file it saved: the restated format, and the oracle's bytes
    po = tmp_path / "o.eakv"
    o.save(str(po))
    cb = ef.read_bytes()
    h, _, _ = F.parse(cb)
    assert (h["n_layers"], h["n_heads"], h["head_dim"], h["seq_len"]) == (nl, nh, d, sl)
    assert cb == po.read_bytes()
