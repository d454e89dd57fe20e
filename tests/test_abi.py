"""CPU-only checks of the C ABI: libeakv.so loads, exports every function
include/eakv.h and include/eakv_hip.h declare (and nothing else), and the
host-side validation that runs before any device call behaves like the
reference (src/cache.c, src/io.c) without a GPU."""
import ctypes as C
import os
import re
import subprocess

import pytest

import eakv_amd as E

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("eakv.h", "eakv_hip.h")]


def declared_functions():
    names = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(eakv_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def exported_functions():
    out = subprocess.run(["nm", "-D", "--defined-only", E.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if " T " in l}


def test_library_loads():
    assert E.lib() is not None


def test_exports_match_headers():
    decl = declared_functions()
    assert len(decl) >= 30
    assert decl == exported_functions()
    assert decl == set(E.SIGNATURES)


def test_reference_api_subset_present():
    # every declaration of reference include/eakv.h:25-83
    ref = {"eakv_cache_create", "eakv_cache_free", "eakv_cache_load_raw",
           "eakv_cache_append", "eakv_cache_advance", "eakv_cache_clear",
           "eakv_checkpoint", "eakv_restore", "eakv_attention_scores",
           "eakv_attention_output", "eakv_cache_save", "eakv_cache_load",
           "eakv_cache_seq_len", "eakv_cache_n_layers", "eakv_cache_n_heads",
           "eakv_cache_head_dim", "eakv_cache_max_seq_len",
           "eakv_cache_compression_ratio"}
    assert ref <= exported_functions()


@pytest.mark.parametrize("dims", [(0, 8, 128, 64), (2, 0, 128, 64), (2, 8, 0, 64),
                                  (2, 8, 128, 0), (2, 3, 100, 64), (-1, 8, 128, 64)])
def test_create_rejects_before_device(dims):
    L = E.lib()
    L.eakv_clear_error()
    assert not L.eakv_cache_create(*dims)
    assert L.eakv_last_error() == E.EAKV_ERR_INVALID


def test_null_handle_calls():
    L = E.lib()
    L.eakv_cache_free(None)
    L.eakv_cache_clear(None)
    buf = (C.c_float * 4)()
    assert L.eakv_cache_load_raw(None, buf, 1) == E.EAKV_ERR_INVALID
    assert L.eakv_cache_append(None, buf, 0, 0, 1) == E.EAKV_ERR_INVALID
    assert L.eakv_cache_advance(None, 1) == E.EAKV_ERR_INVALID
    assert L.eakv_restore(None, 0) == E.EAKV_ERR_INVALID
    assert L.eakv_checkpoint(None) == 0
    for g in ("seq_len", "n_layers", "n_heads", "head_dim", "max_seq_len"):
        assert getattr(L, f"eakv_cache_{g}")(None) == 0
    assert L.eakv_cache_compression_ratio(None) == 0.0
    assert L.eakv_cache_save(None, b"/tmp/x") == E.EAKV_ERR_INVALID
    L.eakv_clear_error()
    L.eakv_attention_scores(None, buf, 0, 1, 1, buf)
    assert L.eakv_last_error() == E.EAKV_ERR_INVALID


def test_load_errors_before_device(tmp_path):
    with pytest.raises(E.EakvError) as e:
        E.Cache.load(str(tmp_path / "missing.eakv"))
    assert e.value.code == E.EAKV_ERR_IO
    p = tmp_path / "bad.eakv"
    p.write_bytes(b"NOPE" + bytes(508))
    with pytest.raises(E.EakvError) as e:
        E.Cache.load(str(p))
    assert e.value.code == E.EAKV_ERR_FORMAT
    p.write_bytes(b"EAKV\x02\x00" + bytes(506))       # version 2
    with pytest.raises(E.EakvError) as e:
        E.Cache.load(str(p))
    assert e.value.code == E.EAKV_ERR_FORMAT
