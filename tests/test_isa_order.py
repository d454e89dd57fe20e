"""Compiled load order of the fused kernel's pipeline (CPU: gfx950 assembly).

mfma_kernel reads LDS slots filled by buffer-load-to-LDS after explicit
`s_waitcnt vmcnt(N)` waits whose N counts the loads issued after the slot's
loads, in source order (the compiler does not order LDS reads after loads to
LDS by itself).  Those counts hold only if the compiled code issues every
pipeline group's loads where the source does: a group is its LDS loads (the
V bytes, then the scales and biases) followed at once by its register loads
(the K bytes, or the V-sum's weights), and each loop block issues whole
groups.  A register load moved into the next block (the compiler once sank
the V-sum's weight loads there) makes a wait too short, and a slot can then
be read before its data has landed.  This test builds the assembly with the
library's own flags (eakv_amd/Makefile, target `asm`) and checks every
mfma_kernel instantiation.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "eakv_amd")
ASM = os.path.join(PKG, "_build", "fused_gfx950.s")
NAME = re.compile(r"^(_ZN12_GLOBAL__N_111mfma_kernelILi(\d+)ELi(\d)ELb(\d)ELi(\d+)E\S*):")


@pytest.fixture(scope="module")
def kernels():
    if not os.path.exists("/opt/rocm/bin/hipcc") and not shutil.which("hipcc"):
        pytest.skip("hipcc not available")
    subprocess.run(["make", "-s", "-C", PKG, "asm"], check=True)
    lines = open(ASM).read().splitlines()
    out = {}
    i = 0
    while i < len(lines):
        m = NAME.match(lines[i])
        if not m:
            i += 1
            continue
        j = i + 1
        while not lines[j].startswith(".Lfunc_end"):
            j += 1
        d, hh, vs, tt = int(m.group(2)), int(m.group(3)), m.group(4) == "1", int(m.group(5))
        out[(d, hh, vs, tt)] = lines[i + 1:j]
        i = j
    return out


def blocks(body):
    """(label, tokens) per basic block: 'D' a buffer load to LDS, 'g' a
    buffer load to registers."""
    res, label, toks = [], "entry", []
    for ln in body:
        t = ln.strip()
        m = re.match(r"^(\.LBB\d+_\d+):", t)
        if m:
            res.append((label, "".join(toks)))
            label, toks = m.group(1), []
        elif t.startswith("buffer_load"):
            toks.append("D" if t.endswith(" lds") else "g")
    res.append((label, "".join(toks)))
    return res


INSTANCES = [(d, hh, vs, tt) for d in (64, 128) for hh in (1, 2) for vs in (False, True)
             for tt in ((32,) if hh == 1 else (32, 64))]


def test_every_instantiation_found(kernels):
    assert set(kernels) == set(INSTANCES)


@pytest.mark.parametrize("d,hh,vs,tt", INSTANCES)
def test_groups_issued_in_source_order(kernels, d, hh, vs, tt):
    gpd = d // 64
    n_scale = max(4 * tt * gpd * 4, 1024) // 1024  # scale loads (1 KB each)
    n_lds = (tt * 32 * gpd) // 1024 + n_scale    # V loads (1 KB each) + the scale loads
    n_reg = (tt // 16) * (hh if vs else gpd)     # weights, or K bytes (16-token parts x groups)
    group = "D" * n_lds + "g" * n_reg
    with_loads = [(lb, tk) for lb, tk in blocks(kernels[(d, hh, vs, tt)]) if tk]
    assert with_loads, "no pipeline loads found"
    # prologue: the 4-byte prime load of a V slot and the first scale load
    # come first (the first explicit wait needs exactly those two)
    assert with_loads[0][1].startswith("DD"), with_loads[0]
    # loop blocks: whole groups, each group's register loads right after its
    # LDS loads
    loop = with_loads[1:]
    assert loop, "no loop blocks with loads"
    for lb, tk in loop:
        assert re.fullmatch("(%s)+" % group, tk), (lb, tk, group)
