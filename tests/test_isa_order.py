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
mfma_kernel instantiation: the order of each group's loads, the values and
places of the compiled vmcnt waits around every group, and that no other
memory instruction or register spill sits in the pipeline.
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


def tokens(body):
    """(label, tokens) per basic block: 'D' / 'g' as in blocks(), ('w', N)
    for an s_waitcnt with vmcnt(N), 'X' for any other vector memory
    instruction (global, scratch, flat, buffer store or atomic)."""
    res, label, toks = [], "entry", []
    for ln in body:
        t = ln.strip()
        m = re.match(r"^(\.LBB\d+_\d+):", t)
        if m:
            res.append((label, toks))
            label, toks = m.group(1), []
        elif t.startswith("buffer_load"):
            toks.append("D" if t.endswith(" lds") else "g")
        elif t.startswith("s_waitcnt") and "vmcnt(" in t:
            toks.append(("w", int(re.search(r"vmcnt\((\d+)\)", t).group(1))))
        elif re.match(r"(global_|scratch_|flat_|buffer_store|buffer_atomic)", t):
            toks.append("X")
    res.append((label, toks))
    return res


def check_waits(loop, n_v, n_scale, n_reg):
    """The waits around each pipeline group in the loop blocks `loop`
    [(label, tokens)] as compiled; returns the number of groups checked.
    Before a group is issued, the loads still outstanding are the older
    group's; its V bytes (the slot the iteration reads first) are in once at
    most its scale and register loads are outstanding: the last wait before
    the group must allow at most that many.  After the group is issued, the
    older group's scales (the slot read next) are in once at most its
    register loads and the whole new group are outstanding: a wait allowing
    at most that many must follow before the next group.  No other vector
    memory instruction may sit in the loop (it would change the counts)."""
    grp = n_v + n_scale + n_reg
    v_wait, k_wait = n_scale + n_reg, n_reg + grp
    run = ["D"] * (n_v + n_scale) + ["g"] * n_reg
    n_groups = 0
    for lb, tk in loop:
        assert "X" not in tk, (lb, tk)
        i = 0
        while i < len(tk):
            if tk[i:i + len(run)] != run:
                i += 1
                continue
            n_groups += 1
            before = [t[1] for t in tk[:i] if isinstance(t, tuple)]
            assert before and before[-1] <= v_wait, (lb, tk, i, v_wait)
            rest = tk[i + len(run):]
            nxt = rest.index("D") if "D" in rest else len(rest)
            after = [t[1] for t in rest[:nxt] if isinstance(t, tuple)]
            assert after and min(after) <= k_wait, (lb, tk, i, k_wait)
            i += len(run)
    return n_groups


@pytest.mark.parametrize("d,hh,vs,tt", INSTANCES)
def test_explicit_waits_cover_the_slots(kernels, d, hh, vs, tt):
    gpd = d // 64
    n_scale = max(4 * tt * gpd * 4, 1024) // 1024
    n_v = (tt * 32 * gpd) // 1024
    n_reg = (tt // 16) * (hh if vs else gpd)
    loop = [(lb, tk) for lb, tk in tokens(kernels[(d, hh, vs, tt)])
            if any(t in ("D", "g") for t in tk)][1:]
    assert loop
    assert check_waits(loop, n_v, n_scale, n_reg) >= 1


def test_check_waits_catches_planted_orders():
    """check_waits on hand-made loop blocks (1 V load, 1 scale load, 2
    register loads per group: V wait 3, scale wait 6): the compiled pattern
    passes; a V wait that allows too many loads, a register load sunk past
    the scale wait, a missing scale wait and a stray store each fail."""
    w = lambda n: ("w", n)
    good = [("L", [w(3), "D", "D", "g", "g", w(6), w(4)])]
    assert check_waits(good, 1, 1, 2) == 1
    bad = [
        [("L", [w(4), "D", "D", "g", "g", w(6)])],            # V wait too weak
        [("L", [w(3), "D", "D", "g", w(6), "g"])],            # a load sunk past the wait
        [("L", [w(3), "D", "D", "g", "g", w(7)])],            # scale wait too weak
        [("L", [w(3), "D", "D", "g", "g", "X", w(6)])],       # another memory instruction
    ]
    for loop in bad:
        with pytest.raises(AssertionError):
            assert check_waits(loop, 1, 1, 2) == 1


def test_no_scratch_in_the_fused_kernels(kernels):
    """A spilled register would put scratch loads and stores, counted by the
    same vmcnt, inside the pipeline: every mfma_kernel instantiation has no
    private segment and no spills."""
    text = open(ASM).read()
    metas = text.split("  - .agpr_count:")[1:]
    seen = 0
    for m in metas:
        name = re.search(r"\.name:\s+(\S+)", m).group(1)
        if "mfma_kernel" not in name:
            continue
        seen += 1
        assert int(re.search(r"\.private_segment_fixed_size:\s+(\d+)", m).group(1)) == 0, name
        assert int(re.search(r"\.vgpr_spill_count:\s+(\d+)", m).group(1)) == 0, name
        assert int(re.search(r"\.sgpr_spill_count:\s+(\d+)", m).group(1)) == 0, name
    assert seen == len(INSTANCES)
