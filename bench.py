"""Benchmark: fused Q4 decode attention on one MI355X.

Default workload (Llama-3-8B-shape GQA, the headline metric): 8 independent
caches (8 concurrent sequences), 32 layers, 32 q heads / 8 kv heads, d=128,
32K context.  One step = append one new token to every sequence (all layers,
K and V, one batched quantize launch), then fused attention over the full
32768-token context for every layer (one launch per layer covering all 8
sequences), then O(1) restore to 32767 tokens so every step sees the same
context.  Inputs are synthetic, seeded, generated on the device; the caches
and queries are resident in HBM before the timed region starts.

Prints ONE JSON line.  `value` is the whole step time per layer (µs);
`roofline` is the fused attention launch: algorithmic bytes (K and V Q4 read
once: 160 B per token-head at d=128, plus q in and out) over its average
duration from HIP events on its stream.  `cpu_baseline` is the CPU oracle's
two-pass fused attention (oracle/eakv_oracle.c) on a bounded sample of the
same workload, run on this host's cores.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
SEED_BASE = 0xEA4B

# name, layers, q heads, kv heads, d, context, sequences, K dist, V dist
CONFIGS = {
    1: dict(name="mha-8h-d128-2k", nl=1, nq=8, nkv=8, d=128, L=2048, nseq=1,
            k="normal", v="normal"),
    2: dict(name="tinyllama-gqa8-d64-4k", nl=22, nq=32, nkv=4, d=64, L=4096, nseq=1,
            k="chan", v="normal"),
    3: dict(name="llama2-7b-mha-d128-8k", nl=32, nq=32, nkv=32, d=128, L=8192, nseq=1,
            k="drift", v="drift"),
    4: dict(name="llama3-8b-gqa4-d128-32k-x8", nl=32, nq=32, nkv=8, d=128, L=32768,
            nseq=8, k="chan", v="normal"),
    5: dict(name="70b-gqa8-d128-128k", nl=80, nq=64, nkv=8, d=128, L=131072, nseq=1,
            k="chan_outlier", v="chan_outlier"),
}


class Synth:
    """ctypes front of eakv_amd/libeakv_synth.so."""

    class Params(C.Structure):
        _fields_ = [("seed", C.c_uint64), ("row0", C.c_int64), ("pos0", C.c_int64),
                    ("sigma", C.c_float), ("chan", C.c_void_p),
                    ("drift_amp", C.c_float), ("drift_period", C.c_float),
                    ("outlier_p", C.c_float), ("outlier_v", C.c_float)]

    def __init__(self):
        self.lib = C.CDLL(os.path.join(ROOT, "eakv_amd", "libeakv_synth.so"))
        self.lib.eakv_synth_fill.restype = C.c_int
        self.lib.eakv_synth_fill.argtypes = [C.c_void_p, C.c_int64, C.c_int64, C.c_int,
                                             C.POINTER(self.Params), C.c_void_p]

    def fill(self, ptr, n_rows, n_tok, d, seed, row0, pos0, kind, chan_ptr=None,
             stream=None):
        p = self.Params(seed=seed, row0=row0, pos0=pos0, sigma=1.0, chan=None,
                        drift_amp=0.0, drift_period=512.0, outlier_p=0.0, outlier_v=0.0)
        if kind in ("chan", "chan_outlier"):
            p.chan = chan_ptr
        if kind == "chan_outlier":
            p.outlier_p, p.outlier_v = 0.01, 20.0
        if kind == "drift":
            p.sigma, p.drift_amp = 1.5, 0.1
        rc = self.lib.eakv_synth_fill(ptr, n_rows, n_tok, d, C.byref(p), stream)
        if rc:
            raise RuntimeError(f"synth launch failed: {rc}")


def channel_scales(cfg, seed):
    """Per (sequence, layer, kv, head, dim) K/V channel multipliers (host)."""
    rng = np.random.default_rng(seed)
    nseq, nl, nkv, d = cfg["nseq"], cfg["nl"], cfg["nkv"], cfg["d"]
    ch = np.ones((nseq, nl, 2, nkv, d), np.float32)
    for kv, kind in ((0, cfg["k"]), (1, cfg["v"])):
        if kind == "chan":
            ch[:, :, kv] = np.exp(rng.uniform(np.log(0.5), np.log(4.0), (nseq, nl, nkv, d)))
            for s in range(nseq):
                for l in range(nl):
                    for h in range(nkv):
                        ch[s, l, kv, h, rng.choice(d, 2, replace=False)] *= 10.0
        elif kind == "chan_outlier":
            ch[:, :, kv] = np.exp(rng.uniform(np.log(0.25), np.log(8.0), (nseq, nl, nkv, d)))
    return ch


class Workload:
    def __init__(self, cfg_id, ctx=None):
        import eakv_amd as E
        from eakv_amd import hipmem as H
        self.E, self.H = E, H
        self.cfg = dict(CONFIGS[cfg_id])
        if ctx:
            self.cfg["L"] = ctx
        c = self.cfg
        self.seed = SEED_BASE + cfg_id
        self.L0 = c["L"] - 1                     # each step appends token L-1
        self.lmax = c["L"] + 64
        self.synth = Synth()
        self.caches = [E.Cache(c["nl"], c["nkv"], c["d"], self.lmax) for _ in range(c["nseq"])]
        self.handles = E.handles(self.caches)
        self.stream = self.caches[0].stream
        self.chan = H.DeviceArray.from_host(channel_scales(c, self.seed))
        self.out = H.DeviceArray((c["nseq"], c["nq"], c["d"]))
        self.tok = H.DeviceArray((c["nseq"], c["nl"], 2, c["nkv"], 1, c["d"]))
        self.quant_ms = None

    def row0(self, s, layer, kv):
        c = self.cfg
        return ((s * c["nl"] + layer) * 2 + kv) * c["nkv"]

    def fill_context(self, time_quantize=True):
        """Synthesize and quantize L0 tokens per layer of every sequence; the
        quantize launches are timed with events."""
        E, H, c = self.E, self.H, self.cfg
        slab = H.DeviceArray((2, c["nkv"], self.L0, c["d"]))
        half = c["nkv"] * self.L0 * c["d"] * 4
        ev0, ev1 = H.Event(), H.Event()
        qtime = 0.0
        for s, cache in enumerate(self.caches):
            cache.clear()
            for l in range(c["nl"]):
                for kv, kind in ((0, c["k"]), (1, c["v"])):
                    r0 = self.row0(s, l, kv)
                    self.synth.fill(slab.ptr + kv * half, c["nkv"], self.L0, c["d"],
                                    self.seed, r0, 0, kind,
                                    self.chan.ptr + r0 * c["d"] * 4, self.stream)
                ev0.record(self.stream)
                for kv in (0, 1):
                    rc = E.lib().eakv_cache_append_device(cache.h, slab.ptr + kv * half, l, kv,
                                                          self.L0, self.stream)
                    assert rc == 0, E.last_error()
                ev1.record(self.stream)
                ev1.synchronize()
                qtime += ev0.elapsed_ms(ev1)
            cache.advance(self.L0)
        slab.free()
        self.quant_ms = qtime
        self.quant_bytes = (c["nseq"] * c["nl"] * 2 * c["nkv"] * self.L0 * c["d"]) * (4 + 0.625)

    def step(self, events=None):
        """Append the token at position L0 everywhere, attend every layer,
        rewind to L0.  events: a pair recorded on the launch stream right
        before the first and right after the last fused-attention call (no
        event between the calls: each is a barrier that drains the queue)."""
        E, c = self.E, self.cfg
        rc = E.lib().eakv_append_batch_device(self.handles, c["nseq"], self.tok.ptr, 1, None)
        assert rc == 0, E.last_error()
        for cache in self.caches:
            cache.advance(1)
        if events:
            events[0].record(self.stream)
        for l in range(c["nl"]):
            rc = E.lib().eakv_attention_fused_batch_device(
                self.handles, c["nseq"], l, self.ql[l].ptr, c["nq"], c["nkv"],
                self.out.ptr, None)
            assert rc == 0, E.last_error()
        if events:
            events[1].record(self.stream)
        for cache in self.caches:
            cache.restore(self.L0)

    def prepare_step_inputs(self):
        """New-token K/V in the batched-append layout
        [seq][layer][kv][head][1][d] and per-layer queries [seq][q][d]."""
        H, c = self.H, self.cfg
        # one call per (seq, layer, kv) keeps row ids and channel scales aligned
        for s in range(c["nseq"]):
            for l in range(c["nl"]):
                for kv, kind in ((0, c["k"]), (1, c["v"])):
                    r0 = self.row0(s, l, kv)
                    self.synth.fill(self.tok.ptr + r0 * c["d"] * 4, c["nkv"], 1, c["d"],
                                    self.seed, r0, self.L0, kind,
                                    self.chan.ptr + r0 * c["d"] * 4, self.stream)
        self.ql = []
        for l in range(c["nl"]):
            a = H.DeviceArray((c["nseq"], c["nq"], c["d"]))
            self.synth.fill(a.ptr, c["nseq"] * c["nq"], 1, c["d"], self.seed + 7,
                            (l + 1) << 20, 0, "normal", stream=self.stream)
            self.ql.append(a)

    def fused_bytes(self):
        c = self.cfg
        ctx = self.L0 + 1
        per_token_head = 2 * (c["d"] // 64) * 40
        return c["nseq"] * (c["nkv"] * ctx * per_token_head + c["nq"] * c["d"] * 4 * 2)


def cpu_baseline(cfg, budget_s=12.0):
    """Time the reference's CPU fused attention (the oracle's two-pass
    restatement of fused_attention.ea, on AVX-512 where the host has it, as
    the reference's kernels compile; else the scalar restatement) over one
    sequence x one layer, all q heads, full context: the median of up to 50
    single-threaded runs after a warmup, then up to 24 units per thread spread
    over up to 16 threads (10-20 s of CPU work at the 32K configuration).
    Per layer = per unit x the configuration's sequences."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    nkv, nq, d, L = cfg["nkv"], cfg["nq"], cfg["d"], cfg["L"]
    rng = np.random.default_rng(SEED_BASE)
    oc = O.OracleCache(1, nkv, d, L)
    data = rng.standard_normal((1, 2, nkv, L, d), dtype=np.float32)
    oc.load_raw(data, L)
    del data
    q = rng.standard_normal((nq, d)).astype(np.float32)
    avx = O.avx512_available()
    run = (lambda: oc.attention_fused_avx512(q, 0, nq, nkv)) if avx else \
        (lambda: oc.attention_fused(q, 0, nq, nkv))
    t0 = time.perf_counter()
    run()                                                   # warmup
    first = time.perf_counter() - t0
    n1 = int(max(3, min(50, budget_s / 2 / max(first, 1e-4))))
    times = []
    for _ in range(n1):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    single = float(np.median(times))
    threads = max(1, min(16, os.cpu_count() or 1))
    reps = threads * max(1, min(24, int(budget_s / 2 / max(single, 1e-4) / 2)))
    t0 = time.perf_counter()
    with ThreadPoolExecutor(threads) as ex:
        list(ex.map(lambda _: run(), range(reps)))
    allcore = (time.perf_counter() - t0) / reps             # s per unit, all threads busy
    per_layer_us = lambda unit_s: unit_s * cfg["nseq"] * 1e6
    what = ("AVX-512 restatement (16-lane intrinsics, bit-identical to the scalar oracle)"
            if avx else "scalar C restatement (this host lacks AVX-512)")
    return {
        "value": round(per_layer_us(allcore), 1), "unit": "us/layer",
        "cores": threads, "kind": "port", "isa": "avx512" if avx else "scalar",
        "single_core_us_per_layer": round(per_layer_us(single), 1),
        "sample": (f"reference CPU fused attention (fused_attention.ea two-pass, extended "
                   f"to GQA), {what}: 1 sequence x 1 layer, {nq}q/{nkv}kv d{d} ctx {L}; "
                   f"single-threaded median of {n1} runs after a warmup; {reps} runs on "
                   f"{threads} threads; scaled x{cfg['nseq']} sequences per layer"),
    }


def copy_calibration(n_bytes, reps=5):
    """Copy n_bytes device-to-device `reps` times with the synth library's
    streaming copy kernel; prints the bytes read and written per launch."""
    from eakv_amd import hipmem as H
    lib = Synth().lib
    lib.eakv_synth_copy.restype = C.c_int
    lib.eakv_synth_copy.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]
    src = H.DeviceArray((n_bytes // 4,))
    dst = H.DeviceArray((n_bytes // 4,))
    e0, e1 = H.Event(), H.Event()
    ms = []
    for _ in range(reps):
        e0.record(None)
        rc = lib.eakv_synth_copy(dst.ptr, src.ptr, n_bytes, None)
        if rc:
            raise RuntimeError(f"copy launch failed: {rc}")
        e1.record(None)
        e1.synchronize()
        ms.append(e0.elapsed_ms(e1))
    print(json.dumps({"copy_bytes_read": n_bytes, "copy_bytes_written": n_bytes,
                      "launches": reps, "ms": [round(m, 4) for m in ms],
                      "gbs_read_plus_write": round(2 * n_bytes / min(ms) / 1e6, 1)}),
          flush=True)


def read_peak(n_bytes, regions=8, reps=3):
    """Sustained HBM read rate of the synth library's plain streaming read
    kernel over passes of n_bytes: `regions` separate buffers read back to
    back (no pass finds its bytes in the last-level cache), best of `reps`
    rounds; 3 blocks of 256 threads per CU.  Returns GB/s."""
    from eakv_amd import hipmem as H
    lib = Synth().lib
    lib.eakv_synth_read.restype = C.c_int
    lib.eakv_synth_read.argtypes = [C.c_void_p, C.c_int64, C.c_void_p, C.c_int, C.c_void_p]
    n_bytes = (n_bytes + 15) // 16 * 16
    lib.eakv_synth_cu_count.restype = C.c_int
    blocks = 3 * (lib.eakv_synth_cu_count() or 256)
    buf = H.DeviceArray((regions * n_bytes // 4,))
    buf.zero()
    H.synchronize()
    sink = H.DeviceArray((blocks * 256,))
    e0, e1 = H.Event(), H.Event()
    best = None
    for _ in range(reps):
        e0.record(None)
        for r in range(regions):
            rc = lib.eakv_synth_read(buf.ptr + r * n_bytes, n_bytes, sink.ptr, blocks, None)
            if rc:
                raise RuntimeError(f"read launch failed: {rc}")
        e1.record(None)
        e1.synchronize()
        ms = e0.elapsed_ms(e1) / regions
        best = ms if best is None else min(best, ms)
    buf.free()
    sink.free()
    return n_bytes / best / 1e6


def dequant_bench(w, steps, warmup):
    """Whole-plane dequantization (eakv_dequantize_range_device) of every
    (layer, kv) block of the first cache, back to back into one f32 buffer:
    40 B read (nibbles, scale, bias) and 256 B written per group.  Returns
    the JSON line."""
    E, H, c = w.E, w.H, w.cfg
    cache = w.caches[0]
    ng = c["nkv"] * w.lmax * c["d"] // 64
    out = H.DeviceArray((ng, 64))
    L = E.lib()
    planes = [(l, kv) for l in range(c["nl"]) for kv in range(2)]

    def one_pass():
        for l, kv in planes:
            rc = L.eakv_dequantize_range_device(cache.h, l, kv, 0, ng, out.ptr, None)
            assert rc == 0, E.last_error()

    for _ in range(warmup):
        one_pass()
    H.synchronize()
    e0, e1 = H.Event(), H.Event()
    e0.record(w.stream)
    for _ in range(steps):
        one_pass()
    e1.record(w.stream)
    e1.synchronize()
    us = e0.elapsed_ms(e1) * 1e3 / (steps * len(planes))
    alg = ng * (40 + 256)
    gbs = alg / (us * 1e-6) / 1e9
    return {"metric": "plane dequantize to f32 GB/s (40 B read + 256 B written per group)",
            "value": round(gbs, 1), "unit": "GB/s", "higher_is_better": True,
            "us_per_plane": round(us, 3), "groups_per_plane": ng, "planes_per_step": len(planes),
            "steps": steps, "n_gpus": 1, "dtype": "q4_1 -> f32",
            "config": {"workload": c["name"], "plane": f"{c['nkv']} kv heads x {w.lmax} tokens x d{c['d']}"},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "alg_bytes_per_launch": alg}}


def validate_bench(w, steps, warmup):
    """The integrity check (eakv_validate) of the first cache: every (layer,
    kv) block's scales and biases over the groups the reference checks, 8 B
    read per group.  eakv_validate returns when its codes are on the host, so
    this times the whole call (host clock): one kernel, a 0xff fill of the
    per-block results and their copy back."""
    E, c = w.E, w.cfg
    cache = w.caches[0]
    res = np.zeros(2 * c["nl"], np.int32)
    L = E.lib()
    for _ in range(warmup):
        assert L.eakv_validate(cache.h, res.ctypes.data) == 0, E.last_error()
    t = []
    for _ in range(steps):
        t0 = time.perf_counter()
        assert L.eakv_validate(cache.h, res.ctypes.data) == 0, E.last_error()
        t.append(time.perf_counter() - t0)
    us = float(np.median(t)) * 1e6
    n = c["nkv"] * c["d"] * cache.seq_len // 64
    alg = 2 * c["nl"] * n * 8
    gbs = alg / (us * 1e-6) / 1e9
    return {"metric": "integrity check GB/s (scale + bias read per group, whole host call)",
            "value": round(gbs, 1), "unit": "GB/s", "higher_is_better": True,
            "us_per_call": round(us, 1), "groups_per_block": n, "blocks": 2 * c["nl"],
            "codes": res.tolist()[:4], "steps": steps, "n_gpus": 1, "dtype": "f32 bit tests",
            "config": {"workload": c["name"]},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "alg_bytes_per_call": alg}}


def ggml_bench(steps, warmup, n_rows=65536, k=4096):
    """The ggml block type's device functions on n_rows rows of k f32 values
    (block_q4_1_eakv, 40 B per 64 values): quantize (4 B read + 0.625 B
    written per value), dequantize (0.625 + 4), vec_dot of every row with
    its own f32 row (0.625 + 4 read per value + 4 B per row), each one launch
    over all rows, timed with HIP events."""
    import eakv_amd as E
    from eakv_amd import hipmem as H
    L = E.lib()
    n = n_rows * k
    x = H.DeviceArray((n,))
    Synth().fill(x.ptr, n_rows, 1, k, SEED_BASE, 0, 0, "normal")
    y = H.DeviceArray((n,))
    Synth().fill(y.ptr, n_rows, 1, k, SEED_BASE + 1, 0, 0, "normal")
    blocks = H.DeviceArray((n // 64 * 40 // 4,))
    deq = H.DeviceArray((n,))
    s = H.DeviceArray((n_rows,))
    row_b = k // 64 * 40
    calls = {
        "quantize_row": (lambda: L.eakv_ggml_quantize_row_device(x.ptr, blocks.ptr, n, None),
                         n * 4 + n // 64 * 40),
        "dequantize_row": (lambda: L.eakv_ggml_dequantize_row_device(blocks.ptr, deq.ptr, n, None),
                           n // 64 * 40 + n * 4),
        "vec_dot": (lambda: L.eakv_ggml_vec_dot_device(k, s.ptr, 4, blocks.ptr, row_b, y.ptr,
                                                       k * 4, n_rows, None),
                    n // 64 * 40 + n * 4 + n_rows * 4),
    }
    res = {}
    for name, (call, alg) in calls.items():
        for _ in range(warmup):
            assert call() == 0, E.last_error()
        H.synchronize()
        e0, e1 = H.Event(), H.Event()
        e0.record(None)
        for _ in range(steps):
            assert call() == 0, E.last_error()
        e1.record(None)
        e1.synchronize()
        us = e0.elapsed_ms(e1) * 1e3 / steps
        gbs = alg / (us * 1e-6) / 1e9
        res[name] = {"us_per_call": round(us, 2), "gbs": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "alg_bytes_per_call": alg}
    return {"metric": "ggml block type device functions, GB/s of algorithmic bytes",
            "unit": "GB/s", "n_gpus": 1, "steps": steps, "dtype": "block_q4_1_eakv <-> f32",
            "config": {"rows": n_rows, "k": k, "bytes_f32": n * 4}, **res}


def unfused_bench(w, steps, warmup):
    """The reference API's unfused path on the first cache, every layer back
    to back: eakv_attention_scores_device (k_score_kernel), then
    eakv_attention_output_device (v_sum_kernel + chunk_sum_kernel) with
    uniform weights 1/L (timing only; parity is the tests' job).  Returns the
    JSON line with each call's mean time and GB/s of its algorithmic bytes:
    K-score n_kv*L*gpd*40 + n_q*L*4 (scores) + n_q*d*4, V-sum
    n_kv*L*gpd*40 + n_q*L*4 (weights) + n_q*d*4."""
    E, H, c = w.E, w.H, w.cfg
    cache = w.caches[0]
    L = w.L0
    nq, nkv, d = c["nq"], c["nkv"], c["d"]
    scores = H.DeviceArray((nq, L))
    wts = H.DeviceArray.from_host(np.full((nq, L), 1.0 / L, np.float32))
    out = H.DeviceArray((nq, d))
    lib = E.lib()

    def run(which):
        for l in range(c["nl"]):
            q = w.ql[l].ptr                        # sequence 0's queries
            if which == "k":
                rc = lib.eakv_attention_scores_device(cache.h, q, l, nq, nkv, scores.ptr, None)
            else:
                rc = lib.eakv_attention_output_device(cache.h, wts.ptr, l, nq, nkv, out.ptr, None)
            assert rc == 0, E.last_error()

    res = {}
    alg = nkv * L * (d // 64) * 40 + nq * L * 4 + nq * d * 4
    for which, name in (("k", "k_score"), ("v", "v_sum")):
        for _ in range(warmup):
            run(which)
        H.synchronize()
        e0, e1 = H.Event(), H.Event()
        e0.record(w.stream)
        for _ in range(steps):
            run(which)
        e1.record(w.stream)
        e1.synchronize()
        us = e0.elapsed_ms(e1) * 1e3 / (steps * c["nl"])
        res[name] = {"us_per_call": round(us, 3), "gbs": round(alg / (us * 1e-6) / 1e9, 1),
                     "frac": round(alg / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "alg_bytes_per_call": alg}
    return {"metric": "unfused K-score / V-sum per layer call, GB/s of algorithmic bytes",
            "unit": "GB/s", "n_gpus": 1, "steps": steps, "dtype": "q4_1 (u8 nibbles + f32 scale/bias), f32 math",
            "config": {"workload": c["name"], "layers": c["nl"], "q_heads": nq, "kv_heads": nkv,
                       "head_dim": d, "context": L, "sequences": 1},
            **res}


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=4, choices=sorted(CONFIGS))
    ap.add_argument("--ctx", type=int, default=None, help="override context length")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--unfused", action="store_true",
                    help="only time the unfused K-score and V-sum calls on the first "
                         "cache, print their JSON line, then exit")
    ap.add_argument("--dequant", action="store_true",
                    help="only time whole-plane dequantization of the first cache, "
                         "print its JSON line, then exit")
    ap.add_argument("--validate", action="store_true",
                    help="only time the integrity check of the first cache, print its "
                         "JSON line, then exit")
    ap.add_argument("--ggml", action="store_true",
                    help="only time the ggml block type's device functions on 1 GiB of "
                         "f32 rows, print their JSON line, then exit")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB, 5 times (the "
                         "known-size kernel for HBM byte counters), then exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for {args.gpus}); "
              "sharding across GPUs is not built in this version", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration << 20)
        return
    if args.ggml:
        print(json.dumps(ggml_bench(max(1, args.steps), 2)), flush=True)
        return

    from eakv_amd import hipmem as H
    log = lambda *a: print(*a, file=sys.stderr, flush=True)
    w = Workload(args.config, args.ctx)
    c = w.cfg
    log(f"bench: config {args.config} {c['name']} ctx {w.L0 + 1}: filling caches")
    w.fill_context()
    w.prepare_step_inputs()
    H.synchronize()
    if args.dequant:
        print(json.dumps(dequant_bench(w, max(1, args.steps // 4), 1)), flush=True)
        return
    if args.validate:
        print(json.dumps(validate_bench(w, max(3, args.steps), 2)), flush=True)
        return
    if args.unfused:
        print(json.dumps(unfused_bench(w, max(1, args.steps // 4), 1)), flush=True)
        return
    log(f"bench: quantize {w.quant_bytes / 1e9:.2f} GB alg in {w.quant_ms:.2f} ms "
        f"({w.quant_bytes / w.quant_ms / 1e6:.0f} GB/s)")

    for _ in range(args.warmup):
        w.step()
    H.synchronize()
    # one event pair per step around its nl back-to-back fused calls: the
    # steps run back to back, the host waits only after the last one
    events = [[H.Event(), H.Event()] for _ in range(args.steps)]
    t0 = time.perf_counter()
    for k in range(args.steps):
        w.step(events[k])
    H.synchronize()
    total_s = time.perf_counter() - t0
    fused = np.array([e0.elapsed_ms(e1) / c["nl"] for e0, e1 in events])
    fused_us = float(fused.mean() * 1e3)
    alg = w.fused_bytes()
    achieved = alg / (fused_us * 1e-6) / 1e9
    ms_step = total_s / args.steps * 1e3
    log(f"bench: {ms_step:.3f} ms/step, fused {fused_us:.2f} us/layer "
        f"(min {fused.min() * 1e3:.2f}), {achieved:.0f} GB/s")

    traffic = None
    tfile = os.path.join(ROOT, "profiles", f"fused_config{args.config}_traffic.json")
    if os.path.exists(tfile):
        traffic = json.load(open(tfile)).get("hbm_bytes_per_launch")

    read_gbs = read_peak(alg)
    log(f"bench: plain streaming read of {alg / 1e6:.1f} MB passes: {read_gbs:.0f} GB/s")

    cpu = None
    if not args.no_cpu:
        log("bench: CPU baseline")
        cpu = cpu_baseline(c)
        cpu["cpu_model"] = cpu_model()

    line = {
        "metric": "fused Q4 attn µs/layer + achieved HBM GB/s, 32Q/8KV d128 32K ctx, 1 GPU",
        "value": round(ms_step * 1e3 / c["nl"], 3),
        "unit": "us/layer",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_1 (u8 nibbles + f32 scale/bias), f32 math",
        "data": "synthetic: seeded device generator, distributions of the configuration",
        "config": {"workload": c["name"], "layers": c["nl"], "q_heads": c["nq"],
                   "kv_heads": c["nkv"], "head_dim": c["d"], "context": w.L0 + 1,
                   "sequences": c["nseq"],
                   "step": "append 1 token x all layers (K,V) + fused attention x all layers"},
        "fused_us_per_layer": round(fused_us, 3),
        "achieved_gbs": round(achieved, 1),
        "quantize_gbs": round(w.quant_bytes / w.quant_ms / 1e6, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "alg_bytes_per_launch": alg,
                     "measured_read_gbs": round(read_gbs, 1),
                     "frac_of_measured_read": round(achieved / read_gbs, 4)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
