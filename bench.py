"""Benchmark: fused Q4 decode attention on one MI355X, every workload.

Headline (`value`): the Llama-3-8B-shape GQA workload.  8 independent caches
(8 concurrent sequences), 32 layers, 32 q heads / 8 kv heads, d=128, 32K
context.  One step = append one new token to every sequence (all layers, K
and V, one batched quantize launch), then fused attention over the full
32768-token context for every layer (one launch per layer covering all 8
sequences), then O(1) restore to 32767 tokens so every step sees the same
context.  Inputs are synthetic, seeded, generated on the device; the caches
and queries are resident in HBM before the timed region starts.

`configs` holds every workload, each with its own timed steps and its CPU
baseline from the same run:
  1  8Q/8KV d128, 2048 tokens, 1 layer: the unfused API step
     (eakv_attention_scores -> row softmax -> eakv_attention_output);
  2  32Q/4KV d64, 4096 tokens, 22 layers: the same per layer;
  3  32Q/32KV d128, 8192 tokens, 32 layers: the same per layer;
  4  the headline workload above;
  5  64Q/8KV d128, 80 layers: bulk quantization of the full 131072-token
     cache, then 64 decode steps of (append one token to every layer, fused
     attention over every layer), the context growing to 131136.
Configs 1-3 also report the fused call on the same caches.

Prints ONE JSON line.  `roofline` is the headline's fused attention launch:
algorithmic bytes (K and V Q4 read once: 160 B per token-head at d=128, plus
q in and out) over its mean duration from HIP events on its stream.
`cpu_baseline` is the reference's CPU kernels restated with AVX-512
intrinsics (the oracle, bit-identical to its scalar form) on a bounded
sample of the same workload, on this host's cores.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import tempfile
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
SEED_BASE = 0xEA4B
# worker threads for the all-core CPU baseline: every CPU this process may
# run on, at most the 16-CPU share of one GPU on the benchmark hosts
CPU_THREADS_MAX = 16

# name, layers, q heads, kv heads, d, context, sequences, K dist, V dist,
# path: "unfused" (scores -> softmax -> output), "fused" (append + fused,
# context restored each step) or "grow" (append + fused, context growing)
CONFIGS = {
    1: dict(name="mha-8h-d128-2k", nl=1, nq=8, nkv=8, d=128, L=2048, nseq=1,
            k="normal", v="normal", path="unfused"),
    2: dict(name="tinyllama-gqa8-d64-4k", nl=22, nq=32, nkv=4, d=64, L=4096, nseq=1,
            k="chan", v="normal", path="unfused"),
    3: dict(name="llama2-7b-mha-d128-8k", nl=32, nq=32, nkv=32, d=128, L=8192, nseq=1,
            k="drift", v="drift", path="unfused"),
    4: dict(name="llama3-8b-gqa4-d128-32k-x8", nl=32, nq=32, nkv=8, d=128, L=32768,
            nseq=8, k="chan", v="normal", path="fused"),
    5: dict(name="70b-gqa8-d128-128k", nl=80, nq=64, nkv=8, d=128, L=131072, nseq=1,
            k="chan_outlier", v="chan_outlier", path="grow"),
}
HEADLINE = 4
DTYPE = ("q4_1 planes (u8 nibbles, f32 scale and bias per 64 values); fused and V-sum dots "
         "on int8 matrix cores (q and softmax weights as 32-bit fixed point in balanced int8 "
         "digits, exact int32 sums), f32 softmax and recombination; unfused K-score f32 fma")


def metric_text(c):
    return (f"fused Q4 attn µs/layer + achieved HBM GB/s, {c['nq']}Q/{c['nkv']}KV "
            f"d{c['d']} {c['L'] // 1024}K ctx, 1 GPU")


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
        self.lib.eakv_synth_softmax.restype = C.c_int
        self.lib.eakv_synth_softmax.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                                C.c_void_p]
        self.lib.eakv_synth_hold.restype = C.c_int
        self.lib.eakv_synth_hold.argtypes = [C.c_int, C.c_void_p]
        self.lib.eakv_synth_dot_scores.restype = C.c_int
        self.lib.eakv_synth_dot_scores.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                                                   C.c_int, C.c_int, C.c_void_p]

    _one = None

    @classmethod
    def get(cls):
        if cls._one is None:
            cls._one = cls()
        return cls._one

    def hold(self, us, stream=None):
        rc = self.lib.eakv_synth_hold(int(us), stream)
        if rc:
            raise RuntimeError(f"hold launch failed: {rc}")

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

    def softmax(self, scores, w, n_rows, L, stream=None):
        rc = self.lib.eakv_synth_softmax(scores, w, n_rows, L, stream)
        if rc:
            raise RuntimeError(f"softmax launch failed: {rc}")

    def dot_scores(self, k, q, scores, nh, L, d, stream=None):
        rc = self.lib.eakv_synth_dot_scores(k, q, scores, nh, L, d, stream)
        if rc:
            raise RuntimeError(f"dot launch failed: {rc}")


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
    """The caches of one configuration, filled on the device, and its step.

    fused: the caches hold L-1 tokens; a step appends token L-1 and restores
    afterwards.  grow: the caches hold L tokens and each step appends the
    next one (max_seq_len L + 64).  unfused: the caches hold L tokens."""

    def __init__(self, cfg_id, ctx=None):
        import eakv_amd as E
        from eakv_amd import hipmem as H
        self.E, self.H = E, H
        self.cfg = dict(CONFIGS[cfg_id])
        if ctx:
            self.cfg["L"] = ctx
        c = self.cfg
        self.seed = SEED_BASE + cfg_id
        self.grow = c["path"] == "grow"
        # the unfused step reads the cache as filled; the decode steps append
        self.L0 = c["L"] if c["path"] in ("grow", "unfused") else c["L"] - 1
        self.lmax = c["L"] + 64
        self.synth = Synth()
        self.caches = [E.Cache(c["nl"], c["nkv"], c["d"], self.lmax) for _ in range(c["nseq"])]
        self.handles = E.handles(self.caches)
        self.stream = self.caches[0].stream
        self.chan = H.DeviceArray.from_host(channel_scales(c, self.seed))
        self.out = H.DeviceArray((c["nseq"], c["nq"], c["d"]))
        self.tok = H.DeviceArray((c["nseq"], c["nl"], 2, c["nkv"], 1, c["d"]))
        self.quant_ms = None

    def free(self):
        for c in self.caches:
            c.free()
        for a in (self.chan, self.out, self.tok):
            a.free()
        for a in getattr(self, "ql", []):
            a.free()

    def row0(self, s, layer, kv):
        c = self.cfg
        return ((s * c["nl"] + layer) * 2 + kv) * c["nkv"]

    def fill_context(self, log=None, every_layer=False):
        """Synthesize and quantize L0 tokens per layer of every sequence; the
        quantize launches are timed with events.  log: a progress line per
        sequence (and per layer with every_layer), printed as each is done."""
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
                if log and every_layer:
                    log(f"bench: filled sequence {s} layer {l}")
            cache.advance(self.L0)
            if log:
                log(f"bench: filled sequence {s} ({c['nl']} layers x {self.L0} tokens)")
        slab.free()
        self.quant_ms = qtime
        self.quant_bytes = (c["nseq"] * c["nl"] * 2 * c["nkv"] * self.L0 * c["d"]) * (4 + 0.625)

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

    def step(self, events=None):
        """Append the next token everywhere, attend every layer (and, for
        the restored context, rewind to L0).  events: a pair recorded on the
        launch stream right before the first and right after the last
        fused-attention call (no event between the calls: each is a barrier
        that drains the queue)."""
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
        if not self.grow:
            for cache in self.caches:
                cache.restore(self.L0)

    def fused_bytes(self, ctx=None):
        c = self.cfg
        ctx = ctx if ctx is not None else self.L0 + 1
        per_token_head = 2 * (c["d"] // 64) * 40
        return c["nseq"] * (c["nkv"] * ctx * per_token_head + c["nq"] * c["d"] * 4 * 2)

    def unfused_bytes(self):
        """K-score: K planes + scores written + q; softmax: scores read,
        weights written; V-sum: V planes + weights read + out."""
        c = self.cfg
        L, planes = self.L0, c["nkv"] * self.L0 * (c["d"] // 64) * 40
        ks = planes + c["nq"] * L * 4 + c["nq"] * c["d"] * 4
        sm = 2 * c["nq"] * L * 4
        vs = planes + c["nq"] * L * 4 + c["nq"] * c["d"] * 4
        return ks, sm, vs


def timed(H, stream, fn, steps, warmup, per, queued=False):
    """Mean µs per unit of `fn` (one call = `per` units) between two events
    on `stream`, after `warmup` untimed calls.

    queued: the timed calls are enqueued behind a hold launch (one sleeping
    wave) that outlasts their issue on the host, so they run back to back
    from a full queue: device time per call, without the host's issue rate.
    A call of a few microseconds is otherwise host-bound (a 3.4 us K-score
    launch issued from Python every 3.5-8.5 us).  Returns (µs, host issue µs
    per unit) in that mode; the hold is doubled and the run repeated while
    the issue outlasts it."""
    t0 = time.perf_counter()
    for _ in range(warmup):
        fn()
    host = (time.perf_counter() - t0) / max(1, warmup)
    H.synchronize()
    hold_us = int(host * 1e6 * steps * 2) + 500
    for _ in range(4 if queued else 1):
        e0, e1 = H.Event(), H.Event()
        if queued:
            Synth.get().hold(hold_us, stream)
        e0.record(stream)
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        issue_us = (time.perf_counter() - t0) * 1e6
        e1.record(stream)
        e1.synchronize()
        us = e0.elapsed_ms(e1) * 1e3 / (steps * per)
        if not queued:
            return us
        if issue_us < 0.8 * hold_us:
            return us, issue_us / (steps * per)
        hold_us *= 2
    raise RuntimeError(f"timed: the host issue ({issue_us:.0f} us) outlasted a "
                       f"{hold_us // 2} us hold")


# ---------------------------------------------------------------- CPU side

def cpu_info():
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = os.cpu_count() or 1
    return {"cpu_model": model, "host_cpus": os.cpu_count(), "affinity_cpus": aff,
            "threads": max(1, min(CPU_THREADS_MAX, aff))}


def cpu_time(run, budget_s):
    """The reference benchmark's method (bench_libeakv.c:17-39): a warmup,
    then the median of up to 50 single-threaded runs; then the same unit on
    every worker thread at once, three rounds, each unit's time = round time
    / units.  Returns (single s, [all-core s per unit per round], threads,
    single runs, units per round)."""
    info = cpu_info()
    t0 = time.perf_counter()
    run()
    first = time.perf_counter() - t0
    n1 = int(max(5, min(50, budget_s / 2 / max(first, 1e-5))))
    times = []
    for _ in range(n1):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    single = float(np.median(times))
    threads = info["threads"]
    per_thread = max(1, min(8, int(budget_s / 6 / max(single, 1e-5))))
    units = threads * per_thread
    rounds = []
    with ThreadPoolExecutor(threads) as ex:
        for _ in range(3):
            t0 = time.perf_counter()
            list(ex.map(lambda _: run(), range(units)))
            rounds.append((time.perf_counter() - t0) / units)
    return single, rounds, threads, n1, units


def cpu_baseline(cfg, budget_s=6.0):
    """The reference's CPU path for one (sequence, layer) unit of the
    workload on this host, scaled to one layer-step (x sequences):
    fused workloads the two-pass fused attention (fused_attention.ea,
    extended to GQA), unfused ones K-score -> softmax -> V-sum
    (fused_k_score*.ea, fused_v_sum*.ea, fused_k_score_gqa*.ea), on AVX-512
    where the host has it (the oracle's intrinsics restatement, bit-identical
    to its scalar form), else the scalar restatement.  Inputs: N(0,1) (the
    timing does not depend on the values); the full context of the workload."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    nkv, nq, d, L = cfg["nkv"], cfg["nq"], cfg["d"], cfg["L"]
    rng = np.random.default_rng(SEED_BASE)
    oc = O.OracleCache(1, nkv, d, L)
    block = rng.standard_normal(1 << 22, dtype=np.float32)
    oc.load_raw(np.resize(block, 2 * nkv * L * d), L)
    q = rng.standard_normal((nq, d)).astype(np.float32)
    avx = O.avx512_available()
    if cfg["path"] == "unfused":
        sc = (oc.attention_scores_avx512 if avx else oc.attention_scores)
        out = (oc.attention_output_avx512 if avx else oc.attention_output)
        what = "K-score -> row softmax -> V-sum"

        def run():
            out(O.softmax_rows(sc(q, 0, nq, nkv)), 0, nq, nkv)
    else:
        fused = oc.attention_fused_avx512 if avx else oc.attention_fused
        what = "two-pass fused attention"

        def run():
            fused(q, 0, nq, nkv)
    single, rounds, threads, n1, units = cpu_time(run, budget_s)
    oc.free()
    scale = cfg["nseq"] * 1e6
    info = cpu_info()
    isa = ("AVX-512 restatement (16-lane intrinsics, bit-identical to the scalar oracle)"
           if avx else "scalar C restatement (this host lacks AVX-512)")
    return {
        "value": round(float(np.median(rounds)) * scale, 1), "unit": "us/layer",
        "cores": threads, "kind": "port", "isa": "avx512" if avx else "scalar",
        "single_core_us_per_layer": round(single * scale, 1),
        "all_core_us_per_layer_rounds": [round(r * scale, 1) for r in rounds],
        "host_cpus": info["host_cpus"], "affinity_cpus": info["affinity_cpus"],
        "cpu_model": info["cpu_model"],
        "sample": (f"reference CPU {what}, {isa}: 1 sequence x 1 layer, {nq}q/{nkv}kv d{d} "
                   f"ctx {L}; single-threaded median of {n1} runs after a warmup; 3 rounds of "
                   f"{units} units on {threads} threads (all-core value = median round); "
                   f"x{cfg['nseq']} sequences per layer-step"),
    }


def cpu_quantize_baseline(cfg, budget_s=4.0):
    """The reference's bulk quantization (quantize_simd.ea, scalar; the
    oracle's restatement) on a 64 MiB sample of the workload's f32 KV:
    GB/s of algorithmic bytes (4 B read + 0.625 B written per value)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    nkv, d = cfg["nkv"], cfg["d"]
    L = (64 << 20) // (2 * nkv * d * 4)
    data = np.resize(np.random.default_rng(SEED_BASE).standard_normal(1 << 22, dtype=np.float32),
                     2 * nkv * L * d)
    caches = {}

    def run():
        import threading
        k = threading.get_ident()
        if k not in caches:
            caches[k] = O.OracleCache(1, nkv, d, L)
        caches[k].load_raw(data, L)
    single, rounds, threads, n1, units = cpu_time(run, budget_s)
    for c in caches.values():
        c.free()
    alg = data.size * 4.625
    return {"single_core_gbs": round(alg / single / 1e9, 3),
            "all_core_gbs": round(alg / float(np.median(rounds)) / 1e9, 3),
            "all_core_gbs_rounds": [round(alg / r / 1e9, 3) for r in rounds],
            "cores": threads,
            "sample": f"{data.size * 4 >> 20} MiB of f32 ({nkv} kv heads x {L} tokens x d{d}, K and V), "
                      f"scalar restatement of quantize_simd.ea; median of {n1} runs, 3 rounds of "
                      f"{units} on {threads} threads"}


# ---------------------------------------------------------------- GPU side

def measure_fused(w, steps, warmup, log=None):
    """The decode step (append + fused attention over every layer): ms per
    step from the host clock around `steps` back-to-back steps, the fused
    calls' mean from one event pair per step on the launch stream.  A
    growing context is rewound after the warmup steps.  log: a line per
    step once it is enqueued (runs under a profiler)."""
    H, c = w.H, w.cfg
    # a growing context has 64 spare tokens: the warmup appends at most 64
    for _ in range(min(warmup, 64) if w.grow else warmup):
        w.step()
    H.synchronize()
    if w.grow:
        for cache in w.caches:
            cache.restore(w.L0)
    events = [[H.Event(), H.Event()] for _ in range(steps)]
    t0 = time.perf_counter()
    for k in range(steps):
        w.step(events[k])
        if log:
            log(f"bench: step {k} enqueued")
    H.synchronize()
    total_s = time.perf_counter() - t0
    fused = np.array([e0.elapsed_ms(e1) / c["nl"] for e0, e1 in events]) * 1e3
    return total_s / steps * 1e3, float(fused.mean()), [round(float(x), 3) for x in
                                                          np.percentile(fused, [0, 50, 100])]


def measure_unfused(w, steps, warmup):
    """The reference API's unfused step on the first cache, every layer:
    eakv_attention_scores_device, the caller's row softmax, then
    eakv_attention_output_device.  Per-call means of each phase (all layers
    back to back, one event pair) and of the whole step, enqueued behind a
    hold so that they run from a full queue; and the whole step as issued by
    this Python loop straight onto an idle device (host-bound for short
    calls)."""
    E, H, c = w.E, w.H, w.cfg
    cache = w.caches[0]
    L, nq, nkv, d = w.L0, c["nq"], c["nkv"], c["d"]
    scores = H.DeviceArray((nq, L))
    wts = H.DeviceArray((nq, L))
    out = H.DeviceArray((nq, d))
    lib = E.lib()

    def ks():
        for l in range(c["nl"]):
            assert lib.eakv_attention_scores_device(cache.h, w.ql[l].ptr, l, nq, nkv,
                                                    scores.ptr, None) == 0, E.last_error()

    def sm():
        for _ in range(c["nl"]):
            w.synth.softmax(scores.ptr, wts.ptr, nq, L, w.stream)

    def vs():
        for l in range(c["nl"]):
            assert lib.eakv_attention_output_device(cache.h, wts.ptr, l, nq, nkv, out.ptr,
                                                    None) == 0, E.last_error()

    def whole():
        for l in range(c["nl"]):
            assert lib.eakv_attention_scores_device(cache.h, w.ql[l].ptr, l, nq, nkv,
                                                    scores.ptr, None) == 0, E.last_error()
            w.synth.softmax(scores.ptr, wts.ptr, nq, L, w.stream)
            assert lib.eakv_attention_output_device(cache.h, wts.ptr, l, nq, nkv, out.ptr,
                                                    None) == 0, E.last_error()

    res, issue = {}, {}
    for name, fn in (("k_score", ks), ("softmax", sm), ("v_sum", vs), ("step", whole)):
        res[name], issue[name] = timed(H, w.stream, fn, steps, warmup, c["nl"], queued=True)
    res["host_issue_us"] = issue
    res["step_host_issued"] = timed(H, w.stream, whole, steps, warmup, c["nl"])
    for a in (scores, wts, out):
        a.free()
    return res


def fused_call_us(w, steps, warmup):
    """Mean µs of one fused call per layer on the caches as filled (the
    fused alternative to the unfused step)."""
    E, H, c = w.E, w.H, w.cfg

    def run():
        for l in range(c["nl"]):
            assert E.lib().eakv_attention_fused_batch_device(
                w.handles, c["nseq"], l, w.ql[l].ptr, c["nq"], c["nkv"], w.out.ptr,
                None) == 0, E.last_error()
    return timed(H, w.stream, run, steps, warmup, c["nl"], queued=True)[0]


def read_peak(n_bytes, regions=8, reps=3, per_cu=3):
    """Sustained HBM read rate of the synth library's plain streaming read
    kernel over passes of n_bytes: `regions` separate buffers read back to
    back (no pass finds its bytes in the last-level cache), best of `reps`
    rounds; per_cu blocks of 256 threads per CU.  Returns GB/s."""
    from eakv_amd import hipmem as H
    lib = Synth().lib
    lib.eakv_synth_read.restype = C.c_int
    lib.eakv_synth_read.argtypes = [C.c_void_p, C.c_int64, C.c_void_p, C.c_int, C.c_void_p]
    n_bytes = (n_bytes + 15) // 16 * 16
    lib.eakv_synth_cu_count.restype = C.c_int
    blocks = per_cu * (lib.eakv_synth_cu_count() or 256)
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


def floors_bench():
    """The floors a dependent launch sits on: µs per launch of the plain
    streaming read, 32 launches back to back on one stream over separate
    buffers, for pass sizes from one 16-byte load (the launch cost alone) to
    the fused call's, at 2, 3 and 4 blocks of 256 threads per CU."""
    sizes = [16, 22_036_480, 41_975_808, 83_951_616, 167_837_696, 335_806_464]
    res = []
    for n in sizes:
        row = {"bytes": n}
        for per_cu in (2, 3, 4):
            g = read_peak(n, regions=32, reps=4, per_cu=per_cu)
            row[f"us_per_launch_{per_cu}_per_cu"] = round(((n + 15) // 16 * 16) / g / 1e3, 2)
        res.append(row)
    return {"metric": "back-to-back plain streaming read, µs per launch", "unit": "us",
            "n_gpus": 1, "note": "32 separate buffers per round, best of 4 rounds; 16 bytes "
            "measures the cost of a dependent launch itself", "floors": res}


def gbs(nbytes, us):
    return nbytes / (us * 1e-6) / 1e9


def run_config(cid, steps, warmup, ctx=None, with_cpu=True, log=print, grow_steps=64,
               progress=False):
    """Fill, time and (optionally) CPU-baseline one configuration; returns
    (summary dict, workload internals for the headline line).  grow_steps:
    decode steps of the growing-context workload; progress: a line per layer
    of the fill and per timed step (for runs under a profiler)."""
    H = __import__("eakv_amd.hipmem", fromlist=["x"])
    w = Workload(cid, ctx)
    c = w.cfg
    log(f"bench: config {cid} {c['name']}: filling {c['nseq']} x {c['nl']} layers x "
        f"{w.L0} tokens")
    w.fill_context(log, every_layer=progress)
    w.prepare_step_inputs()
    H.synchronize()
    qgbs = w.quant_bytes / w.quant_ms / 1e6
    r = {"workload": c["name"], "layers": c["nl"], "q_heads": c["nq"], "kv_heads": c["nkv"],
         "head_dim": c["d"], "context": w.L0 + (0 if c["path"] == "unfused" else 1),
         "sequences": c["nseq"]}
    extra = {}
    if c["path"] == "unfused":
        u = measure_unfused(w, max(steps, 10), warmup)
        ks_b, sm_b, vs_b = w.unfused_bytes()
        alg = ks_b + sm_b + vs_b
        fz = fused_call_us(w, max(steps, 10), warmup)
        r.update({
            "path": "eakv_attention_scores_device -> row softmax -> eakv_attention_output_device",
            "us_per_layer_step": round(u["step"], 3),
            "gbs": round(gbs(alg, u["step"]), 1), "frac": round(gbs(alg, u["step"]) / HBM_PEAK_GBS, 4),
            "alg_bytes_per_layer_step": alg,
            "kernels_us_per_layer": {k: round(u[k], 3) for k in ("k_score", "softmax", "v_sum")},
            "timing": "device time of calls enqueued behind a hold (run back to back from "
                      "a full queue); host_issued_us_per_layer_step: the same step issued "
                      "from Python onto an idle device",
            "host_issued_us_per_layer_step": round(u["step_host_issued"], 3),
            "host_issue_us_per_call": {k: round(v, 3) for k, v in u["host_issue_us"].items()},
            "k_score_gbs": round(gbs(ks_b, u["k_score"]), 1),
            "v_sum_gbs": round(gbs(vs_b, u["v_sum"]), 1),
            "fused_call_us_per_layer": round(fz, 3),
            "fused_call_gbs": round(gbs(w.fused_bytes(w.L0), fz), 1),
        })
        extra = {"ms_step": u["step"] * c["nl"] / 1e3, "fused_us": u["step"], "alg": alg,
                 "steps": max(steps, 10)}
    else:
        n_steps = grow_steps if c["path"] == "grow" else steps
        ms, fused_us, fused_pct = measure_fused(w, n_steps, warmup, log if progress else None)
        ctx_mid = w.L0 + (n_steps + 1) / 2 if c["path"] == "grow" else w.L0 + 1
        alg = int(w.fused_bytes(ctx_mid))
        r.update({
            "path": "append 1 token x all layers (batched) + eakv_attention_fused_batch_device "
                    "x all layers" + (f", context growing over {n_steps} steps"
                                      if c["path"] == "grow" else ", context restored each step"),
            "steps": n_steps,
            "us_per_layer_step": round(ms * 1e3 / c["nl"], 3),
            "fused_us_per_layer": round(fused_us, 3),
            "fused_us_per_layer_min_median_max_over_steps": fused_pct,
            "gbs": round(gbs(alg, fused_us), 1), "frac": round(gbs(alg, fused_us) / HBM_PEAK_GBS, 4),
            "alg_bytes_per_layer_step": alg,
        })
        extra = {"ms_step": ms, "fused_us": fused_us, "alg": alg, "steps": n_steps}
    r["quantize"] = {"gb_alg": round(w.quant_bytes / 1e9, 2), "ms": round(w.quant_ms, 3),
                     "gbs": round(qgbs, 1), "frac": round(qgbs / HBM_PEAK_GBS, 4)}
    log(f"bench: config {cid}: {r['us_per_layer_step']} us/layer-step, {r['gbs']} GB/s, "
        f"quantize {qgbs:.0f} GB/s")
    w.free()
    H.synchronize()
    if with_cpu:
        log(f"bench: config {cid}: CPU baseline")
        r["cpu"] = cpu_baseline(c, budget_s=8.0 if cid == HEADLINE else 5.0)
        if c["path"] == "grow":
            r["cpu_quantize"] = cpu_quantize_baseline(c)
    return r, extra


def reference_shapes_bench():
    """The reference's own benchmark table (bench_libeakv.c:156-240) at its
    shapes (1 layer 8 heads d128 at 2048 and 8192 tokens; 32 layers at 2048,
    measured on layer 0) with its inputs (ramps (i % 2000)/200 - 5, queries
    0.1) and method (5 warmups, median of 20): the host-pointer
    eakv_attention_scores and eakv_attention_output (PCIe copies and a stream
    wait included), the device-pointer scores, load_raw (2 warmups, median of
    10), its two K-score baselines on the device (dequantize the K plane to
    f32 with eakv_dequantize_range_device, then a plain f32 dot, :76-98; the
    f32 dot on the raw f32 K alone, :110-122) and .eakv save and load (1
    warmup, median of 5, :222-223); beside the reference's published
    single-core K-score times (README.md:34-39)."""
    import eakv_amd as E
    from eakv_amd import hipmem as H
    published = {(1, 2048): 210, (1, 8192): 844, (32, 2048): 213}
    res = []
    for nl, sl in ((1, 2048), (1, 8192), (32, 2048)):
        nh, hd = 8, 128
        data = ((np.arange(nl * 2 * nh * sl * hd, dtype=np.int32) % 2000).astype(np.float32)
                / np.float32(200.0) - np.float32(5.0))
        c = E.Cache(nl, nh, hd, sl)

        def med(fn, warm, runs):
            for _ in range(warm):
                fn()
            t = []
            for _ in range(runs):
                t0 = time.perf_counter()
                fn()
                t.append(time.perf_counter() - t0)
            return float(np.median(t)) * 1e6

        t_load = med(lambda: c.load_raw(data, sl), 2, 10)
        q = np.full((nh, hd), 0.1, np.float32)
        scores = np.empty((nh, sl), np.float32)
        wts = np.full((nh, sl), 1.0 / sl, np.float32)
        out = np.empty((nh, hd), np.float32)
        L = E.lib()
        t_ks = med(lambda: L.eakv_attention_scores(c.h, q.ctypes.data, 0, nh, nh,
                                                   scores.ctypes.data), 5, 20)
        t_vs = med(lambda: L.eakv_attention_output(c.h, wts.ctypes.data, 0, nh, nh,
                                                   out.ctypes.data), 5, 20)
        dq = H.DeviceArray.from_host(q)
        ds = H.DeviceArray((nh, sl))

        def dev():
            assert L.eakv_attention_scores_device(c.h, dq.ptr, 0, nh, nh, ds.ptr, None) == 0
            c.sync()
        t_dev = med(dev, 5, 20)
        # dequant + dot: layer 0's K plane (all heads: the cache's
        # max_seq_len is sl, so the plane is [head][token][dim]) to f32, then
        # the plain dot; and the plain dot on the raw f32 K
        sy = Synth.get()
        n_groups = nh * sl * hd // 64
        kf = H.DeviceArray((nh, sl, hd))
        raw_k = H.DeviceArray.from_host(data[: nh * sl * hd].reshape(nh, sl, hd))

        def deq_dot():
            assert L.eakv_dequantize_range_device(c.h, 0, 0, 0, n_groups, kf.ptr, None) == 0
            sy.dot_scores(kf.ptr, dq.ptr, ds.ptr, nh, sl, hd, c.stream)
            c.sync()

        def f32_dot():
            sy.dot_scores(raw_k.ptr, dq.ptr, ds.ptr, nh, sl, hd, c.stream)
            c.sync()

        t_deq_dot = med(deq_dot, 5, 20)
        t_f32_dot = med(f32_dot, 5, 20)
        path = os.path.join(tempfile.gettempdir(), f"bench_eakv_{os.getpid()}.eakv")
        t_save = med(lambda: c.save(path), 1, 5)
        loaded = []
        t_load_file = med(lambda: loaded.append(E.Cache.load(path)) or loaded.pop().free(), 1, 5)
        file_mb = os.path.getsize(path) / 1e6
        os.unlink(path)
        res.append({"shape": f"{nl} layer(s), 8 heads, d128, {sl} tokens",
                    "published_cpu_k_score_us": published[(nl, sl)],
                    "host_api_k_score_us": round(t_ks, 1), "host_api_v_output_us": round(t_vs, 1),
                    "device_api_k_score_us_with_sync": round(t_dev, 1),
                    "device_dequant_then_dot_us_with_sync": round(t_deq_dot, 1),
                    "device_f32_dot_us_with_sync": round(t_f32_dot, 1),
                    "host_api_load_raw_us": round(t_load, 1),
                    "save_eakv_us": round(t_save, 1), "load_eakv_us": round(t_load_file, 1),
                    "eakv_file_mb": round(file_mb, 2)})
        for a in (dq, ds, kf, raw_k):
            a.free()
        c.free()
    return {"method": "bench_libeakv.c: inputs (i % 2000)/200 - 5, queries 0.1, median of 20 "
                      "after 5 warmups (load_raw: 10 after 2; save and load of the .eakv "
                      "file: 5 after 1), host clock; host_api_* include the H2D copy of the "
                      "inputs, the D2H copy of the results and the wait; device_* are "
                      "device-pointer calls followed by a wait; the load of the file "
                      "includes creating and freeing the cache",
            "shapes": res}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # The first ~10-15 decode steps after the GPU has idled run 3-10% slower
    # (clocks and power settling: 8 x 32Q/8KV at 32767 tokens, 64-67 us per
    # call in steps 2-5, 56.6-57.0 from step 15 on); 40 untimed steps cover
    # that transient, so the timed steps measure the sustained rate.
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--config", type=int, default=None, choices=sorted(CONFIGS),
                    help="only this configuration (its own line as the headline)")
    ap.add_argument("--ctx", type=int, default=None, help="override context length "
                    "(with --config)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--grow-steps", type=int, default=64, choices=range(1, 65),
                    metavar="1..64", help="decode steps of the growing-context workload "
                    "(its definition: 64)")
    ap.add_argument("--progress", action="store_true",
                    help="a line per filled layer and per timed step (runs under a "
                         "profiler, whose counters slow every launch)")
    ap.add_argument("--unfused", action="store_true",
                    help="with --config: only time the unfused K-score and V-sum calls, "
                         "print their JSON line, then exit")
    ap.add_argument("--dequant", action="store_true",
                    help="only time whole-plane dequantization of the first cache of "
                         "--config (default 4), print its JSON line, then exit")
    ap.add_argument("--validate", action="store_true",
                    help="only time the integrity check of the first cache, print its "
                         "JSON line, then exit")
    ap.add_argument("--ggml", action="store_true",
                    help="only time the ggml block type's device functions on 1 GiB of "
                         "f32 rows, print their JSON line, then exit")
    ap.add_argument("--floors", action="store_true",
                    help="only time back-to-back plain reads of the workloads' pass sizes "
                         "(the launch and read floors), print their JSON line, then exit")
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
    if args.floors:
        print(json.dumps(floors_bench()), flush=True)
        return
    log = lambda *a: print(*a, file=sys.stderr, flush=True)
    if args.dequant or args.validate or args.unfused:
        from eakv_amd import hipmem as H
        w = Workload(args.config or HEADLINE, args.ctx)
        w.fill_context(log, every_layer=args.progress)
        w.prepare_step_inputs()
        H.synchronize()
        if args.dequant:
            line = dequant_bench(w, max(1, args.steps // 4), 1)
        elif args.validate:
            line = validate_bench(w, max(3, args.steps), 2)
        else:
            line = unfused_bench(w, max(1, args.steps // 4), 1)
        print(json.dumps(line), flush=True)
        return

    head_id = args.config or HEADLINE
    ids = [args.config] if args.config else sorted(CONFIGS)
    summaries, head = {}, None
    for cid in ids:
        r, extra = run_config(cid, args.steps if cid == head_id else max(5, args.steps // 2),
                              args.warmup, args.ctx if args.config else None,
                              with_cpu=not args.no_cpu, log=log, grow_steps=args.grow_steps,
                              progress=args.progress)
        summaries[str(cid)] = r
        if cid == head_id:
            head = (r, extra)
    r, extra = head
    c = CONFIGS[head_id]
    line = {
        "metric": metric_text(dict(c, L=args.ctx or c["L"])),
        "value": r["us_per_layer_step"], "unit": "us/layer",
        "n_gpus": 1, "steps": extra.get("steps", args.steps), "warmup": args.warmup,
        "ms_per_step": round(extra["ms_step"], 4) if extra else None,
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": DTYPE,
        "data": "synthetic: seeded device generator, distributions of the configuration",
        "config": {k: r[k] for k in ("workload", "layers", "q_heads", "kv_heads", "head_dim",
                                     "context", "sequences", "path")},
    }
    if extra:
        alg = extra["alg"]
        read_gbs = read_peak(alg)
        log(f"bench: plain streaming read of {alg / 1e6:.1f} MB passes: {read_gbs:.0f} GB/s")
        traffic = None
        tfile = os.path.join(ROOT, "profiles", f"fused_config{head_id}_traffic.json")
        if os.path.exists(tfile):
            traffic = json.load(open(tfile)).get("hbm_bytes_per_launch")
        achieved = gbs(alg, extra["fused_us"])
        line.update({
            "fused_us_per_layer": round(extra["fused_us"], 3),
            "achieved_gbs": round(achieved, 1),
            "quantize_gbs": r["quantize"]["gbs"],
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                         "traffic": traffic, "alg_bytes_per_launch": alg,
                         "measured_read_gbs": round(read_gbs, 1),
                         "frac_of_measured_read": round(achieved / read_gbs, 4)},
        })
    line["cpu_baseline"] = r.get("cpu")
    line["configs"] = summaries
    if not args.config:
        log("bench: reference benchmark shapes (host-pointer API)")
        line["reference_shapes"] = reference_shapes_bench()
    print(json.dumps(line), flush=True)


# ------------------------------------------------------ single-purpose modes

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

    us = timed(H, w.stream, one_pass, steps, warmup, len(planes))
    alg = ng * (40 + 256)
    g = gbs(alg, us)
    return {"metric": "plane dequantize to f32 GB/s (40 B read + 256 B written per group)",
            "value": round(g, 1), "unit": "GB/s", "higher_is_better": True,
            "us_per_plane": round(us, 3), "groups_per_plane": ng, "planes_per_step": len(planes),
            "steps": steps, "n_gpus": 1, "dtype": "q4_1 -> f32",
            "config": {"workload": c["name"], "plane": f"{c['nkv']} kv heads x {w.lmax} tokens x d{c['d']}"},
            "roofline": {"bound": "hbm", "achieved": round(g, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(g / HBM_PEAK_GBS, 4),
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
    g = gbs(alg, us)
    return {"metric": "integrity check GB/s (scale + bias read per group, whole host call)",
            "value": round(g, 1), "unit": "GB/s", "higher_is_better": True,
            "us_per_call": round(us, 1), "groups_per_block": n, "blocks": 2 * c["nl"],
            "codes": res.tolist()[:4], "steps": steps, "n_gpus": 1, "dtype": "f32 bit tests",
            "config": {"workload": c["name"]},
            "roofline": {"bound": "hbm", "achieved": round(g, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(g / HBM_PEAK_GBS, 4),
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
        def checked(call=call):
            rc = call()
            if rc:
                raise RuntimeError(E.last_error())
        us = timed(H, None, checked, steps, warmup, 1)
        g = gbs(alg, us)
        res[name] = {"us_per_call": round(us, 2), "gbs": round(g, 1),
                     "frac": round(g / HBM_PEAK_GBS, 4), "alg_bytes_per_call": alg}
    return {"metric": "ggml block type device functions, GB/s of algorithmic bytes",
            "unit": "GB/s", "n_gpus": 1, "steps": steps, "dtype": "block_q4_1_eakv <-> f32",
            "config": {"rows": n_rows, "k": k, "bytes_f32": n * 4}, **res}


def unfused_bench(w, steps, warmup):
    """The reference API's unfused calls on the first cache, every layer
    back to back, each phase timed on its own: K-score, the caller's row
    softmax, V-sum.  Returns the JSON line with each call's mean time and
    GB/s of its algorithmic bytes (K-score n_kv*L*gpd*40 + n_q*L*4 + n_q*d*4,
    softmax 2*n_q*L*4, V-sum n_kv*L*gpd*40 + n_q*L*4 + n_q*d*4)."""
    c = w.cfg
    u = measure_unfused(w, steps, warmup)
    ks_b, sm_b, vs_b = w.unfused_bytes()
    res = {}
    for name, b in (("k_score", ks_b), ("softmax", sm_b), ("v_sum", vs_b)):
        res[name] = {"us_per_call": round(u[name], 3), "gbs": round(gbs(b, u[name]), 1),
                     "frac": round(gbs(b, u[name]) / HBM_PEAK_GBS, 4), "alg_bytes_per_call": b}
    return {"metric": "unfused K-score / softmax / V-sum per layer call, GB/s of algorithmic bytes",
            "unit": "GB/s", "n_gpus": 1, "steps": steps, "dtype": DTYPE,
            "config": {"workload": c["name"], "layers": c["nl"], "q_heads": c["nq"],
                       "kv_heads": c["nkv"], "head_dim": c["d"], "context": w.L0,
                       "sequences": 1},
            "step_us_per_layer": round(u["step"], 3), **res}


if __name__ == "__main__":
    main()
