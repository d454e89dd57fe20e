"""bench.py's host-side contract, on the CPU: one GPU only, and the queued
timing of short calls (the hold launch must outlast the host's issue of the
timed calls, else it is doubled and the run repeated)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


class _FakeEvent:
    def record(self, stream=None):
        pass

    def synchronize(self):
        pass

    def elapsed_ms(self, later):
        return 1.0


class _FakeH:
    Event = _FakeEvent

    @staticmethod
    def synchronize():
        pass


class _FakeSynth:
    def __init__(self):
        self.holds = []

    def hold(self, us, stream=None):
        self.holds.append(us)


@pytest.fixture
def fake_synth(monkeypatch):
    fs = _FakeSynth()
    monkeypatch.setattr(bench.Synth, "get", classmethod(lambda cls: fs))
    return fs


def test_queued_timing_holds_then_times(fake_synth):
    calls = []
    us, issue = bench.timed(_FakeH, None, lambda: calls.append(1), steps=10, warmup=3,
                            per=2, queued=True)
    assert len(calls) == 13                      # 3 warmup + 10 timed
    assert len(fake_synth.holds) == 1 and fake_synth.holds[0] >= 500
    assert us == pytest.approx(1.0 * 1e3 / 20)   # event ms -> us per unit
    assert issue >= 0.0


def test_queued_timing_doubles_a_short_hold(fake_synth, monkeypatch):
    # the host's issue of the timed calls takes ~1 s on the first two tries
    # and nothing after: the hold doubles until it outlasts the issue
    clock = {"t": 0.0, "n": 0}

    def fake_perf_counter():
        return clock["t"]

    def fn():
        clock["n"] += 1
        if clock["n"] > 1 and len(fake_synth.holds) <= 2:
            clock["t"] += 0.1

    monkeypatch.setattr(bench.time, "perf_counter", fake_perf_counter)
    bench.timed(_FakeH, None, fn, steps=10, warmup=1, per=1, queued=True)
    assert len(fake_synth.holds) == 3
    assert fake_synth.holds[1] == 2 * fake_synth.holds[0]
    assert fake_synth.holds[2] == 2 * fake_synth.holds[1]


def test_queued_timing_gives_up_after_four_holds(fake_synth, monkeypatch):
    clock = {"t": 0.0}

    def fn():
        clock["t"] += 1.0                        # every call: a second of host time

    monkeypatch.setattr(bench.time, "perf_counter", lambda: clock["t"])
    with pytest.raises(RuntimeError, match="outlasted"):
        bench.timed(_FakeH, None, fn, steps=4, warmup=0, per=1, queued=True)
    assert len(fake_synth.holds) == 4


def test_grow_steps_bounded_by_the_spare_tokens():
    """The growing-context workload's caches hold 64 spare tokens: --grow-steps
    outside 1..64 is refused before anything runs; --progress is accepted."""
    for bad in ("0", "65"):
        r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--grow-steps", bad],
                           capture_output=True, text=True, timeout=120)
        assert r.returncode == 2 and "grow-steps" in r.stderr, (bad, r.stderr)
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--help"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "--progress" in r.stdout and "--grow-steps" in r.stdout
