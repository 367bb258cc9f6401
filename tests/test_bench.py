"""bench.py's host logic on the CPU: the one-GPU contract and the rotating
timer that keeps decode-sized weights and 4096^2 rows out of the last-level
cache."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in r.stdout + r.stderr


class _FakeLib:
    """Records launches; events are launch counts, so elapsed = launches."""

    def __init__(self):
        self.launched = []

    def launch(self, k, args):
        self.launched.append(args[0])

    def sync(self):
        pass

    def event_record(self):
        return len(self.launched)

    def event_elapsed(self, a, b):
        return float(b - a)


def test_rotating_timer_cycles_through_every_argument_set():
    T = _FakeLib()
    sets = [["w%d" % i] for i in range(5)]
    t = bench.RotTimed(T, "k", sets)
    t.warm(seconds=0.0, min_launches=7)
    assert set(T.launched) == {"w%d" % i for i in range(5)}
    T.launched.clear()
    per = t.run(12)
    assert per == 1.0  # one launch per iteration
    assert len(T.launched) == 12
    # consecutive launches never reuse the set just used
    assert all(a != b for a, b in zip(T.launched, T.launched[1:]))
    counts = [T.launched.count("w%d" % i) for i in range(5)]
    assert max(counts) - min(counts) <= 1
