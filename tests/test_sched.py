"""The scheduler's integer stream on the CPU (src/llm/sched.rs:52-179):
tsl_schedule_trace runs tsl_generate's scheduler with a scripted model and
records every step's tokens, positions, slots (:98, :141), starts, block
tables and lens; these must equal, bit for bit, the committed fixtures that
tests/golden/make_sched.py (a pure-Python restatement of sched.rs) wrote.
The fixtures themselves are pinned by invariants that any correct paged
scheduler satisfies, and the request checks (max_new < 1, a request larger
than the pool) by their errors."""

import json
import os

import pytest

import tessel_amd as T

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = json.load(open(os.path.join(HERE, "golden", "sched_cases.json")))


def run(c):
    reqs = [(r["prompt"], r["max_new"]) for r in c["requests"]]
    return T.schedule_trace(T.Limits(*c["limits"]), c["eos"], reqs, c["max_batch"], c["packed"], c["script"])


@pytest.mark.parametrize("c", CASES, ids=[c["name"] for c in CASES])
def test_schedule_matches_the_golden_stream(c):
    steps, toks, st = run(c)
    assert toks == c["tokens"]
    assert len(steps) == len(c["steps"])
    for i, (got, want) in enumerate(zip(steps, c["steps"])):
        assert got == want, f"step {i}"
    assert st.prefill_steps == sum(s["mode"] != 2 for s in c["steps"])
    assert st.decode_steps == sum(s["mode"] == 2 for s in c["steps"])
    assert st.prompt_tokens == sum(len(r["prompt"]) for r in c["requests"])
    assert st.generated == sum(len(t) for t in c["tokens"])
    assert st.largest_batch == max([len(s["tokens"]) for s in c["steps"] if s["mode"] == 2], default=0)


def test_the_python_restatement_rewrites_the_same_fixture():
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_sched", os.path.join(HERE, "golden", "make_sched.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    assert json.loads(json.dumps(m.build())) == CASES


@pytest.mark.parametrize("c", CASES, ids=[c["name"] for c in CASES])
def test_fixture_invariants(c):
    """What pins the fixtures beyond the restatement: every request gets
    max_new tokens unless its script hits eos first; the slots of a step are
    distinct and lie in pages the sequence owns at its position; live
    sequences never share a page; pages come from [0, pages); a sequence's
    next token is fed back as its next decode input; prefills cover whole
    prompts at positions 0..n-1."""
    page, pages, max_tokens, msp = c["limits"]
    eos = c["eos"]
    for r, sc, got in zip(c["requests"], c["script"], c["tokens"]):
        n = next((i + 1 for i, t in enumerate(sc) if t == eos), r["max_new"])
        assert got == sc[:min(n, r["max_new"])]
    last = {}
    for s in c["steps"]:
        n = len(s["tokens"])
        assert len(set(s["slots"])) == n and n <= max_tokens
        assert all(0 <= x < page * pages for x in s["slots"])
        if s["mode"] == 2:
            owned = [set(tb[:-(-(l - 1 + 1) // page)]) for tb, l in zip(s["tables"], s["lens"])]
            for b in range(n):
                assert s["lens"][b] == s["pos"][b] + 1
                assert s["tables"][b][s["pos"][b] // page] * page + s["pos"][b] % page == s["slots"][b]
                for b2 in range(b):
                    assert not (owned[b] & owned[b2])
            assert s["want"] == list(range(n)) and n <= c["max_batch"]
        else:
            starts = s.get("starts", [0] * n)
            seqs = sorted(set(starts))
            assert len(seqs) == len(s["want"]) and (c["packed"] or len(seqs) == 1)
            for k, s0 in enumerate(seqs):
                end = seqs[k + 1] if k + 1 < len(seqs) else n
                assert s["pos"][s0:end] == list(range(end - s0)) and s["want"][k] == end - 1


def test_request_checks():
    lim = T.Limits(4, 8, 16, 8)
    with pytest.raises(RuntimeError, match="max_new must be at least 1"):
        T.schedule_trace(lim, 1, [([1, 2], 0)], 4, True, [[]])
    with pytest.raises(RuntimeError, match="does not fit"):  # 9 pages needed, 8 in the pool
        T.schedule_trace(T.Limits(4, 8, 16, 16), 1, [([1] * 16, 20)], 4, True, [[0] * 20])
    with pytest.raises(RuntimeError, match="does not fit"):
        T.schedule_trace(lim, 1, [([], 2)], 4, True, [[0, 0]])
    steps, toks, _ = T.schedule_trace(lim, 1, [([1, 2], 1)], 4, True, [[5]])
    assert toks == [[5]] and len(steps) == 1


def test_schedule_trace_rejects_null_arguments():
    # With requests present, a null prompts / offsets / max_new / script /
    # output pointer is an argument error (TSL_ERR_ARG), not a host read
    # out of bounds.
    import ctypes

    import numpy as np
    L = T.lib()
    lim = T.Limits(8, 16, 32, 4)
    prompts = np.array([1, 2, 3], np.int32)
    offsets = np.array([0, 3], np.int64)
    max_new = np.array([2], np.int32)
    script = np.array([5, 6], np.int32)
    out = np.zeros(2, np.int32)
    counts = np.zeros(1, np.int32)
    trace = np.zeros(256, np.int32)
    used = ctypes.c_int64(0)
    full = [prompts.ctypes.data, offsets.ctypes.data, max_new.ctypes.data, script.ctypes.data, out.ctypes.data,
            counts.ctypes.data]
    for hole in range(len(full)):
        p = list(full)
        p[hole] = None
        r = L.tsl_schedule_trace(ctypes.byref(lim), -1, 1, p[0], p[1], p[2], 2, 1, p[3], p[4], p[5], None,
                                 trace.ctypes.data, 256, ctypes.byref(used))
        assert r != 0 and b"null" in L.tsl_last_error(), hole
    r = L.tsl_schedule_trace(ctypes.byref(lim), -1, 1, *full[:3], 2, 1, *full[3:], None, trace.ctypes.data, 256,
                             ctypes.byref(used))
    assert r == 0 and out.tolist() == [5, 6]
