"""Writes tests/golden/sched_cases.json: the integer inputs that tessel's
scheduler hands the engine, step by step, for a few seeded request sets.

A pure-Python restatement of sched::generate_with (src/llm/sched.rs:52-179),
written from the reference as text (the Rust cannot run here): admission in
arrival order while the batch (:75), the step's token budget (:75) and the
free pages (:76) allow, whole sequences' pages reserved up front from a LIFO
free list (:60, :80), one packed or single prefill step for what was
admitted (:83-104), else one decode step for every running sequence
(:128-149); a sequence leaves at max_new tokens or at eos and returns its
pages to the free list (:116-125, :157-168). The model is replaced by a
script: a step's next token for request r is the next entry of script[r].

Run `python tests/golden/make_sched.py` to rewrite the fixture.
"""

import json
import os
from collections import deque

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "sched_cases.json")


def generate(lim, eos, requests, max_batch, packed, script):
    """lim = (page, pages, max_tokens, max_seq_pages). Returns (steps, tokens)."""
    page, pages, max_tokens, max_seq_pages = lim
    free = list(range(pages))[::-1]
    waiting = deque(range(len(requests)))
    running = []  # [id, pages, len, last, left]
    out = [[] for _ in requests]
    steps = []
    max_batch = min(max_batch, max_tokens)

    def model(ids):
        return [script[i][len(out[i])] for i in ids]

    while waiting or running:
        admit, tokens = [], 0
        while waiting:
            rid = waiting[0]
            prompt, max_new = requests[rid]
            need = -(-(len(prompt) + max_new) // page)
            if not prompt or len(prompt) > max_tokens or need > max_seq_pages:
                raise ValueError(f"request {rid}: prompt of {len(prompt)} tokens does not fit")
            room = len(running) + len(admit) < max_batch and tokens + len(prompt) <= max_tokens
            if not room or need > len(free) or (not packed and admit):
                break
            waiting.popleft()
            tokens += len(prompt)
            admit.append((rid, [free.pop() for _ in range(need)]))
        if admit:
            toks, pos, slots, starts, last = [], [], [], [], []
            for rid, pg in admit:
                s0 = len(toks)
                for i, t in enumerate(requests[rid][0]):
                    toks.append(t)
                    pos.append(i)
                    slots.append(pg[i // page] * page + i % page)
                    starts.append(s0)
                last.append(len(toks) - 1)
            mode = 0 if len(admit) == 1 else 1
            step = {"mode": mode, "tokens": toks, "pos": pos, "slots": slots}
            if mode == 1:
                step["starts"] = starts
            step["want"] = last
            steps.append(step)
            nxt = model([rid for rid, _ in admit])
            for (rid, pg), t in zip(admit, nxt):
                out[rid].append(t)
                s = [rid, pg, len(requests[rid][0]), t, requests[rid][1] - 1]
                if s[4] == 0 or t == eos:
                    free.extend(pg)
                else:
                    running.append(s)
            continue
        if not running:
            continue
        step = {
            "mode": 2,
            "tokens": [s[3] for s in running],
            "pos": [s[2] for s in running],
            "slots": [s[1][s[2] // page] * page + s[2] % page for s in running],
            "tables": [s[1] + [0] * (max_seq_pages - len(s[1])) for s in running],
            "lens": [s[2] + 1 for s in running],
            "want": list(range(len(running))),
        }
        steps.append(step)
        nxt = model([s[0] for s in running])
        keep = []
        for s, t in zip(running, nxt):
            s[2] += 1
            s[3] = t
            s[4] -= 1
            out[s[0]].append(t)
            if s[4] == 0 or t == eos:
                free.extend(s[1])
            else:
                keep.append(s)
        running = keep
    return steps, out


def xorshift(seed):
    """bench::Rng's bits() (src/bench.rs:13-35)."""
    s = (seed * 0x9E3779B97F4A7C15 | 1) & (2**64 - 1)
    while True:
        s ^= (s << 13) & (2**64 - 1)
        s ^= s >> 7
        s ^= (s << 17) & (2**64 - 1)
        yield s


def case(name, seed, lim, eos, nreq, max_batch, packed, plen=(1, 14), mnew=(1, 9), vocab=50):
    r = xorshift(seed)
    rnd = lambda lo, hi: lo + next(r) % (hi - lo + 1)
    requests, script = [], []
    for _ in range(nreq):
        p = [rnd(0, vocab - 1) for _ in range(rnd(*plen))]
        m = rnd(*mnew)
        requests.append((p, m))
        script.append([rnd(0, vocab - 1) for _ in range(m)])
    steps, out = generate(lim, eos, requests, max_batch, packed, script)
    return {"name": name, "limits": list(lim), "eos": eos, "max_batch": max_batch, "packed": packed,
            "requests": [{"prompt": p, "max_new": m} for p, m in requests], "script": script,
            "steps": steps, "tokens": out}


CASES = [
    # (page, pages, max_tokens, max_seq_pages)
    ("packed", 1, (4, 40, 24, 8), 7, 9, 4, True),
    ("single_prefills", 2, (4, 40, 24, 8), 7, 7, 3, False),
    ("tight_pool_lifo_reuse", 3, (4, 9, 16, 6), 3, 10, 8, True),
    ("page_1_eos_early", 4, (1, 40, 12, 24), 1, 8, 5, True, (1, 10), (1, 9), 6),
    ("batch_1", 5, (8, 6, 32, 3), 11, 5, 1, True),
]


def build():
    return [case(*c) for c in CASES]


if __name__ == "__main__":
    with open(FIXTURE, "w") as f:
        json.dump(build(), f, separators=(",", ":"))
    print("wrote", FIXTURE)
