"""Benchmark of tessel's kernel hot path on one MI355X.

A step is one launch of the fp16 GEMM 4096x4096x4096 (the headline
workload; A, B ~ N(0,1)/sqrt(K) f16, f32 accumulation, f16 out), inputs
resident in HBM. W untimed warm-up steps, then K steps timed with HIP
events on the library's stream, bracketed by stream synchronisation.
`value` is TFLOP/s (2MNK per step). The same JSON line carries:
  roofline      the GEMM kernel's achieved TFLOP/s against the 2.5 PFLOP/s
                fp16 dense MFMA peak; traffic = HBM bytes per launch from
                the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summaries;
  cpu_baseline  tessel's interpreter semantics (the oracle's C++
                restatement) on a bounded sample of the same GEMM's programs;
  cases         the other benchmark workloads measured the same way: GEMM
                1024^3/2048^3, causal FlashAttention H32 D64 S 512..4096,
                paged GQA decode (GB/s against 8 TB/s), paged_attention (G = H),
                the engine's prefill_attention and its five projections at
                decode (32 rows, GB/s) and prefill (1024 rows, TFLOP/s) sizes,
                RMSNorm and softmax 4096^2, TinyLlama-shape decode tokens/s
                (skip with --no-llm), and calibration probes (the matrix
                cores' sustained rate on random against near-constant f16,
                the streaming-read floor at the engine's kernel sizes).
"""

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_MFMA_F16 = 2500.0  # TFLOP/s, MI355X dense fp16
PEAK_HBM = 8000.0  # GB/s, MI355X HBM3E


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def f16(a):
    return np.ascontiguousarray(a, np.float16)


class Timed:
    """Event-timed launches of one kernel on the library stream."""

    def __init__(self, T, k, args):
        self.T, self.k, self.args = T, k, args

    def warm(self, seconds=0.2, min_launches=3):
        self._warm(seconds, min_launches)

    def _warm(self, seconds, min_launches):
        # At least 200 ms of launches, as src/runtime.rs:295-316 does, so the
        # clocks have ramped up.
        T = self.T
        t0, n = time.perf_counter(), 0
        while n < min_launches or time.perf_counter() - t0 < seconds:
            T.launch(self.k, self.args)
            n += 1
            if n % 8 == 0:
                T.sync()
        T.sync()

    def run(self, iters):
        """Per-launch milliseconds over `iters` back-to-back launches."""
        T = self.T
        T.sync()
        a = T.event_record()
        for _ in range(iters):
            T.launch(self.k, self.args)
        b = T.event_record()
        T.sync()
        return T.event_elapsed(a, b) / iters

    def median(self, iters, reps=5):
        return float(np.median([self.run(iters) for _ in range(reps)]))


def gemm_inputs(T, n, seed):
    rng = np.random.default_rng(seed)
    a = f16(rng.standard_normal((n, n), np.float32) / np.float32(np.sqrt(n)))
    b = f16(rng.standard_normal((n, n), np.float32) / np.float32(np.sqrt(n)))
    return a, b


def gemm_case(T, n, seed=0):
    a, b = gemm_inputs(T, n, seed)
    bufs = [T.tensor(a), T.tensor(b), T.alloc(n * n * 2)]
    k = T.kernel("matmul", "matmul", [[n, n]] * 3)
    return Timed(T, k, bufs), 2.0 * n ** 3, (a, b)


def load_traffic(name):
    """HBM bytes per launch of a kernel, from the committed rocprofv3 PMC
    summaries (profiles/traffic.json), or None."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(p) as f:
            return json.load(f).get(name)
    except (OSError, ValueError):
        return None


def _oracle_gemm_rate(oracle, a, b, threads, budget_s):
    """TFLOP/s of the oracle on whole BM=BN=128 programs of the GEMM, the
    sample doubling until it has run for about budget_s seconds."""
    n = a.shape[0]
    per_prog = 2.0 * 128 * 128 * n
    total = (n // 128) ** 2
    npids, spent, done = threads, 0.0, 0
    c = np.zeros((n, n), np.float16)
    # Each call first widens A and B to f64 (B transposed), a per-call cost
    # of the restatement that a call with no programs measures; it is taken
    # out of every sample so the rate is the programs' own.
    t0 = time.perf_counter()
    oracle.matmul(a, b, 128, 128, 32, 8, threads=threads, first_pid=0, npids=0, C=c)
    setup = time.perf_counter() - t0
    while spent < budget_s and done < total:
        npids = min(npids, total - done)
        t0 = time.perf_counter()
        oracle.matmul(a, b, 128, 128, 32, 8, threads=threads, first_pid=done, npids=npids, C=c)
        spent += max(time.perf_counter() - t0 - setup, 1e-9)
        done += npids
        npids *= 2
    return per_prog * done / spent / 1e12, done, total, spent


def cpu_baseline(a, b, budget_s):
    """tessel's CPU path: the interpreter's semantics (the oracle's C++
    restatement of src/interp.rs: f64 dot products rounded per op, the f32
    accumulator rounded per BK=32 tile) on bounded samples of the same
    workloads, timed on this host. The headline value is the 4096^3 GEMM on
    all the threads used (OpenMP over independent programs); beside it the
    same GEMM on one thread, as interp::run executes programs in sequence
    (src/interp.rs:360-367), and per-program extrapolations of causal
    FlashAttention S=4096 (whole heads) and paged decode config 4 (whole
    sequences), each stated with its sample."""
    import oracle

    nproc = os.cpu_count() or 1
    threads = min(nproc, 16)
    tf, done, total, spent = _oracle_gemm_rate(oracle, a, b, threads, budget_s)
    tf1, done1, _, spent1 = _oracle_gemm_rate(oracle, a, b, 1, budget_s / 2)
    others = [{"case": "matmul 4096^3, one thread", "value": round(tf1, 6), "unit": "TFLOP/s", "cores": 1,
               "sample": f"{done1} of {total} programs, {spent1:.1f} s of program time"}]
    # FlashAttention S=4096 (H 32, D 64): heads are independent programs of
    # equal cost, so whole heads are timed and the rate extrapolates.
    rng = np.random.default_rng(9)
    s, nh = 4096, max(2, threads // 2)
    q, k, v = (f16(rng.standard_normal((nh, s, 64), np.float32)) for _ in range(3))
    t0 = time.perf_counter()
    oracle.flash_attention(q, k, v, 0.125, threads=threads)
    dt = time.perf_counter() - t0
    others.append({"case": "flash_attention H32 S4096 D64 causal", "value": round(2.0 * nh * s * s * 64 / dt / 1e12, 6),
                   "unit": "TFLOP/s", "cores": threads,
                   "sample": f"{nh} of 32 heads in {dt:.2f} s; the full call extrapolates to {dt * 32 / nh:.1f} s"})
    # Paged decode, config 4: the whole call, repeated for about a second,
    # bytes read per second.
    q, kc, vc, table, lens, nb, toks = decode_inputs(2)
    calls, t0 = 0, time.perf_counter()
    while calls == 0 or time.perf_counter() - t0 < 1.0:
        oracle.decode_attention(q, kc, vc, table, lens, float(1.0 / np.sqrt(128.0)), threads=threads)
        calls += 1
    dt = (time.perf_counter() - t0) / calls
    others.append({"case": "decode_attention B64 H32 G8 D128 P16 ctx~U[128,4096]", "value": round(nb / dt / 1e9, 4),
                   "unit": "GB/s", "cores": threads,
                   "sample": f"the whole call ({toks} context tokens), {calls} calls, {dt * 1e3:.1f} ms each"})
    return {"value": round(tf, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port", "nproc": nproc,
            "sample": f"{done} of {total} BM=BN=128 programs of the 4096^3 matmul (oracle, {threads} threads "
                      f"of {nproc}), {spent:.1f} s of program time (the per-call f16->f64 widening of A and B "
                      "excluded)",
            "others": others}


def vendor_gemm(T, sizes=(1024, 2048, 4096, 8192)):
    """hipBLASLt through torch (torch.matmul: A B with B [K, N], the matmul.tl
    layout; F.linear: A B^T with B^T [N, K]) against this library's matmul,
    in the same process, on N(0,1)/sqrt(K) f16 inputs: back-to-back launches
    timed with torch's events (torch's stream) and with the library's."""
    import torch

    def timed(f, n):
        for _ in range(20):
            f()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            f()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n

    out = []
    for n in sizes:
        g = torch.Generator(device="cuda").manual_seed(n)
        a = (torch.randn(n, n, device="cuda", generator=g) / n ** 0.5).half()
        b = (torch.randn(n, n, device="cuda", generator=g) / n ** 0.5).half()
        bt = b.t().contiguous()
        fl = 2.0 * n ** 3
        iters = 200 if n < 8192 else 40
        nn = timed(lambda: torch.matmul(a, b), iters)
        nt = timed(lambda: torch.nn.functional.linear(a, bt), iters)
        t, _, _ = gemm_case(T, n, seed=n)
        t.warm()
        ours = t.median(iters)
        out.append({"case": f"vendor gemm {n}^3", "hipblaslt_nn_tflops": round(fl / nn / 1e9, 1),
                    "hipblaslt_nt_tflops": round(fl / nt / 1e9, 1), "ours_nn_tflops": round(fl / ours / 1e9, 1)})
        del a, b, bt
    return out


def attention_case(T, s, seed=1):
    rng = np.random.default_rng(seed)
    h, d = 32, 64
    q, k, v = (f16(rng.standard_normal((h, s, d), np.float32)) for _ in range(3))
    bufs = [T.tensor(q), T.tensor(k), T.tensor(v), T.alloc(h * s * d * 2), T.F32(0.125)]
    kern = T.kernel("attention", "flash_attention", [[h, s, d]] * 4)
    return Timed(T, kern, bufs), 2.0 * h * s * s * d


def decode_inputs(seed=2, b=64, h=32, g=8, d=128, p=16):
    """The paged GQA decode inputs: lens ~ U[128, 4096], pages by seeded
    permutation into int32 tables, KV pool N(0,1) f16. Returns q, kc, vc,
    table, lens, the bytes a call must move, and the context tokens."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(128, 4097, b).astype(np.int32)
    need = (lens + p - 1) // p
    mp = 256
    npages = int(need.sum())
    perm = rng.permutation(npages).astype(np.int32)
    table = np.zeros((b, mp), np.int32)
    o = 0
    for i in range(b):
        table[i, :need[i]] = perm[o:o + need[i]]
        o += need[i]
    q = f16(rng.standard_normal((b, h, d), np.float32))
    kc = f16(rng.standard_normal((npages, p, g, d), np.float32))
    vc = f16(rng.standard_normal((npages, p, g, d), np.float32))
    nbytes = float(lens.sum()) * g * d * 2 * 2 + b * h * d * 2 * 2 + 4 * b * mp + 4 * b
    return q, kc, vc, table, lens, nbytes, int(lens.sum())


def decode_case(T, seed=2):
    """Paged GQA decode on the GPU: one decode_attention launch per step."""
    q, kc, vc, table, lens, nbytes, toks = decode_inputs(seed)
    b, h, d = q.shape
    bufs = [T.tensor(q), T.tensor(kc), T.tensor(vc), T.tensor(table), T.tensor(lens), T.alloc(q.nbytes),
            T.F32(1.0 / np.sqrt(d))]
    kern = T.kernel("llm", "decode_attention", [q.shape, kc.shape, vc.shape, table.shape, lens.shape, q.shape])
    flops = 4.0 * toks * h * d
    return Timed(T, kern, bufs), nbytes, flops, toks


class RotTimed(Timed):
    """Timed launches that cycle through several argument lists (weight
    copies whose total exceeds the 256 MB last-level cache, so every launch
    streams its weights from HBM, as the engine's 22 layers do)."""

    def __init__(self, T, k, arg_sets):
        super().__init__(T, k, arg_sets[0])
        self.sets, self.i = arg_sets, 0

    def _next(self):
        self.i = (self.i + 1) % len(self.sets)
        return self.sets[self.i]

    def _warm(self, seconds, min_launches):
        T = self.T
        t0, n = time.perf_counter(), 0
        while n < min_launches or time.perf_counter() - t0 < seconds:
            T.launch(self.k, self._next())
            n += 1
            if n % 8 == 0:
                T.sync()
        T.sync()

    def run(self, iters):
        T = self.T
        T.sync()
        a = T.event_record()
        for _ in range(iters):
            T.launch(self.k, self._next())
        b = T.event_record()
        T.sync()
        return T.event_elapsed(a, b) / iters


def rows_case(T, kind):
    """basic.softmax / basic.rmsnorm over 4096^2, cycling through input and
    output copies totalling 512 MB or more, so rows come from HBM and not from
    the 256 MB last-level cache."""
    rng = np.random.default_rng(3)
    r = c = 4096
    if kind == "softmax":
        x = (rng.random((r, c), np.float32) * 8 - 4).astype(np.float32)
        k = T.kernel("basic", "softmax", [[r, c]] * 2, [("BR", 1), ("BC", c)])
        sets = [[T.tensor(x), T.alloc(r * c * 4)] for _ in range(4)]
        return RotTimed(T, k, sets), 8.0 * r * c
    x = f16(rng.random((r, c), np.float32) * 4 - 2)
    w = T.tensor(f16(rng.random(c, np.float32) * 2 - 1))
    k = T.kernel("basic", "rmsnorm", [[r, c], [c], [r, c]], [("BR", 1), ("BC", c)])
    sets = [[T.tensor(x), w, T.alloc(r * c * 2), T.F32(1e-5)] for _ in range(8)]
    return RotTimed(T, k, sets), 4.0 * r * c


def prefill_case(T, seed=4, lens=(512, 512), h=32, g=4, d=64):
    """kernels/llm.tl prefill_attention at the engine's prefill step
    (the engine workload: two 512-token prompts packed into 1024 rows)."""
    rng = np.random.default_rng(seed)
    t = sum(lens)
    q = f16(rng.standard_normal((t, h, d), np.float32))
    k, v = (f16(rng.standard_normal((t, g, d), np.float32)) for _ in range(2))
    starts = np.concatenate([np.full(l, sum(lens[:i]), np.int32) for i, l in enumerate(lens)])
    bufs = [T.tensor(q), T.tensor(k), T.tensor(v), T.tensor(starts), T.alloc(q.nbytes), T.F32(1.0 / np.sqrt(d))]
    kern = T.kernel("llm", "prefill_attention", [q.shape, k.shape, v.shape, starts.shape, q.shape])
    flops = sum(2.0 * h * l * l * d for l in lens)  # the causal half of 4 H L^2 D per prompt
    return Timed(T, kern, bufs), flops


# The TinyLlama projections (the engine workload: dim 2048, QKV 2560, FFN 5632,
# vocab 32000) as the engine runs them: name, K, N.
PROJ = (("linear", 2048, 2560, "qkv"), ("linear_residual", 2048, 2048, "o"), ("gate_up", 2048, 5632, "gate_up"),
        ("linear_residual", 5632, 2048, "down"), ("logits", 2048, 32000, "logits"))


def proj_case(T, name, m, k, n, seed=6):
    """One kernels/llm.tl projection X[m, k] W^T. Returns the timer, its
    flops and the HBM bytes it must move (weights once, X, Y, and R read and
    written for linear_residual). Decode-sized (m <= 64) products cycle
    through weight copies totalling more than 512 MB, so the weights come
    from HBM and not from the last-level cache."""
    rng = np.random.default_rng(seed)
    x = f16(rng.standard_normal((m, k), np.float32))
    ws = [f16(rng.standard_normal((n, k), np.float32) / np.float32(np.sqrt(k)))
          for _ in range(2 if name == "gate_up" else 1)]
    copies = max(1, -(-(512 << 20) // sum(w.nbytes for w in ws))) if m <= 64 else 1
    if name == "linear_residual":
        y = T.tensor(np.zeros((m, n), np.float32))
        ybytes = 8 * m * n
    elif name == "logits":
        y = T.alloc(4 * m * n)
        ybytes = 4 * m * n
    else:
        y = T.alloc(2 * m * n)
        ybytes = 2 * m * n
    xb = T.tensor(x)
    wbs = [[T.tensor(w) for w in ws] for _ in range(copies)]
    kern = T.kernel("llm", name, [x.shape] + [w.shape for w in ws] + [(m, n)])
    flops = 2.0 * m * n * k * len(ws)
    nbytes = 2.0 * n * k * len(ws) + 2.0 * m * k + ybytes
    if copies == 1:
        return Timed(T, kern, [xb] + wbs[0] + [y]), flops, nbytes
    return RotTimed(T, kern, [[xb] + wb + [y] for wb in wbs]), flops, nbytes


def paged_case(T, seed=3, b=16, h=32, d=128, p=16):
    """kernels/attention.tl paged_attention (G = H) with context lengths
    ~ U[128, 4096] and pages by seeded permutation, as decode_case."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(128, 4097, b).astype(np.int32)
    need = (lens + p - 1) // p
    mp = 256
    npages = int(need.sum())
    perm = rng.permutation(npages).astype(np.int32)
    table = np.zeros((b, mp), np.int32)
    o = 0
    for i in range(b):
        table[i, :need[i]] = perm[o:o + need[i]]
        o += need[i]
    q = f16(rng.standard_normal((b, h, d), np.float32))
    kc = f16(rng.standard_normal((npages, p, h, d), np.float32))
    vc = f16(rng.standard_normal((npages, p, h, d), np.float32))
    bufs = [T.tensor(q), T.tensor(kc), T.tensor(vc), T.tensor(table), T.tensor(lens), T.alloc(b * h * d * 2),
            T.F32(1.0 / np.sqrt(d))]
    kern = T.kernel("attention", "paged_attention", [[b, h, d], [npages, p, h, d], [npages, p, h, d], [b, mp], [b],
                                                     [b, h, d]])
    nbytes = float(lens.sum()) * h * d * 2 * 2 + b * h * d * 2 * 2 + 4 * b * mp + 4 * b
    return Timed(T, kern, bufs), nbytes


def llm_case(T, seqs=32, prompt=512, new=128, graphs=True):
    """The engine workload: TinyLlama-1.1B shape, random fp16 weights, 32
    prompts of 512 random ids, 128 greedy steps under continuous batching."""
    cfg = T.Config.tinyllama()
    t0 = time.perf_counter()
    w = T.weights_random(cfg, 7)
    lim = T.Limits(16, seqs * ((prompt + new + 15) // 16) + 64, 1024, (prompt + new + 15) // 16)
    e = T.Engine(cfg, lim, w, graphs=graphs)
    del w
    rng = np.random.default_rng(5)
    reqs = [(rng.integers(3, cfg.vocab, prompt).tolist(), new) for _ in range(seqs)]
    # A short untimed run first: kernel specialisation, tuning, graph capture.
    e.generate([(reqs[0][0][:64], 4)] * 2, seqs)
    setup = time.perf_counter() - t0
    outs, st = e.generate(reqs, seqs)
    # Where a decode step's time goes (untimed runs of the same workload):
    # the GPU span of each step (input upload to last kernel end, by events)
    # under graph replay and under eager launches, and the wall time per
    # step (the difference: the scheduler's host work and the token download).
    split = {}
    if graphs:
        e.step_times(True)
        _, sg = e.generate(reqs, seqs)
        tg = e.step_times(True)["graph"]
        e.set(False, True)
        _, se = e.generate(reqs, seqs)
        te = e.step_times(False)["eager"]
        e.set(True, True)
        us = lambda ms, n: round(1e3 * ms / n, 1) if n else None
        split = {"step_split_us": {
            "graph_gpu_span": us(tg[1], tg[0]), "graph_wall": us(1e3 * sg.decode_seconds, sg.decode_steps),
            "eager_gpu_span": us(te[1], te[0]), "eager_wall": us(1e3 * se.decode_seconds, se.decode_steps),
            "steps": sg.decode_steps}}
    e.close()
    return {"case": "llm_decode", "model": "TinyLlama-1.1B shape (random fp16 weights)", **split,
            "sequences": seqs, "prompt": prompt, "new_tokens": new,
            "generated_tok_s": round(st.generated / st.seconds, 1),
            "decode_tok_s": round(st.decode_tokens / st.decode_seconds, 1) if st.decode_seconds else None,
            "seconds": round(st.seconds, 3), "decode_seconds": round(st.decode_seconds, 3),
            "prefill_steps": st.prefill_steps, "decode_steps": st.decode_steps,
            "largest_batch": st.largest_batch, "setup_s": round(setup, 1)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cases", action="store_true", help="only the headline GEMM")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--llm", action="store_true", help="(default) run the TinyLlama decode case (config 5)")
    ap.add_argument("--no-llm", action="store_true", help="skip the TinyLlama decode case")
    ap.add_argument("--no-graphs", action="store_true",
                    help="TinyLlama case: launch decode steps kernel by kernel (for kernel traces)")
    ap.add_argument("--only", default="", help="comma list of cases: gemm1024,gemm2048,fa512..fa4096,decode,paged,"
                    "prefill,proj,probes,"
                    "rmsnorm,softmax,llm,copy (counter calibration),vendor (hipBLASLt via torch, opt-in); "
                    "'none' for the headline GEMM alone")
    ap.add_argument("--profile", action="store_true",
                    help="few launches, no clock warm-up: for rocprofv3 counter passes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(every kernel here runs on one MI355X; the measured value is one GPU's throughput)", file=sys.stderr)
        sys.exit(2)

    only = set(filter(None, args.only.split(",")))
    if "vendor" in only:
        import torch  # (initialised before the library opens the device: torch enumerates devices once)

        torch.cuda.init()
    import tessel_amd as T

    T.open()
    cus, mhz = T.device_info()
    log("device:", T.device_name(), cus, "CUs", mhz, "MHz")

    # ---- headline: GEMM 4096^3
    if args.profile:
        Timed.warm = lambda self, seconds=0.0, min_launches=2: Timed._warm(self, seconds, min_launches)
        Timed.median = lambda self, iters, reps=1: Timed.run(self, min(iters, 5))
    g, flops, (a, b) = gemm_case(T, 4096)
    g.warm()
    for _ in range(args.warmup):
        T.launch(g.k, g.args)
    T.sync()
    wall0 = time.perf_counter()
    ms = g.run(args.steps)
    wall = time.perf_counter() - wall0
    value = flops / (ms * 1e-3) / 1e12
    kern_ms = ms  # one launch per step: the kernel's average duration over the timed region
    achieved = value
    traffic = load_traffic("matmul_4096")
    line = {
        "metric": "fp16 GEMM/attn TFLOP/s, paged-decode HBM GB/s, % of MI355X roofline",
        "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 5), "wall_s": round(wall, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16 (f32 accumulation)", "data": "synthetic",
        "config": {"workload": "matmul 4096x4096x4096 (kernels/matmul.tl), A,B ~ N(0,1)/sqrt(K) f16",
                   "M": 4096, "N": 4096, "K": 4096, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_MFMA_F16, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_MFMA_F16, 4), "traffic": traffic,
                     "kernel": "gemm_pp16<false, 0> (matmul)", "kernel_ms": round(kern_ms, 5),
                     "algorithmic_per_launch": "2MNK = 137.44 GFLOP"},
        "device": {"name": T.device_name(), "cus": cus, "mhz": mhz},
    }
    cases = []
    if not args.no_cases:
        def want(n):
            return not only or n in only

        for n in (1024, 2048):
            if not want(f"gemm{n}"):
                continue
            t, fl, _ = gemm_case(T, n, seed=n)
            t.warm()
            m = t.median(100)
            cases.append({"case": f"gemm {n}^3", "ms": round(m, 5), "tflops": round(fl / m / 1e9, 2),
                          "frac_mfma": round(fl / m / 1e9 / PEAK_MFMA_F16, 4)})
        for s in (512, 1024, 2048, 4096):
            if not want(f"fa{s}"):
                continue
            t, fl = attention_case(T, s)
            t.warm()
            m = t.median(50)
            cases.append({"case": f"flash_attention H32 S{s} D64 causal", "ms": round(m, 5),
                          "tflops": round(fl / m / 1e9, 2), "frac_mfma": round(fl / m / 1e9 / PEAK_MFMA_F16, 4)})
        if want("decode"):
            t, nb, fl, toks = decode_case(T)
            t.warm()
            m = t.median(50)
            gbs = nb / m / 1e6
            cases.append({"case": "decode_attention B64 H32 G8 D128 P16 ctx~U[128,4096]", "ms": round(m, 5),
                          "gbps": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM, 4), "bytes": nb,
                          "context_tokens": toks, "tflops": round(fl / m / 1e9, 3),
                          "traffic": load_traffic("decode_attention")})
        if want("paged"):
            t, nb = paged_case(T)
            t.warm()
            m = t.median(50)
            cases.append({"case": "paged_attention B16 H32 D128 P16 ctx~U[128,4096]", "ms": round(m, 5),
                          "gbps": round(nb / m / 1e6, 1), "frac_hbm": round(nb / m / 1e6 / PEAK_HBM, 4)})
        if want("prefill"):
            t, fl = prefill_case(T)
            t.warm()
            m = t.median(50)
            cases.append({"case": "prefill_attention T1024 (2 x 512 packed) H32 G4 D64", "ms": round(m, 5),
                          "tflops": round(fl / m / 1e9, 2), "frac_mfma": round(fl / m / 1e9 / PEAK_MFMA_F16, 4)})
        if want("proj"):
            # Decode-sized (32 rows: a weight stream, HBM-bound) and
            # prefill-sized (1024 rows: MFMA-bound) engine projections.
            for name, k, n, label in PROJ:
                for rows in (32, 1024):
                    t, fl, nb = proj_case(T, name, rows, k, n)
                    t.warm()
                    m = t.median(50)
                    c = {"case": f"{label} ({name}) M{rows} N{n} K{k}", "ms": round(m, 5)}
                    if rows == 32:
                        c.update(gbps=round(nb / m / 1e6, 1), frac_hbm=round(nb / m / 1e6 / PEAK_HBM, 4))
                    else:
                        c.update(tflops=round(fl / m / 1e9, 2), frac_mfma=round(fl / m / 1e9 / PEAK_MFMA_F16, 4))
                    cases.append(c)
        if "copy" in only:  # counter calibration (rocprofv3 passes), not a bench line
            n = 32 << 20
            bufs = [T.alloc(4 * n), T.alloc(4 * n), T.alloc(4 * n)]
            t = Timed(T, T.kernel("basic", "add", [[n]] * 3), bufs)
            t.warm()
            m = t.median(20)
            cases.append({"case": "add f32 32Mi (reads 256 MiB, writes 128 MiB)", "ms": round(m, 5),
                          "gbps": round(12.0 * n / m / 1e6, 1)})
        if "vendor" in only:  # the vendor library on the same inputs (opt-in: torch / hipBLASLt), not a bench line
            cases += vendor_gemm(T)
        if want("probes"):
            # Calibration, not bench lines: what the matrix cores sustain on the
            # GEMM's MFMA pattern with random against nearly constant operands
            # (the clock drops under the power limit with random data), and the
            # streaming-read floor at the sizes of the engine's kernels.
            for rnd in (False, True):
                for reads in (False, True):
                    tf = T.probe_mfma(rnd, reads)
                    cases.append({"case": "probe: mfma 32x32x16 f16, " + ("random" if rnd else "near-constant") +
                                  " operands" + (", with the GEMM's LDS operand reads" if reads else ""),
                                  "tflops": round(tf, 1), "frac_mfma": round(tf / PEAK_MFMA_F16, 4)})
            for rnd in (False, True):
                tf = T.probe_mfma16(rnd)
                cases.append({"case": "probe: mfma 16x16x32 f16 (the GEMMs' form), " +
                                      ("random" if rnd else "near-constant") + " operands, registers only",
                              "tflops": round(tf, 1), "frac_mfma": round(tf / PEAK_MFMA_F16, 4)})
            big = T.alloc(1 << 30)
            T.write(big, 0, np.ones(1 << 28, np.float32))
            for mb in (10, 23, 46, 131, 512):
                gbs = T.probe_stream(big, mb << 20)
                cases.append({"case": f"probe: streaming read of {mb} MiB", "us": round((mb << 20) / gbs / 1e3, 2),
                              "gbps": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM, 4)})
            T.free(big)
        for kind in ("rmsnorm", "softmax"):
            if not want(kind):
                continue
            t, nb = rows_case(T, kind)
            t.warm()
            m = t.median(50)
            cases.append({"case": f"{kind} 4096x4096", "ms": round(m, 5), "gbps": round(nb / m / 1e6, 1),
                          "frac_hbm": round(nb / m / 1e6 / PEAK_HBM, 4)})
        if not args.no_llm and want("llm"):
            cases.append(llm_case(T, graphs=not args.no_graphs))
    if cases:
        line["cases"] = cases
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(a, b, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
