"""The tessel command line (src/main.rs) on this library: the `bench`,
`llm` and `llm-tiny` subcommands with the reference's flags and the same
JSON lines, so tools that read tessel's output (its summarize script) read
these unchanged.

    python -m tessel_amd bench [--quick] [--iters 100] [--json OUT] [--tuned FILE]
    python -m tessel_amd llm MODEL_DIR --prompts FILE [--max-new 64] [--batch 16]
        [--page 16] [--pages 1024] [--max-tokens 1024] [--warmup] [--json OUT]
        [--logits OUT] [--no-graphs] [--no-tune] [--no-pack]
    python -m tessel_amd llm-tiny DIR

Differences, all stated in the output or the usage text: the device is
"Hip" (there is no CPU emulator: `--device emu` is refused) and `sm_mhz`
is null (no clock query). The code generators (ir, cuda, metal, pallas)
and `run` (which checks against the interpreter) are not part of this
library.
"""

import json
import math
import os
import sys
import time

import numpy as np

import tessel_amd as T

USAGE = """tessel (tessel_amd): the tessel kernel hot path on MI355X

usage:
  python -m tessel_amd bench [--quick] [--iters 100] [--json OUT] [--tuned FILE]
               (the benchmark suite on the GPU, tuned per case; FILE keeps the
               chosen configurations, so later runs time only those)

  python -m tessel_amd llm MODEL_DIR --prompts FILE [--max-new 64] [--batch 16] [--device hip]
             [--page 16] [--pages 1024] [--max-tokens 1024] [--warmup] [--json OUT]
             [--logits OUT]  (also writes the logits after the first prompt, as JSON)
             [--no-graphs]   (launch every decode step's kernels one by one, not as a HIP graph)
             [--no-tune]     (default matmul tiles instead of tuning them on the GPU)
             [--profile]     (then runs it all once more timing every kernel launch: time by kernel)
             [--no-pack]     (each new prompt in a prefill step of its own, not packed together)
               (greedy generation with the engine of tessel kernels, continuous
               batching over a paged KV cache; MODEL_DIR is a Hugging Face Llama
               checkpoint, FILE a JSON list of token-id lists)
  python -m tessel_amd llm-tiny DIR   (writes a small random Llama checkpoint, for trying llm)"""


class CliError(Exception):
    pass


def flag(args, name):
    """The value after `name` (src/main.rs:44-49 flag)."""
    if name in args:
        i = args.index(name)
        if i + 1 < len(args):
            return args[i + 1]
    return None


def json_str(s):
    return '"' + s.replace("\\", "\\\\").replace('"', '\\"') + '"'


def rust_e(x, prec=None):
    """Rust's `{:e}` (shortest round trip, f32) or `{:.N e}`: no '+' and no
    leading zeros in the exponent."""
    if math.isnan(x):
        return "NaN"
    if math.isinf(x):
        return "inf" if x > 0 else "-inf"
    if prec is None:
        s = np.format_float_scientific(np.float32(x), unique=True, trim="-", exp_digits=1)
    else:
        s = f"{x:.{prec}e}"
    mant, exp = s.split("e")
    return f"{mant}e{int(exp)}"


# ---------------------------------------------------------------- bench (src/bench.rs)

class Case:
    def __init__(self, kind, file, kernel, label, args, flops, bytes_, configs, verify):
        self.kind, self.file, self.kernel, self.label = kind, file, kernel, label
        self.args, self.flops, self.bytes, self.configs, self.verify = args, flops, bytes_, configs, verify


def _rel(err, scale):
    return err / max(scale, 1e-6)


def _gemm(r, m, k, n, quick):
    """src/bench.rs:56-100: C = A B, 256 sampled entries checked."""
    args = [r.tensor("f16", [m, k]), r.tensor("f16", [k, n]), np.zeros((m, n), np.float16)]
    configs = [([("BM", 128), ("BN", 128), ("BK", 32)], 4), ([("BM", 128), ("BN", 128), ("BK", 32)], 8),
               ([("BM", 128), ("BN", 64), ("BK", 32)], 4), ([("BM", 64), ("BN", 128), ("BK", 32)], 4),
               ([("BM", 64), ("BN", 64), ("BK", 32)], 4), ([("BM", 128), ("BN", 256), ("BK", 32)], 8),
               ([("BM", 256), ("BN", 128), ("BK", 32)], 8), ([("BM", 64), ("BN", 64), ("BK", 64)], 4)]
    if quick:
        configs = configs[:2]
    seed = r.bits()

    def verify(a):
        rr = T.Rng(seed)
        A, B, C = (x.astype(np.float64) for x in a[:3])
        err = scale = 0.0
        for _ in range(256):
            i = rr.below(m)
            j = rr.below(n)
            want = float(A[i] @ B[:, j])
            err = max(err, abs(C[i, j] - want))
            scale = max(scale, abs(want))
        return _rel(err, scale)

    return Case("gemm", "matmul", "matmul", f"{m}x{k}x{n}", args, 2.0 * m * k * n, 2.0 * (m * k + k * n + m * n),
                configs, verify)


def _attention(r, h, s, d, quick):
    """src/bench.rs:102-162: causal FlashAttention, 4 sampled query rows."""
    scale = np.float32(1.0 / math.sqrt(d))
    args = [r.tensor("f16", [h, s, d]), r.tensor("f16", [h, s, d]), r.tensor("f16", [h, s, d]),
            np.zeros((h, s, d), np.float16), T.F32(float(scale))]
    configs = [([("BM", 64), ("BN", 64)], 4), ([("BM", 128), ("BN", 64)], 8), ([("BM", 64), ("BN", 32)], 4),
               ([("BM", 128), ("BN", 32)], 8), ([("BM", 32), ("BN", 64)], 2), ([("BM", 128), ("BN", 64)], 4),
               ([("BM", 128), ("BN", 128)], 8)]
    if quick:
        configs = configs[:2]
    seed = r.bits()

    def verify(a):
        rr = T.Rng(seed)
        Q, K, V, O = (x.astype(np.float64) for x in a[:4])
        err = sc = 0.0
        for _ in range(4):
            hh = rr.below(h)
            i = rr.below(s)
            scores = (K[hh, :i + 1] @ Q[hh, i]) * float(scale)
            e = np.exp(scores - scores.max())
            want = (e @ V[hh, :i + 1]) / e.sum()
            err = max(err, float(np.abs(O[hh, i] - want).max()))
            sc = max(sc, float(np.abs(want).max()))
        return _rel(err, sc)

    return Case("attention", "attention", "flash_attention", f"H{h} S{s} D{d} causal", args,
                2.0 * 2.0 * h * s * s * d / 2.0, 2.0 * 4.0 * h * s * d, configs, verify)


def _softmax(r, rows, cols):
    """src/bench.rs:164-197."""
    args = [r.tensor("f32", [rows, cols], 4.0), np.zeros((rows, cols), np.float32)]
    configs = [([("BR", 1), ("BC", cols)], 4), ([("BR", 2), ("BC", cols)], 4), ([("BR", 4), ("BC", cols)], 8)]

    def verify(a):
        X, Y = a[0].astype(np.float64), a[1].astype(np.float64)
        err = 0.0
        for i in range(0, rows, 97):
            x = X[i]
            e = np.exp(x - x.max())
            err = max(err, float(np.abs(Y[i] - e / e.sum()).max()))
        return err

    return Case("softmax", "basic", "softmax", f"{rows}x{cols} f32", args, 0.0, 8.0 * rows * cols, configs, verify)


def _rmsnorm(r, rows, cols):
    """src/bench.rs:199-237."""
    args = [r.tensor("f16", [rows, cols], 2.0), r.tensor("f16", [cols], 1.0), np.zeros((rows, cols), np.float16),
            T.F32(1e-5)]
    configs = [([("BR", 1), ("BC", cols)], 4), ([("BR", 2), ("BC", cols)], 4), ([("BR", 4), ("BC", cols)], 8)]

    def verify(a):
        X, W, Y = (x.astype(np.float64) for x in a[:3])
        err = sc = 0.0
        for i in range(0, rows, 97):
            inv = 1.0 / math.sqrt(float((X[i] ** 2).sum()) / cols + 1e-5)
            want = X[i] * inv * W
            err = max(err, float(np.abs(Y[i] - want).max()))
            sc = max(sc, float(np.abs(want).max()))
        return _rel(err, sc)

    return Case("rmsnorm", "basic", "rmsnorm", f"{rows}x{cols} f16", args, 0.0, 4.0 * rows * cols, configs, verify)


def suite(quick):
    """src/bench.rs:239-253: the cases, inputs from Rng::new(7) in order."""
    r = T.Rng(7)
    cases = [_gemm(r, n, n, n, quick) for n in ([1024] if quick else [1024, 2048, 4096])]
    cases += [_attention(r, 32, s, 64, quick) for s in ([1024] if quick else [512, 1024, 2048, 4096])]
    cases += [_softmax(r, 4096, 4096), _rmsnorm(r, 4096, 4096)]
    return cases


def config_name(meta, warps):
    """Rust's `format!("{meta:?} warps {warps}")` of a [(&str, i64)] list."""
    return "[" + ", ".join(f'("{k}", {v})' for k, v in meta) + f"] warps {warps}"


def _upload(args):
    return [a if isinstance(a, (T.F32, T.I32)) else T.tensor(np.ascontiguousarray(a)) for a in args]


def _free(bufs):
    for b in bufs:
        if isinstance(b, T.Buf):
            T.free(b)


def time_kernel(k, bufs, iters):
    """Compiled::time (src/runtime.rs:294-316): >= 200 ms (and 3) warm-up
    launches, then the median and minimum ms of `iters` launches, each timed
    on its own with events."""
    t0 = time.perf_counter()
    n = 0
    while n < 3 or time.perf_counter() - t0 < 0.2:
        T.launch(k, bufs)
        n += 1
        if n % 8 == 0:
            T.sync()
    T.sync()
    ts = sorted(T.time_each(k, bufs, iters))
    return ts[len(ts) // 2], ts[0]


def warm_up():
    """src/bench.rs:262-290: ~1.5 s of 2048^2 matmuls, so timings start at
    the sustained clock."""
    n = 2048
    r = T.Rng(1)
    k = T.kernel("matmul", "matmul", [[n, n]] * 3)
    bufs = _upload([r.tensor("f16", [n, n]), r.tensor("f16", [n, n]), np.zeros((n, n), np.float16)])
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 1.5:
        for _ in range(20):
            T.launch(k, bufs)
        T.sync()
    _free(bufs)


# Meta values the launchers read (rows.hip / gemm.hip: the column chunk of
# the row kernels). Tiles, stages and wavefronts are chosen from the shape, so
# BM/BN/BK/BR and the warp count enter only a kernel's cache key.
CODE_META = ("BC",)


def distinct_configs(configs):
    """The candidates of a case that run different code: one per distinct
    value of the meta the launchers read (CODE_META), the first of each."""
    seen, keep = set(), []
    for meta, warps in configs:
        code = tuple((k, v) for k, v in meta if k in CODE_META)
        if code not in seen:
            seen.add(code)
            keep.append((meta, warps))
    return keep


def bench(quick, iters, tuned, out):
    """bench::run (src/bench.rs:292-407): tunes (or takes the configuration
    tuned before, from `tuned`) and times every case; one JSON line each.
    The reference times every tile configuration; here the tiles follow from
    the shape, so only candidates that run different code (distinct_configs)
    are timed, and the line says so ("tiles": "by shape")."""
    T.open()
    device = T.device_name()
    cache = {}
    if tuned and os.path.exists(tuned):
        for line in open(tuned):
            if "\t" in line:
                key, val = line.rstrip("\n").split("\t", 1)
                cache[key] = val
    warm_up()
    for case in suite(quick):
        shapes = [list(a.shape) for a in case.args if isinstance(a, np.ndarray)]
        key = f"{device}|{case.kind}|{case.label}"
        chosen = cache.get(key)
        tried = []
        best = None
        bufs = None
        for meta, warps in distinct_configs(case.configs):
            name = config_name(meta, warps)
            if chosen is not None and chosen != name:
                continue
            try:
                k = T.kernel(case.file, case.kernel, shapes, meta=meta, warps=warps)
            except T.TesselError as e:
                tried.append(f'{{"config": {json_str(name)}, "error": {json_str(str(e).splitlines()[0])}}}')
                continue
            if bufs is None:
                bufs = _upload(case.args)
            med, mn = time_kernel(k, bufs, 30)
            tried.append(f'{{"config": {json_str(name)}, "median_ms": {med:.4f}, "min_ms": {mn:.4f}}}')
            if best is None or mn < best[0]:
                best = (mn, k, name)
        if best is None:
            out(f'{{"kind": {json_str(case.kind)}, "label": {json_str(case.label)}, "engine": "tessel", '
                f'"error": "no configuration compiled", "tried": [{", ".join(tried)}]}}')
            continue
        _, k, name = best
        if chosen is None and tuned:
            with open(tuned, "a") as f:
                f.write(f"{key}\t{name}\n")
        med, mn = time_kernel(k, bufs, iters)
        _free(bufs)
        # One more launch on fresh inputs, checked against the CPU.
        fresh = _upload(case.args)
        T.launch(k, fresh)
        got = [T.read_array(b, a.dtype, a.shape) if isinstance(a, np.ndarray) else a
               for a, b in zip(case.args, fresh)]
        _free(fresh)
        err = case.verify(got)
        tflops = case.flops / (med * 1e-3) / 1e12 if case.flops > 0 else 0.0
        gbps = case.bytes / (med * 1e-3) / 1e9
        out(f'{{"kind": {json_str(case.kind)}, "label": {json_str(case.label)}, "engine": "tessel", '
            f'"device": {json_str(device)}, "median_ms": {med:.4f}, "min_ms": {mn:.4f}, "tflops": {tflops:.3f}, '
            f'"gbps": {gbps:.1f}, "rel_err": {rust_e(err, 3)}, "sm_mhz": null, "config": {json_str(name)}, '
            f'"tiles": "by shape", "tried": [{", ".join(tried)}]}}')


# ---------------------------------------------------------------- llm (src/main.rs:199-318)

def llm(args):
    if len(args) < 3:
        raise CliError(USAGE)
    model = args[2]

    def num(k, d):
        v = flag(args, k)
        if v is None:
            return d
        try:
            return int(v)
        except ValueError:
            raise CliError(f"bad {k}") from None

    dev = flag(args, "--device") or "hip"
    if dev not in ("hip", "cuda"):
        raise CliError(f"unknown device {dev}" + (" (this library has no CPU emulator)" if dev == "emu" else ""))
    path = flag(args, "--prompts")
    if path is None:
        raise CliError("--prompts is required")
    try:
        text = open(path).read()
    except OSError as e:
        raise CliError(f"{path}: {e.strerror}") from None
    ps = json.loads(T.json_roundtrip(text))
    if not isinstance(ps, list):
        raise CliError(f"{path}: not a JSON list")
    max_new = num("--max-new", 64)
    if max_new < 1:
        raise CliError("--max-new must be at least 1")
    reqs = []
    for p in ps:
        if not isinstance(p, list):
            raise CliError(f"{path}: each prompt is a list of token ids")
        reqs.append(([int(x) if isinstance(x, (int, float)) else 0 for x in p], max_new))
    t0 = time.perf_counter()
    cfg, weights = T.load_checkpoint(model)
    load_s = time.perf_counter() - t0
    T.open()
    page = num("--page", 16)
    lim = T.Limits(page, num("--pages", 1024), num("--max-tokens", 1024), max(cfg.max_pos // page, 1))
    t0 = time.perf_counter()
    graphs = "--no-graphs" not in args
    e = T.Engine(cfg, lim, weights, graphs=graphs, tune="--no-tune" not in args)
    del weights
    upload_s = time.perf_counter() - t0
    batch = num("--batch", 16)
    pack = "--no-pack" not in args
    try:
        lp = flag(args, "--logits")
        if lp is not None:
            pr = reqs[0][0]
            n = len(pr)
            pos = list(range(n))
            lg = e.step(pr, pos, pos, mode=0, want=[n - 1])[0]
            with open(lp, "w") as f:
                f.write("[" + ", ".join(rust_e(float(x)) for x in lg) + "]\n")
        warm_s = 0.0
        if "--warmup" in args:  # the same work once, so the timed run finds every kernel specialised
            t0 = time.perf_counter()
            e.generate(reqs, batch, pack)
            warm_s = time.perf_counter() - t0
        outs, st = e.generate(reqs, batch, pack)
        ttft = e.first_token_s
        # The same work once more with every launch timed on its own (and
        # without graphs), after the timed run so it does not change it.
        prof = ""
        if "--profile" in args:
            e.profile(True)
            e.generate(reqs, batch, pack)
            rows = e.profile_rows()
            e.profile(False)
            total = sum(ms for ph, _, _, ms in rows if ph == "decode")
            print(f"decode, kernel time by kernel ({total:.1f} ms in all, launched one at a time):", file=sys.stderr)
            items = []
            for ph, kn, n, ms in rows:
                if ph == "decode":
                    print(f"  {100.0 * ms / max(total, 1e-9):>5.1f}%  {ms:>9.2f} ms  {n:>6}x  {kn}", file=sys.stderr)
                items.append(f'{{"phase": "{ph}", "kernel": "{kn.replace(chr(34), chr(39))}", "launches": {n}, '
                             f'"ms": {ms:.3f}}}')
            prof = ', "profile": [' + ", ".join(items) + "]"
    finally:
        e.close()
    ids = ", ".join("[" + ", ".join(str(t) for t in o) + "]" for o in outs)
    line = (f'{{"engine": "tessel", "device": "Hip", "requests": {len(reqs)}, "batch": {batch}, '
            f'"max_new": {max_new}, "prompt_tokens": {st.prompt_tokens}, "generated": {st.generated}, '
            f'"seconds": {st.seconds:.4f}, "tokens_per_s": {st.generated / st.seconds:.2f}, '
            f'"decode_steps": {st.decode_steps}, "decode_seconds": {st.decode_seconds:.4f}, '
            f'"decode_tokens_per_s": {st.decode_tokens / max(st.decode_seconds, 1e-9):.2f}, '
            f'"largest_batch": {st.largest_batch}, "graphs": {"true" if graphs else "false"}, '
            f'"packed": {"true" if pack else "false"}, "load_s": {load_s:.2f}, "upload_s": {upload_s:.2f}, '
            f'"warmup_s": {warm_s:.2f}, "first_token_s": [{", ".join(f"{x:.4f}" for x in ttft)}], '
            f'"outputs": [{ids}]{prof}}}')
    print(line, flush=True)
    jp = flag(args, "--json")
    if jp is not None:
        with open(jp, "w") as f:
            f.write(line + "\n")


def llm_tiny(args):
    if len(args) < 3:
        raise CliError(USAGE)
    d = args[2]
    os.makedirs(d, exist_ok=True)
    cfg = T.Config.tiny()
    T.save_checkpoint(d, cfg, T.weights_random(cfg, 1))
    print(f"wrote a tiny random Llama to {d}")


def main(argv=None):
    args = ["tessel"] + list(sys.argv[1:] if argv is None else argv)
    cmd = args[1] if len(args) > 1 else ""
    try:
        if cmd == "bench":
            iters = flag(args, "--iters")
            try:
                iters = int(iters) if iters is not None else 100
            except ValueError:
                iters = 100
            jp = flag(args, "--json")

            def out(line):
                print(line, flush=True)
                if jp is not None:
                    with open(jp, "a") as f:
                        f.write(line + "\n")

            bench("--quick" in args, iters, flag(args, "--tuned"), out)
        elif cmd == "llm":
            llm(args)
        elif cmd == "llm-tiny":
            llm_tiny(args)
        else:
            print(USAGE)
            return 0
    except (CliError, T.TesselError) as e:
        print(f"tessel: {e}", file=sys.stderr)
        return 1
    return 0
