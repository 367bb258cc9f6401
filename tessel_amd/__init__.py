"""tessel_amd: tessel's kernel hot path on MI355X (gfx950).

The kernels and their launch surface live in the native library
tessel_amd/libtessel_hip.so (C ABI: include/tessel.h). This module is the
host-side mirror of tessel's src/gpu.rs (Gpu: buffers, kernels keyed by
file/name/shapes/meta/warps, launches with Arg::{Buf,F32,I32}, graph
capture/replay) and of the engine entry points, over ctypes. There is no
fallback: without the library every call raises.
"""

import ctypes
import json
import os
import struct

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# TSL_LIB selects another build of the same library (the sanitized host
# build of `python tessel_amd/build.py --sanitize`).
LIB_PATH = os.environ.get("TSL_LIB") or os.path.join(_HERE, "libtessel_hip.so")
_lib = None


class TesselError(RuntimeError):
    pass


def lib():
    """The loaded native library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise TesselError(f"{LIB_PATH} is missing: build it with `python tessel_amd/build.py` "
                              "(or __graft_entry__.build())")
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_U64 = ctypes.c_uint64
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_P = ctypes.c_void_p

EXPORTS = [
    "tsl_last_error", "tsl_open", "tsl_device_name", "tsl_device_info", "tsl_sync", "tsl_stream", "tsl_alloc",
    "tsl_free", "tsl_upload", "tsl_download", "tsl_fill_nan", "tsl_kernel", "tsl_kernel_key", "tsl_launch",
    "tsl_time_launches", "tsl_capture_begin", "tsl_capture_end", "tsl_replay", "tsl_event_record",
    "tsl_event_elapsed", "tsl_weights_sizes", "tsl_weights_random", "tsl_engine_new", "tsl_engine_free",
    "tsl_engine_set", "tsl_engine_step", "tsl_generate", "tsl_checkpoint_config", "tsl_checkpoint_load",
    "tsl_checkpoint_save", "tsl_json_roundtrip", "tsl_rng_new", "tsl_rng_bits", "tsl_rng_tensor",
    "tsl_time_each", "tsl_engine_profile", "tsl_engine_profile_rows", "tsl_schedule_trace",
    "tsl_graph_nodes", "tsl_engine_graphs", "tsl_engine_fallbacks", "tsl_engine_step_times", "tsl_probe_mfma", "tsl_probe_mfma16", "tsl_probe_stream",
    "tsl_decode_attention_noalloc",
]


class Config(ctypes.Structure):
    """tsl_config: src/llm/mod.rs:15-28."""

    _fields_ = [(n, ctypes.c_int32) for n in ("dim", "layers", "heads", "kv_heads", "head_dim", "ffn", "vocab")] + [
        ("eps", ctypes.c_float), ("rope_theta", ctypes.c_float),
        ("max_pos", ctypes.c_int32), ("bos", ctypes.c_int32), ("eos", ctypes.c_int32)]

    @staticmethod
    def tiny():
        """Config::tiny (src/llm/mod.rs:37-52)."""
        return Config(64, 2, 4, 2, 16, 128, 256, 1e-5, 10000.0, 256, 1, 2)

    @staticmethod
    def tinyllama():
        """TinyLlama-1.1B's shape (random weights; no checkpoint)."""
        return Config(2048, 22, 32, 4, 64, 5632, 32000, 1e-5, 10000.0, 2048, 1, 2)

    def qkv(self):
        return (self.heads + 2 * self.kv_heads) * self.head_dim


class Limits(ctypes.Structure):
    """tsl_limits: src/llm/engine.rs:23-32."""

    _fields_ = [(n, ctypes.c_int32) for n in ("page", "pages", "max_tokens", "max_seq_pages")]


class Stats(ctypes.Structure):
    """tsl_stats: src/llm/sched.rs:22-33."""

    _fields_ = [(n, ctypes.c_int64) for n in ("prefill_steps", "decode_steps", "prompt_tokens", "generated",
                                             "largest_batch", "decode_tokens")] + [
        ("seconds", ctypes.c_double), ("decode_seconds", ctypes.c_double)]


def _declare(L):
    L.tsl_last_error.restype = ctypes.c_char_p
    L.tsl_device_name.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
    L.tsl_device_info.argtypes = [ctypes.POINTER(_INT), ctypes.POINTER(_INT)]
    L.tsl_stream.restype = _P
    L.tsl_alloc.argtypes = [ctypes.c_size_t, ctypes.POINTER(_U64)]
    L.tsl_free.argtypes = [_U64]
    L.tsl_upload.argtypes = [_U64, _P, ctypes.c_size_t]
    L.tsl_download.argtypes = [_P, _U64, ctypes.c_size_t]
    L.tsl_fill_nan.argtypes = [_U64, ctypes.c_size_t]
    L.tsl_kernel.argtypes = [ctypes.c_char_p, ctypes.c_char_p, _INT, ctypes.POINTER(_INT), ctypes.POINTER(_I64), _INT,
                             ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_I64), _INT, ctypes.POINTER(_INT)]
    L.tsl_kernel_key.argtypes = [_INT, ctypes.c_char_p, ctypes.c_size_t]
    L.tsl_launch.argtypes = [_INT, ctypes.POINTER(_U64), _INT]
    L.tsl_time_launches.argtypes = [_INT, ctypes.POINTER(_U64), _INT, _INT, ctypes.POINTER(ctypes.c_float)]
    L.tsl_capture_end.argtypes = [ctypes.POINTER(_INT)]
    L.tsl_replay.argtypes = [_INT]
    L.tsl_event_record.argtypes = [ctypes.POINTER(_INT)]
    L.tsl_event_elapsed.argtypes = [_INT, _INT, ctypes.POINTER(ctypes.c_float)]
    L.tsl_weights_sizes.argtypes = [ctypes.POINTER(Config)] + [ctypes.POINTER(ctypes.c_size_t)] * 4
    L.tsl_weights_random.argtypes = [ctypes.POINTER(Config), _U64, _P, _P, _P, _P]
    L.tsl_engine_new.argtypes = [ctypes.POINTER(Config), ctypes.POINTER(Limits), _P, _P, _P, _P, ctypes.POINTER(_INT)]
    L.tsl_engine_free.argtypes = [_INT]
    L.tsl_engine_set.argtypes = [_INT, _INT, _INT]
    L.tsl_engine_step.argtypes = [_INT, _INT, _P, _P, _P, _INT, _P, _INT, _P, _P, _INT, _P, _P]
    L.tsl_generate.argtypes = [_INT, _INT, _P, _P, _P, _INT, _INT, _P, _P, ctypes.POINTER(Stats), _P]
    L.tsl_graph_nodes.argtypes = [_INT, _P]
    L.tsl_probe_mfma.argtypes = [_INT, _INT, _INT, ctypes.POINTER(ctypes.c_double)]
    L.tsl_probe_mfma16.argtypes = [_INT, _INT, ctypes.POINTER(ctypes.c_double)]
    L.tsl_probe_stream.argtypes = [_U64, ctypes.c_size_t, ctypes.c_size_t, _INT, ctypes.POINTER(ctypes.c_double)]
    L.tsl_engine_graphs.argtypes = [_INT, _P, _P, _INT, ctypes.POINTER(_INT)]
    L.tsl_engine_fallbacks.argtypes = [_INT, ctypes.POINTER(_I64)]
    L.tsl_engine_step_times.argtypes = [_INT, _INT, _P, _P]
    L.tsl_decode_attention_noalloc.argtypes = [_U64] * 6 + [ctypes.c_float] + [_INT] * 7
    L.tsl_schedule_trace.argtypes = [ctypes.POINTER(Limits), _INT, _INT, _P, _P, _P, _INT, _INT, _P, _P, _P,
                                     ctypes.POINTER(Stats), _P, _I64, ctypes.POINTER(_I64)]
    L.tsl_checkpoint_config.argtypes = [ctypes.c_char_p, ctypes.POINTER(Config)]
    L.tsl_checkpoint_load.argtypes = [ctypes.c_char_p, ctypes.POINTER(Config), _P, _P, _P, _P, ctypes.POINTER(_INT)]
    L.tsl_checkpoint_save.argtypes = [ctypes.c_char_p, ctypes.POINTER(Config), _P, _P, _P, _P]
    L.tsl_json_roundtrip.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]
    L.tsl_engine_profile.argtypes = [_INT, _INT]
    L.tsl_engine_profile_rows.argtypes = [_INT, ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]
    L.tsl_time_each.argtypes = [_INT, ctypes.POINTER(_U64), _INT, _INT, _P]
    L.tsl_rng_new.argtypes = [_U64, ctypes.POINTER(_U64)]
    L.tsl_rng_bits.argtypes = [ctypes.POINTER(_U64), ctypes.POINTER(_U64)]
    L.tsl_rng_tensor.argtypes = [ctypes.POINTER(_U64), ctypes.c_size_t, ctypes.c_float, _INT, _P]


def check(rc):
    if rc != 0:
        raise TesselError(lib().tsl_last_error().decode())


def open():  # noqa: A001 - mirrors runtime::cuda() / Cuda::open
    check(lib().tsl_open())


def device_name():
    buf = ctypes.create_string_buffer(256)
    check(lib().tsl_device_name(buf, 256))
    return buf.value.decode()


def device_info():
    cus, mhz = _INT(), _INT()
    check(lib().tsl_device_info(ctypes.byref(cus), ctypes.byref(mhz)))
    return cus.value, mhz.value


# ---------------------------------------------------------------- src/gpu.rs

class Buf:
    """A device buffer: its address and size in bytes (src/gpu.rs:15-18)."""

    __slots__ = ("ptr", "bytes")

    def __init__(self, ptr, nbytes):
        self.ptr = ptr
        self.bytes = nbytes

    def __repr__(self):
        return f"Buf(0x{self.ptr:x}, {self.bytes})"


class F32:
    """An f32 scalar argument (Arg::F32)."""

    def __init__(self, x):
        self.bits = struct.unpack("<I", struct.pack("<f", float(x)))[0]


class I32:
    """An i32 scalar argument (Arg::I32)."""

    def __init__(self, x):
        self.bits = int(x) & 0xFFFFFFFF


def _raw(args):
    raw = (_U64 * max(len(args), 1))()
    for i, a in enumerate(args):
        if isinstance(a, Buf):
            raw[i] = a.ptr
        elif isinstance(a, (F32, I32)):
            raw[i] = a.bits
        else:
            raise TypeError(f"argument {i}: {a!r} is not a Buf, F32 or I32")
    return raw


class Kernel:
    __slots__ = ("handle", "name")

    def __init__(self, handle, name):
        self.handle = handle
        self.name = name

    @property
    def key(self):
        buf = ctypes.create_string_buffer(4096)
        check(lib().tsl_kernel_key(self.handle, buf, 4096))
        return buf.value.decode()


def kernel(file, name, shapes, meta=(), warps=4):
    """Gpu::kernel (src/gpu.rs:148-172): `name` of `file` for these array
    shapes and meta overrides, specialised once and then reused."""
    shapes = [list(map(int, s)) for s in shapes]
    ranks = (_INT * max(len(shapes), 1))(*[len(s) for s in shapes])
    flat = [d for s in shapes for d in s]
    dims = (_I64 * max(len(flat), 1))(*flat)
    names = (ctypes.c_char_p * max(len(meta), 1))(*[m[0].encode() for m in meta])
    vals = (_I64 * max(len(meta), 1))(*[int(m[1]) for m in meta])
    h = _INT()
    check(lib().tsl_kernel(file.encode(), name.encode(), len(shapes), ranks, dims, len(meta), names, vals, int(warps),
                           ctypes.byref(h)))
    return Kernel(h.value, name)


def launch(k, args):
    """Gpu::launch (src/gpu.rs:179-216): asynchronous, on the library's stream."""
    check(lib().tsl_launch(k.handle, _raw(args), len(args)))


def time_launches(k, args, iters):
    """Milliseconds (total) of `iters` event-timed launches."""
    ms = ctypes.c_float()
    check(lib().tsl_time_launches(k.handle, _raw(args), len(args), int(iters), ctypes.byref(ms)))
    return ms.value


def time_each(k, args, iters):
    """Milliseconds of each of `iters` launches, each timed on its own."""
    raw = _raw(args)
    ms = np.zeros(max(iters, 1), np.float32)
    check(lib().tsl_time_each(k.handle, raw, len(args), iters, ms.ctypes.data))
    return ms[:iters].tolist()


def sync():
    check(lib().tsl_sync())


def alloc(nbytes):
    p = _U64()
    check(lib().tsl_alloc(int(nbytes), ctypes.byref(p)))
    return Buf(p.value, int(nbytes))


def free(buf):
    check(lib().tsl_free(buf.ptr))


def write(buf, offset, data):
    """Gpu::write (src/gpu.rs:88-107): bounds-checked, synchronous."""
    data = np.ascontiguousarray(data)
    n = data.nbytes
    if offset + n > buf.bytes:
        raise TesselError(f"write of {n} bytes at {offset} into a buffer of {buf.bytes}")
    check(lib().tsl_upload(buf.ptr + offset, data.ctypes.data, n))


def read(buf, offset, nbytes):
    """Gpu::read (src/gpu.rs:110-133): waits for the GPU, bounds-checked."""
    if offset + nbytes > buf.bytes:
        raise TesselError(f"read of {nbytes} bytes at {offset} from a buffer of {buf.bytes}")
    out = np.empty(nbytes, np.uint8)
    check(lib().tsl_download(out.ctypes.data, buf.ptr + offset, nbytes))
    return out


def tensor(a):
    """A device copy of numpy array `a` (Gpu::tensor, src/gpu.rs:257-262)."""
    a = np.ascontiguousarray(a)
    b = alloc(max(a.nbytes, 4))
    if a.nbytes:
        write(b, 0, a)
    return b


def read_array(buf, dtype, shape):
    dtype = np.dtype(dtype)
    n = int(np.prod(shape)) * dtype.itemsize
    return read(buf, 0, n).view(dtype).reshape(shape)


def fill_nan(buf):
    check(lib().tsl_fill_nan(buf.ptr, buf.bytes // 4))


def capture_begin():
    check(lib().tsl_capture_begin())


def capture_end():
    g = _INT()
    check(lib().tsl_capture_end(ctypes.byref(g)))
    return g.value


def replay(g):
    check(lib().tsl_replay(int(g)))


def graph_nodes(g):
    """Node counts of recorded graph g by type: kernel, memset, memcpy, other."""
    c = np.zeros(4, np.int64)
    check(lib().tsl_graph_nodes(int(g), c.ctypes.data))
    return dict(zip(("kernel", "memset", "memcpy", "other"), c.tolist()))


def probe_mfma(random, lds_reads, iters=2000):
    """TFLOP/s the matrix cores sustain on the GEMM's MFMA pattern (a
    calibration probe: random or nearly constant f16 operands, with or
    without the GEMM's LDS operand reads)."""
    v = ctypes.c_double()
    check(lib().tsl_probe_mfma(int(random), int(lds_reads), int(iters), ctypes.byref(v)))
    return v.value


def probe_mfma16(random, iters=2000):
    """TFLOP/s the matrix cores sustain on v_mfma_f32_16x16x32_f16 from
    registers (the GEMMs' MFMA form), random or nearly constant f16 operands."""
    v = ctypes.c_double()
    check(lib().tsl_probe_mfma16(int(random), int(iters), ctypes.byref(v)))
    return v.value


def probe_stream(buf, nbytes, iters=40):
    """GB/s of back-to-back streaming reads of nbytes each, cycling through
    the windows of device buffer buf."""
    v = ctypes.c_double()
    check(lib().tsl_probe_stream(buf.ptr, buf.bytes, int(nbytes), int(iters), ctypes.byref(v)))
    return v.value


def event_record():
    e = _INT()
    check(lib().tsl_event_record(ctypes.byref(e)))
    return e.value


def event_elapsed(a, b):
    ms = ctypes.c_float()
    check(lib().tsl_event_elapsed(a, b, ctypes.byref(ms)))
    return ms.value


def run(file, name, arrays, scalars=(), meta=(), warps=4, outputs=None):
    """Uploads numpy `arrays` (in .tl parameter order, then `scalars` as
    F32/I32), launches once and returns the arrays read back (as
    Compiled::run does, src/runtime.rs:151-196). `outputs`: indices to read
    back (default: all)."""
    k = kernel(file, name, [a.shape for a in arrays], meta, warps)
    bufs = [tensor(a) for a in arrays]
    launch(k, bufs + list(scalars))
    sync()
    idx = range(len(arrays)) if outputs is None else outputs
    out = {i: read_array(bufs[i], arrays[i].dtype, arrays[i].shape) for i in idx}
    for b in bufs:
        free(b)
    return out


# ---------------------------------------------------------------- the LLM engine

def weights_random(cfg, seed):
    """Weights::random (src/llm/mod.rs:80-108) from the library: (embed,
    layers (flat, layer after layer), norm, head) as float16 arrays."""
    sz = [ctypes.c_size_t() for _ in range(4)]
    check(lib().tsl_weights_sizes(ctypes.byref(cfg), *[ctypes.byref(s) for s in sz]))
    embed = np.zeros(sz[0].value, np.float16)
    layers = np.zeros(sz[1].value * cfg.layers, np.float16)
    norm = np.zeros(sz[2].value, np.float16)
    head = np.zeros(sz[3].value, np.float16)
    check(lib().tsl_weights_random(ctypes.byref(cfg), int(seed), embed.ctypes.data, layers.ctypes.data,
                                   norm.ctypes.data, head.ctypes.data))
    return embed, layers, norm, head


def checkpoint_config(path):
    """safetensors::config (src/llm/safetensors.rs:190-226): the Config of a
    Hugging Face checkpoint directory."""
    cfg = Config()
    check(lib().tsl_checkpoint_config(os.fsencode(path), ctypes.byref(cfg)))
    return cfg


def load_checkpoint(path):
    """safetensors::load (src/llm/safetensors.rs:324-358): (cfg, (embed,
    layers, norm, head)) with head None when the checkpoint ties it to the
    embedding; arrays in the weights_random layout, float16."""
    cfg = checkpoint_config(path)
    sz = [ctypes.c_size_t() for _ in range(4)]
    check(lib().tsl_weights_sizes(ctypes.byref(cfg), *[ctypes.byref(s) for s in sz]))
    embed = np.zeros(sz[0].value, np.float16)
    layers = np.zeros(sz[1].value * cfg.layers, np.float16)
    norm = np.zeros(sz[2].value, np.float16)
    head = np.zeros(sz[3].value, np.float16)
    has = _INT()
    check(lib().tsl_checkpoint_load(os.fsencode(path), ctypes.byref(cfg), embed.ctypes.data, layers.ctypes.data,
                                    norm.ctypes.data, head.ctypes.data, ctypes.byref(has)))
    return cfg, (embed, layers, norm, head if has.value else None)


def save_checkpoint(path, cfg, weights):
    """safetensors::save (src/llm/safetensors.rs:362-444): config.json and one
    F16 model.safetensors under the directory `path` (created if needed);
    weights = (embed, layers, norm, head or None)."""
    os.makedirs(path, exist_ok=True)
    embed, layers, norm, head = weights
    arrs = [np.ascontiguousarray(a, np.float16) for a in (embed, layers, norm)]
    h = None if head is None else np.ascontiguousarray(head, np.float16)
    check(lib().tsl_checkpoint_save(os.fsencode(path), ctypes.byref(cfg), arrs[0].ctypes.data, arrs[1].ctypes.data,
                                    arrs[2].ctypes.data, None if h is None else h.ctypes.data))


def json_roundtrip(text):
    """The checkpoint reader's JSON parser, parsed then written back (a syntax
    error raises TesselError)."""
    b = text.encode("utf-8")
    n = ctypes.c_size_t()
    check(lib().tsl_json_roundtrip(b, None, 0, ctypes.byref(n)))
    buf = ctypes.create_string_buffer(n.value + 1)
    check(lib().tsl_json_roundtrip(b, buf, n.value + 1, ctypes.byref(n)))
    return buf.value.decode("utf-8")


def _i32(a):
    return np.ascontiguousarray(a, np.int32)


class Engine:
    """Engine (src/llm/engine.rs): device weights, paged KV cache, one
    decoder step as a sequence of llm.tl launches."""

    PREFILL, PACKED, DECODE = 0, 1, 2

    def __init__(self, cfg, limits, weights, graphs=True, tune=True):
        embed, layers, norm, head = (np.ascontiguousarray(w, np.float16) for w in weights)
        self.cfg = cfg
        self.limits = limits
        h = _INT()
        check(lib().tsl_engine_new(ctypes.byref(cfg), ctypes.byref(limits), embed.ctypes.data, layers.ctypes.data,
                                   norm.ctypes.data, head.ctypes.data if head is not None else None,
                                   ctypes.byref(h)))
        self.handle = h.value
        self.set(graphs, tune)

    def set(self, graphs, tune):
        check(lib().tsl_engine_set(self.handle, int(graphs), int(tune)))

    def close(self):
        if self.handle is not None:
            check(lib().tsl_engine_free(self.handle))
            self.handle = None

    def step(self, tokens, pos, slots, mode=0, starts=None, tables=None, lens=None, want=()):
        """Engine::step: logits [len(want), vocab] of the rows in `want`."""
        tokens, pos, slots = _i32(tokens), _i32(pos), _i32(slots)
        n = tokens.size
        st = _i32(starts) if starts is not None else None
        nseq = 0
        tb = ln = None
        if tables is not None:
            mp = self.limits.max_seq_pages
            nseq = len(tables)
            tb = np.zeros((nseq, mp), np.int32)
            for i, row in enumerate(tables):
                tb[i, :len(row)] = row
            ln = _i32(lens)
        want = _i32(list(want))
        out = np.zeros((want.size, self.cfg.vocab), np.float32)
        check(lib().tsl_engine_step(self.handle, n, tokens.ctypes.data, pos.ctypes.data, slots.ctypes.data, mode,
                                    st.ctypes.data if st is not None else None, nseq,
                                    tb.ctypes.data if tb is not None else None,
                                    ln.ctypes.data if ln is not None else None, want.size,
                                    want.ctypes.data if want.size else None, out.ctypes.data))
        return out

    def graphs(self):
        """{padded rows: graph} of the decode steps recorded so far."""
        rows, ids, n = np.zeros(64, np.int32), np.zeros(64, np.int32), _INT()
        check(lib().tsl_engine_graphs(self.handle, rows.ctypes.data, ids.ctypes.data, 64, ctypes.byref(n)))
        return dict(zip(rows[:n.value].tolist(), ids[:n.value].tolist()))

    def fallbacks(self):
        """Decode steps recomputed with every rmsnorm applied first, because
        the deferred form's Y = f16(R Wn) overflowed."""
        n = _I64()
        check(lib().tsl_engine_fallbacks(self.handle, ctypes.byref(n)))
        return n.value

    def step_times(self, on=True):
        """Decode-step GPU spans summed since the previous call (then
        cleared; timing on from now when `on`): {"graph": (steps, ms),
        "eager": (steps, ms)}."""
        n, ms = np.zeros(2, np.int64), np.zeros(2, np.float64)
        check(lib().tsl_engine_step_times(self.handle, int(bool(on)), n.ctypes.data, ms.ctypes.data))
        return {"graph": (int(n[0]), float(ms[0])), "eager": (int(n[1]), float(ms[1]))}

    def profile(self, on):
        """Gpu::profile: time every launch on its own (graphs off) from now."""
        check(lib().tsl_engine_profile(self.handle, int(bool(on))))

    def profile_rows(self):
        """[(phase, kernel, launches, ms)], largest time first."""
        n = ctypes.c_size_t()
        check(lib().tsl_engine_profile_rows(self.handle, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(n.value + 1)
        check(lib().tsl_engine_profile_rows(self.handle, buf, n.value + 1, ctypes.byref(n)))
        return [(r["phase"], r["kernel"], r["launches"], r["ms"]) for r in json.loads(buf.value.decode())]

    def generate(self, requests, max_batch, packed=True):
        """sched::generate_with: requests = [(prompt tokens, max_new)] ->
        (token lists, Stats). Afterwards self.first_token_s and self.done_s
        hold each request's Output times (src/llm/sched.rs:14-20)."""
        prompts = _i32([t for p, _ in requests for t in p])
        offsets = np.zeros(len(requests) + 1, np.int64)
        offsets[1:] = np.cumsum([len(p) for p, _ in requests])
        max_new = _i32([m for _, m in requests])
        out = np.zeros(max(int(max_new.sum()), 1), np.int32)
        counts = np.zeros(len(requests), np.int32)
        st = Stats()
        times = np.zeros(2 * max(len(requests), 1), np.float64)
        check(lib().tsl_generate(self.handle, len(requests), prompts.ctypes.data, offsets.ctypes.data,
                                 max_new.ctypes.data, int(max_batch), int(packed), out.ctypes.data,
                                 counts.ctypes.data, ctypes.byref(st), times.ctypes.data))
        self.first_token_s = times[0:2 * len(requests):2].tolist()
        self.done_s = times[1:2 * len(requests):2].tolist()
        res, base = [], 0
        for i, m in enumerate(max_new):
            res.append(out[base:base + counts[i]].tolist())
            base += int(m)
        return res, st


def schedule_trace(limits, eos, requests, max_batch, packed, script):
    """The scheduler of Engine.generate run on the CPU with no model
    (tsl_schedule_trace): requests = [(prompt tokens, max_new)], script =
    per request the token ids its steps return, in order. Returns (the steps
    as dicts of the integer inputs sched.rs hands Engine::step, token lists,
    Stats)."""
    prompts = _i32([t for p, _ in requests for t in p])
    offsets = np.zeros(len(requests) + 1, np.int64)
    offsets[1:] = np.cumsum([len(p) for p, _ in requests])
    max_new = _i32([m for _, m in requests])
    flat = np.zeros(max(int(max_new.clip(0).sum()), 1), np.int32)
    base = 0
    for (_, m), sc in zip(requests, script):
        flat[base:base + min(len(sc), max(m, 0))] = sc[:max(m, 0)]
        base += max(m, 0)
    out = np.zeros_like(flat)
    counts = np.zeros(max(len(requests), 1), np.int32)
    st = Stats()
    used = _I64(0)
    cap = 1 << 16
    while True:
        trace = np.zeros(cap, np.int32)
        r = lib().tsl_schedule_trace(ctypes.byref(limits), int(eos), len(requests), prompts.ctypes.data,
                                     offsets.ctypes.data, max_new.ctypes.data, int(max_batch), int(packed),
                                     flat.ctypes.data, out.ctypes.data, counts.ctypes.data, ctypes.byref(st),
                                     trace.ctypes.data, cap, ctypes.byref(used))
        if r != 0 and used.value > cap:
            cap = int(used.value)
            continue
        check(r)
        break
    steps, i, mp = [], 0, limits.max_seq_pages
    while i < used.value:
        mode, n, nw = (int(x) for x in trace[i:i + 3])
        i += 3
        s = {"mode": mode}
        for k in ("tokens", "pos", "slots"):
            s[k] = trace[i:i + n].tolist()
            i += n
        if mode == 1:
            s["starts"] = trace[i:i + n].tolist()
            i += n
        if mode == 2:
            s["tables"] = trace[i:i + n * mp].reshape(n, mp).tolist()
            i += n * mp
            s["lens"] = trace[i:i + n].tolist()
            i += n
        s["want"] = trace[i:i + nw].tolist()
        i += nw
        steps.append(s)
    toks, base = [], 0
    for k, (_, m) in enumerate(requests):
        toks.append(out[base:base + counts[k]].tolist())
        base += m
    return steps, toks, st


class Rng:
    """bench::Rng (src/bench.rs:13-35), the xorshift generator of the
    benchmark suite's inputs, through the library (tsl_rng_*)."""

    def __init__(self, seed):
        self.state = _U64(0)
        check(lib().tsl_rng_new(seed, ctypes.byref(self.state)))

    def bits(self):
        out = _U64(0)
        check(lib().tsl_rng_bits(ctypes.byref(self.state), ctypes.byref(out)))
        return out.value

    def below(self, n):
        return self.bits() % n

    def tensor(self, dtype, shape, scale=1.0):
        """Rng::tensor: uniform [-1, 1) times scale, as 'f32' or 'f16'."""
        n = int(np.prod(shape)) if len(shape) else 1
        code, npdt = {"f32": (0, np.float32), "f16": (1, np.float16)}[dtype]
        out = np.empty(n, npdt)
        check(lib().tsl_rng_tensor(ctypes.byref(self.state), n, scale, code, out.ctypes.data))
        return out.reshape(shape)


def padded(n):
    """Rows a step is compiled for (src/llm/engine.rs:96-98)."""
    return 1 << (max(n, 16) - 1).bit_length()


def mm_candidates(m, two):
    """The tile configurations the engine's tuner tries for an m-row matmul
    (src/llm/engine.rs:106-147): [(meta, warps)], the default first."""
    def c(bm, bn, bk, w):
        return [("BM", bm), ("BN", bn), ("BK", bk)], w
    if m >= 64:
        if two:
            return [c(64, 64, 32, 4), c(128, 64, 32, 4), c(64, 32, 32, 4)]
        return [c(64, 128, 32, 4), c(64, 64, 32, 4), c(128, 128, 32, 4), c(128, 64, 32, 4)]
    if m >= 32:
        v = [c(32, 64, 64, 4), c(32, 32, 64, 4), c(32, 32, 128, 4), c(32, 64, 128, 4), c(32, 16, 128, 2),
             c(16, 64, 64, 4), c(16, 32, 128, 4)]
        if not two:
            v.append(c(32, 16, 256, 2))
        return v
    return [c(16, 64, 64, 4), c(16, 32, 64, 4), c(16, 32, 128, 4), c(16, 64, 128, 4), c(16, 16, 128, 2),
            c(16, 16, 256, 2)]
