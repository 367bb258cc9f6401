/*
 * tessel_amd: the C ABI of the MI355X (gfx950) kernel library.
 *
 * One device, one stream, driven from one thread at a time: the launch
 * surface of tessel's GPU layer (src/gpu.rs, src/runtime.rs, src/driver.rs),
 * with hand-written HIP kernels behind the same kernel names and argument
 * order as the .tl sources (kernels/{basic,matmul,attention,llm}.tl).
 *
 * Every call returns 0 on success or a negative status; tsl_last_error()
 * then gives the message ("{what}: HIP error {code} {name}" for HIP
 * failures, as src/driver.rs:181-195 formats CUDA ones). Plain pointers and
 * sizes only: device pointers travel as uint64_t.
 */
#ifndef TESSEL_H
#define TESSEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TSL_OK 0
#define TSL_ERR_HIP (-1)     /* a HIP call failed */
#define TSL_ERR_ARG (-2)     /* bad argument: arity, shape, meta, bounds */
#define TSL_ERR_NOKERNEL (-3) /* no such file/kernel */

/* The message of the last failed call on this thread ("" if none). */
const char* tsl_last_error(void);

/* ---- device (src/driver.rs:110-179 Cuda::open/bind; src/runtime.rs:48-52) */

/* Opens device 0 and creates the library's stream (idempotent). */
int tsl_open(void);
/* Device name (gcnArchName + marketing name) into buf. */
int tsl_device_name(char* buf, size_t len);
/* Compute units and peak clock in MHz, for roofline figures. */
int tsl_device_info(int* cus, int* mhz);
/* Waits for the stream (src/driver.rs:274-277 Cuda::sync). */
int tsl_sync(void);
/* The library's stream, as a hipStream_t cast to a pointer. */
void* tsl_stream(void);

/* ---- memory (src/gpu.rs:70-133, src/driver.rs:197-272) */

/* A zero-filled device buffer of at least max(bytes, 4) bytes. */
int tsl_alloc(size_t bytes, uint64_t* dptr);
/* Frees a buffer from tsl_alloc (the reference never frees; added). */
int tsl_free(uint64_t dptr);
/* Synchronous host->device copy of n bytes (src/driver.rs:245-254). */
int tsl_upload(uint64_t dst, const void* src, size_t n);
/* Synchronous device->host copy of n bytes, after the stream drains
 * (src/gpu.rs:110-133, src/driver.rs:256-264). */
int tsl_download(void* dst, uint64_t src, size_t n);
/* Fills n 32-bit words with a quiet NaN (src/driver.rs:266-272). */
int tsl_fill_nan(uint64_t dst, size_t n);

/* ---- kernels (src/gpu.rs:148-216 Gpu::kernel / Gpu::launch,
 *                src/runtime.rs:202-236 Compiled::launch_raw) */

/*
 * Kernel `name` of file `file` ("basic", "matmul", "attention", "llm"),
 * specialised for the array shapes given in parameter order: nshapes
 * arrays, array i has ranks[i] dimensions stored consecutively in dims.
 * meta_names/meta_values override the kernel's meta constants (an unknown
 * name is an error, src/ir.rs:1039-1043); warps is recorded in the key.
 * The same key "{file}/{name} {shapes:?} {meta:?} {warps}"
 * (src/gpu.rs:156) returns the same handle.
 */
int tsl_kernel(const char* file, const char* name, int nshapes, const int* ranks, const int64_t* dims,
               int nmeta, const char* const* meta_names, const int64_t* meta_values, int warps,
               int* handle);
/* The cache key of a handle, into buf. */
int tsl_kernel_key(int handle, char* buf, size_t len);
/*
 * Launches kernel `handle` asynchronously on the library stream with one
 * 64-bit argument per .tl parameter, in declaration order: arrays are
 * device pointers, f32/i32 scalars their bit pattern in the low 32 bits
 * (src/gpu.rs:179-195). An arity mismatch is an error (src/runtime.rs:203).
 */
int tsl_launch(int handle, const uint64_t* args, int nargs);

/* ---- timing and graphs (src/driver.rs:340-380, src/runtime.rs:295-316) */

/* Event-timed milliseconds of `iters` launches of handle (after the stream
 * drains); ms receives the total. */
int tsl_time_launches(int handle, const uint64_t* args, int nargs, int iters, float* ms);
/* Each of `iters` launches of handle timed on its own with a pair of events
 * (Cuda::time, src/driver.rs:365-380, as Compiled::time uses it,
 * src/runtime.rs:294-316): ms[i] receives launch i's milliseconds. */
int tsl_time_each(int handle, const uint64_t* args, int nargs, int iters, float* ms);
/* Starts recording this thread's launches on the stream into a graph
 * (relaxed capture mode, src/driver.rs:340-348). */
int tsl_capture_begin(void);
/* Ends the recording and instantiates it: *graph identifies it. */
int tsl_capture_end(int* graph);
/* The nodes a recorded graph holds, counted by type when it was recorded
 * (hipGraphGetNodes before instantiation): counts[0] kernels, [1] memsets,
 * [2] memcpys, [3] any other node. No reference counterpart: a check that
 * captured sequences are kernels only. */
int tsl_graph_nodes(int graph, int64_t* counts);
/* Replays a recorded graph asynchronously (src/driver.rs:360-363). */
int tsl_replay(int graph);
/* Events on the stream, for timing a caller's own sequence. */
int tsl_event_record(int* event);
int tsl_event_elapsed(int start, int end, float* ms);

/*
 * decode_attention (kernels/llm.tl:150-172) with no allocation. This entry
 * point has no counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). It takes the arguments of the
 * decode_attention launch as plain device pointers and sizes (q [B,H,D],
 * kc/vc [NP,P,G,D] f16; table i32 [B,MP]; lens i32 [B]; o [B,H,D] f16),
 * runs the same kernels as tsl_launch of a decode_attention handle, and
 * keeps their partial states in a library-owned device array of
 * TSL_NOALLOC_SCRATCH_BYTES per GPU (resident until the process ends)
 * instead of a per-handle allocation. A shape needing more scratch is
 * TSL_ERR_ARG. Every call on one GPU shares that array: calls that overlap
 * on one GPU (other threads, other streams) race. Nothing in it needs to
 * start at zero; the kernels write every state they read. Asynchronous on
 * the library stream; calls no hipMalloc/hipFree.
 */
#define TSL_NOALLOC_SCRATCH_BYTES (64u << 20)
int tsl_decode_attention_noalloc(uint64_t q, uint64_t kc, uint64_t vc, uint64_t table, uint64_t lens, uint64_t o,
                                 float scale, int B, int H, int G, int D, int NP, int P, int MP);

/* ---- calibration probes (no reference counterpart: they measure what this
 * GPU sustains on the hot path's building blocks, for the roofline notes) */

/* TFLOP/s of v_mfma_f32_32x32x16_f16 issued back to back by 8 wavefronts per
 * CU (the GEMM's occupancy and 8 accumulators per wave, a workgroup barrier
 * every 32 MFMAs), operands random f16 (random = 1) or nearly constant, with
 * or without the GEMM's LDS operand reads (lds_reads = 1). One launch of
 * iters iterations after a warm-up launch. */
int tsl_probe_mfma(int random, int lds_reads, int iters, double* tflops);
/* The same with v_mfma_f32_16x16x32_f16 (8 independent 16x16 accumulators
 * per wave, operands in registers): the MFMA form the GEMMs use. */
int tsl_probe_mfma16(int random, int iters, double* tflops);
/* GB/s of iters back-to-back streaming reads of bytes each (512 workgroups,
 * four 16-byte loads in flight per lane), launch i reading window i (mod the
 * windows that fit) of the buf_bytes at device address buf. */
int tsl_probe_stream(uint64_t buf, size_t buf_bytes, size_t bytes, int iters, double* gbps);

/* ---- the LLM engine (src/llm/engine.rs, src/llm/sched.rs, src/llm/mod.rs) */

/* Config (src/llm/mod.rs:15-28). */
typedef struct {
    int32_t dim, layers, heads, kv_heads, head_dim, ffn, vocab;
    float eps, rope_theta;
    int32_t max_pos, bos, eos;
} tsl_config;

/* Limits (src/llm/engine.rs:23-32). */
typedef struct {
    int32_t page, pages, max_tokens, max_seq_pages;
} tsl_limits;

/* bench::Rng (src/bench.rs:13-35), the xorshift generator of the benchmark
 * suite's inputs: Rng::new(seed) into *state; bits() into *out; tensor(dtype,
 * n, scale) into out as n f32 (dtype 0) or f16 bits rounded to nearest even
 * (dtype 1). The state advances as the reference's does. */
int tsl_rng_new(uint64_t seed, uint64_t* state);
int tsl_rng_bits(uint64_t* state, uint64_t* out);
int tsl_rng_tensor(uint64_t* state, size_t n, float scale, int dtype, void* out);

/* Weights::random(cfg, seed) (src/llm/mod.rs:80-108) into host arrays of
 * f16 bits: embed[vocab*dim], per layer (attn_norm[dim],
 * wqkv[(H+2G)*D*dim], wo[dim*H*D], mlp_norm[dim], wg[ffn*dim],
 * wu[ffn*dim], wd[dim*ffn]) concatenated layer after layer, norm[dim],
 * lm_head[vocab*dim]. Sizes from tsl_weights_sizes. */
int tsl_weights_sizes(const tsl_config* cfg, size_t* embed, size_t* per_layer, size_t* norm, size_t* head);
int tsl_weights_random(const tsl_config* cfg, uint64_t seed, uint16_t* embed, uint16_t* layers, uint16_t* norm,
                       uint16_t* head);

/* Engine::new (src/llm/engine.rs:150-223): uploads the weights (layout as
 * tsl_weights_random; head may be NULL to tie it to embed). */
int tsl_engine_new(const tsl_config* cfg, const tsl_limits* lim, const uint16_t* embed, const uint16_t* layers,
                   const uint16_t* norm, const uint16_t* head, int* engine);
int tsl_engine_free(int engine);
/* Engine flags: graphs (decode-step graph replay), tune (matmul tuner). */
int tsl_engine_set(int engine, int graphs, int tune);

/* Gpu::profile for the engine's launches (src/gpu.rs:40, :197-228): on != 0
 * clears the profile and times every launch on its own (graphs are not
 * replayed meanwhile); rows: the profile as JSON text, a list of {"phase":
 * "prefill"|"decode", "kernel": "{name} -> {output shape}", "launches": n,
 * "ms": total}, largest time first. *len gets the text's length; out gets
 * the text (NUL-terminated) when cap > *len. */
int tsl_engine_profile(int engine, int on);
int tsl_engine_profile_rows(int engine, char* out, size_t cap, size_t* len);

/* The decode-step graphs the engine has recorded (src/llm/engine.rs:
 * 330-350 keeps one per padded batch size): up to cap (rows, graph) pairs
 * into rows/graphs, *n the number recorded. */
int tsl_engine_graphs(int engine, int32_t* rows, int32_t* graphs, int cap, int* n);

/* No counterpart in the reference (the reference normalises before every
 * projection): decode steps of up to 32 rows defer each rmsnorm into the
 * consuming projection, through Y = f16(R Wn), which overflows f16 where
 * |R Wn| >= 65520 although rmsnorm(R) Wn need not. Such a step is recomputed
 * with every norm applied first; *n gets how many steps were. */
int tsl_engine_fallbacks(int engine, int64_t* n);

/* No counterpart in the reference: decode-step timing. From this call on
 * (on != 0), each decode step's GPU span (its input upload to the end of its
 * last kernel, by events on the stream) is summed, apart for graph replays
 * (index 0) and eager launches (index 1). The call returns, in steps[2] and
 * ms[2], what was summed since the previous call, and clears it. */
int tsl_engine_step_times(int engine, int on, int64_t* steps, double* ms);

/* Engine::step (src/llm/engine.rs:275-354). mode 0 = Prefill, 1 = Packed
 * (starts[n]), 2 = Decode (tables: nseq rows of max_seq_pages pages, lens:
 * nseq). logits receives nwant * vocab floats for rows want[0..nwant). */
int tsl_engine_step(int engine, int n, const int32_t* tokens, const int32_t* pos, const int32_t* slots, int mode,
                    const int32_t* starts, int nseq, const int32_t* tables, const int32_t* lens, int nwant,
                    const int32_t* want, float* logits);

/* sched::generate_with (src/llm/sched.rs:52-179): greedy generation of
 * nreq requests (prompt r = prompts[offsets[r] .. offsets[r+1]), max_new[r]
 * tokens). out_tokens gets sum(max_new) slots: request r's tokens start at
 * the prefix sum of max_new; out_counts[r] is how many it produced.
 * stats: prefill_steps, decode_steps, prompt_tokens, generated,
 * largest_batch, decode_tokens (int64) and seconds, decode_seconds.
 * out_times (may be NULL): 2 nreq doubles, request r's Output::first_token_s
 * and done_s (seconds from the start of the call, src/llm/sched.rs:14-20).
 * Every request is checked before any step runs: an empty prompt, one
 * longer than max_tokens, max_new < 1, or more pages than max_seq_pages or
 * the whole pool holds is TSL_ERR_ARG. */
typedef struct {
    int64_t prefill_steps, decode_steps, prompt_tokens, generated, largest_batch, decode_tokens;
    double seconds, decode_seconds;
} tsl_stats;
int tsl_generate(int engine, int nreq, const int32_t* prompts, const int64_t* offsets, const int32_t* max_new,
                 int max_batch, int packed, int32_t* out_tokens, int32_t* out_counts, tsl_stats* stats,
                 double* out_times);
/* The scheduler of tsl_generate with no model and no device: the same
 * admission, page allocation and step inputs, where each step's next token
 * for request r is taken in order from script (laid out as out_tokens), so
 * the integer stream sched.rs feeds Engine::step (src/llm/sched.rs:52-179:
 * slots :98 and :141, LIFO pages :60 :88 :125 :168) can be checked on a CPU.
 * Every step appends to trace: mode, n, nwant, tokens[n], pos[n], slots[n],
 * starts[n] (mode 1 only), tables[n * max_seq_pages] and lens[n] (mode 2
 * only), want[nwant]. *used receives the words written (or needed, when
 * more than cap). Errors as tsl_generate. */
int tsl_schedule_trace(const tsl_limits* lim, int eos, int nreq, const int32_t* prompts, const int64_t* offsets,
                       const int32_t* max_new, int max_batch, int packed, const int32_t* script, int32_t* out_tokens,
                       int32_t* out_counts, tsl_stats* stats, int32_t* trace, int64_t cap, int64_t* used);

/* ---- checkpoints (src/llm/safetensors.rs) */

/* The shape of a Hugging Face Llama-family checkpoint directory, from its
 * config.json (src/llm/safetensors.rs:190-226 config): required
 * hidden_size, num_hidden_layers, num_attention_heads, intermediate_size,
 * vocab_size; num_key_value_heads, head_dim, rms_norm_eps (1e-6),
 * rope_theta (10000), max_position_embeddings (2048, capped at 8192),
 * bos_token_id (1), eos_token_id (a number or the first of a list, else -1)
 * default as there; a non-null rope_scaling is an error. */
int tsl_checkpoint_config(const char* dir, tsl_config* cfg);
/* Its tensors (model.safetensors, else the shards that
 * model.safetensors.index.json lists) as f16 bits in the layout of
 * tsl_weights_random; F16 is copied, BF16 and F32 are rounded to nearest
 * even. q/k/v projections are stacked into wqkv. *has_head is 0 when there
 * is no lm_head.weight (head untouched: tie it to embed), else head is
 * filled. Biases, missing tensors, other shapes and other dtypes are
 * errors, reported as the reference words them
 * (src/llm/safetensors.rs:229-358 index/read/load). cfg must be the
 * directory's tsl_checkpoint_config. */
int tsl_checkpoint_load(const char* dir, const tsl_config* cfg, uint16_t* embed, uint16_t* layers, uint16_t* norm,
                        uint16_t* head, int* has_head);
/* Writes weights (the tsl_weights_random layout; head NULL: tied) as a
 * checkpoint directory that exists already: config.json and one F16
 * model.safetensors laid out as Hugging Face lays one out
 * (src/llm/safetensors.rs:362-444 save). */
int tsl_checkpoint_save(const char* dir, const tsl_config* cfg, const uint16_t* embed, const uint16_t* layers,
                        const uint16_t* norm, const uint16_t* head);
/* The checkpoint reader's JSON parser (src/llm/safetensors.rs:44-187
 * parse_json): text parsed and written back normalised (members in file
 * order, strings unescaped then re-escaped, numbers shortest round-trip);
 * *len gets its length, out the text when cap > *len. A syntax error
 * returns TSL_ERR_ARG with the byte offset in the message. */
int tsl_json_roundtrip(const char* text, char* out, size_t cap, size_t* len);

#ifdef __cplusplus
}
#endif

#endif
