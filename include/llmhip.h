/*
 * llmhip.h — the C-ABI of the MI355X (gfx950) forward pass for llama / qwen2
 * GGUF models: the drop-in for the GPU half of go-wasmcontainers/llm.
 *
 * Two layers, both plain C (pointers, sizes, status codes; no C++ or torch
 * types):
 *
 *  1. llmhip_*  — the device layer.  This is what the Go package's cgo wrapper
 *     binds (its NewGPU keeps parsing the GGUF header and ConfigFrom in Go and
 *     streams raw tensor bytes in, go/gpu_hip.go).  It replaces the
 *     webgpu Device / Recorder / Submit / Readback the reference drives.
 *  2. llm_*     — a C++ restatement of the reference's host package for hosts
 *     without Go (tests, benchmarks, the C++ `generate` tool): the GGUF header
 *     parser, ConfigFrom, NewGPU's streaming loader, Generate, PrefillLogits,
 *     Peek.  It only calls layer 1.
 *
 * Conventions (those of the reference's Go API, gpu.go):
 *  - every function returns 0 (LLMHIP_OK) or a negative LLMHIP_ERR_* code;
 *    llmhip_last_error() is the thread's last message, prefixed "llm:" like
 *    the reference's errors.  No partial results on error.
 *  - host buffers are caller-owned and copied synchronously; the library never
 *    retains a caller pointer (cgo's rule).
 *  - a model owns every device resource it allocates until llmhip_model_free;
 *    it is not safe for concurrent use (one HIP stream per model).
 *  - pointers named *_dev are device pointers (hipMalloc / torch tensors).
 */
#ifndef LLMHIP_H
#define LLMHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define LLMHIP_API __attribute__((visibility("default")))
#else
#define LLMHIP_API
#endif

/* status codes */
enum {
  LLMHIP_OK = 0,
  LLMHIP_ERR_ARG = -1,     /* a bad argument (sizes, names, alignment) */
  LLMHIP_ERR_DEVICE = -2,  /* a HIP runtime failure or no device */
  LLMHIP_ERR_BUDGET = -3,  /* MemoryBudget would be exceeded (gpu.go:175-177) */
  LLMHIP_ERR_TYPE = -4,    /* a tensor type without a kernel (gpu.go:326) */
  LLMHIP_ERR_CONTEXT = -5, /* prompt + tokens exceed the context (gpu.go:948-950) */
  LLMHIP_ERR_FORMAT = -6,  /* a malformed GGUF header or model (gguf.go, config.go) */
  LLMHIP_ERR_STATE = -7,   /* a call out of order (e.g. decode before prefill) */
  LLMHIP_ERR_IO = -8       /* reading the model file failed */
};

/* ggml tensor types, gguf/gguf.go:60-69 */
enum { LLMHIP_F32 = 0, LLMHIP_F16 = 1, LLMHIP_Q4_0 = 2, LLMHIP_Q4_1 = 3, LLMHIP_Q8_0 = 8 };

/* The thread's last error message ("" when none). */
LLMHIP_API const char* llmhip_last_error(void);

/* ------------------------------------------------------------- limits */

/* Limits, gpu.go:28-36.  Filled from hipDeviceProp_t by llmhip_device_limits;
 * MemoryBudget (bytes of device memory a model may hold) is honoured by every
 * allocation of a model exactly as in gpu.go:170-185. */
typedef struct llmhip_limits {
  uint32_t max_invocations_per_workgroup;
  uint32_t max_workgroup_storage;
  uint32_t max_workgroups_per_dimension;
  uint32_t max_storage_buffers;
  uint64_t max_binding_size;
  uint64_t max_buffer_size;
  uint64_t memory_budget;
} llmhip_limits;

/* Number of HIP devices. */
LLMHIP_API int llmhip_device_count(int* n);
/* The device's limits (memory_budget = its total memory). */
LLMHIP_API int llmhip_device_limits(int ordinal, llmhip_limits* out);

/* Device memory for callers with no allocator of their own (the tests and
 * benchmarks of the kernel-level entry points): zeroed at allocation.  Reads
 * and writes are synchronous and pass through pinned staging, never DMA to
 * or from caller memory.  No counterpart in the reference (its buffers are
 * webgpu Buffers). */
LLMHIP_API int llmhip_buffer_alloc(int ordinal, uint64_t bytes, void** out);
LLMHIP_API void llmhip_buffer_free(void* dev);
LLMHIP_API int llmhip_buffer_write(void* dev, const void* host, uint64_t bytes);
LLMHIP_API int llmhip_buffer_read(void* host, const void* dev, uint64_t bytes);
LLMHIP_API int llmhip_device_synchronize(int ordinal);
/* Measurement helpers: the pinned host-to-device copy rate in GB/s over
 * `iters` copies of `bytes` (the bound of the loader), and one
 * device-to-device copy of `bytes` (a copy of known size, for scaling the
 * FETCH_SIZE / WRITE_SIZE counters). */
LLMHIP_API int llmhip_bench_h2d(int ordinal, uint64_t bytes, int iters, float* gbps);
LLMHIP_API int llmhip_copy_calibration(int ordinal, uint64_t bytes);

/* --------------------------------------------------- quantised matrices */

/* A quantised [rows][k] matrix on one device, repacked on the device from raw
 * GGUF blocks into the kernels' tiled layout (Q4_0, Q4_1, Q8_0; k a multiple
 * of 32).  The kernel-level surface used by the isolated-kernel sweep and the
 * bit-exact dequantisation tests; the model uses the same code internally.
 * Replaces gpu.go:297-391 (loadMatRows / streamMat) for one matrix. */
typedef struct llmhip_qmat llmhip_qmat;

LLMHIP_API int llmhip_qmat_create(int ordinal, uint32_t ggml_type, uint64_t rows, uint64_t k, llmhip_qmat** out);
/* Upload raw GGUF blocks (host memory) covering bytes [byte_offset,
 * byte_offset+nbytes) of the tensor's data; both must be whole blocks.  Pieces
 * may arrive in any order; the repack runs on the device. */
LLMHIP_API int llmhip_qmat_upload(llmhip_qmat* m, const void* raw, uint64_t nbytes, uint64_t byte_offset);
/* out_dev[rows][k] = the f32 value of every weight, bit-exact with the CPU
 * path's dequantisation (cpu.go:233-251). */
LLMHIP_API int llmhip_qmat_dequant(llmhip_qmat* m, float* out_dev, void* hip_stream);
/* y_dev[n][rows] (+)= W x_dev[n][k] for n tokens (1 <= n <= 64), in f32:
 * the matvec of cpu.go:143-222 for each token.  accumulate != 0 adds into y. */
LLMHIP_API int llmhip_qmat_gemv(llmhip_qmat* m, const float* x_dev, float* y_dev, int n, int accumulate, void* hip_stream);
/* llmhip_qmat_gemv without any allocation, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, hosts that
 * forbid it).  No counterpart in the reference.  Products of 5 or more tokens
 * stage their activations in one static device array per GPU (about 2.2 MB,
 * held until the process ends) instead of a buffer the matrix allocates:
 * k at most LLMHIP_NOALLOC_MAX_K (LLMHIP_ERR_ARG above it), n at most 64.
 * Every call on a GPU shares that GPU's array, so calls that overlap on one GPU
 * (on different streams, or from different threads) race; calls in one stream
 * are ordered and safe.  Same kernels and results as llmhip_qmat_gemv. */
#define LLMHIP_NOALLOC_MAX_K 8192
LLMHIP_API int llmhip_qmat_gemv_noalloc(llmhip_qmat* m, const float* x_dev, float* y_dev, int n, int accumulate,
                                        void* hip_stream);
/* The ExactGGML form (cpu.go:117-140, 166-214): each token's x quantised to
 * Q8_0 blocks (Q8_1 for Q4_1 weights) as quantizeQ8 does, then ggml's integer
 * block products scaled by d_w * d_x (+ m_w * s_x); y_dev = the result. */
LLMHIP_API int llmhip_qmat_gemv_q8(llmhip_qmat* m, const float* x_dev, float* y_dev, int n, void* hip_stream);
/* Device bytes the matrix holds (equal to its GGUF bytes when rows % 16 == 0). */
LLMHIP_API uint64_t llmhip_qmat_bytes(const llmhip_qmat* m);
/* Algorithmic (GGUF-format) bytes of the matrix: rows * k / 32 * block bytes. */
LLMHIP_API uint64_t llmhip_qmat_gguf_bytes(const llmhip_qmat* m);
/* Average device time in microseconds of one llmhip_qmat_gemv over `iters`
 * back-to-back launches cycling through the `count` matrices (same shape and
 * type), measured with hipEvents on `hip_stream` after `warmup` launches.
 * Cycling through copies whose total exceeds the 256 MB Infinity Cache makes
 * the weights come from HBM. */
LLMHIP_API int llmhip_qmat_bench(llmhip_qmat* const* mats, int count, const float* x_dev, float* y_dev, int n, int iters,
                      int warmup, void* hip_stream, float* avg_us);
/* The same measured over hipGraph replays: the launches (cycling through the
 * `count` matrices, at least 16 per graph) are captured once on `hip_stream`
 * (a stream of its own when null) after `warmup` direct launches, and the
 * graph is replayed until `iters` launches are timed.  No counterpart in the
 * reference (a measurement entry point, as the reference's bench mode is). */
LLMHIP_API int llmhip_qmat_bench_graph(llmhip_qmat* const* mats, int count, const float* x_dev, float* y_dev, int n,
                                       int iters, int warmup, void* hip_stream, float* avg_us);
/* A copy of m on the same device (device-to-device): rotating copies whose
 * total exceeds the Infinity Cache makes a benchmark read HBM. */
LLMHIP_API int llmhip_qmat_clone(const llmhip_qmat* m, llmhip_qmat** out);
LLMHIP_API void llmhip_qmat_free(llmhip_qmat* m);

/* -------------------------------------------------------------- models */

/* Config, config.go:11-23 (what ConfigFrom reads from the GGUF metadata). */
typedef struct llmhip_config {
  int32_t layers, embd, ff, heads, kv_heads, head_dim, vocab, ctx;
  float rope_base, eps;
  int32_t arch; /* 0 llama (rope NORM), 1 qwen2 (rope NEOX, QKV biases) */
  int32_t rope_neox, bias, tied_output;
} llmhip_config;

/* Stats, gpu.go:56-60: submits are graph launches / synchronising calls,
 * dispatches are kernel launches (graph nodes replayed). */
typedef struct llmhip_stats {
  int64_t submits, dispatches, tokens;
} llmhip_stats;

typedef struct llmhip_model llmhip_model;

/* The allocating half of NewGPU (gpu.go:465-541): ctx is clamped to cfg->ctx
 * when <= 0 or larger (gpu.go:470-472); activations, the f32 KV cache and the
 * RoPE table (cos and sin of pos * base^(-2i/hd) in double, gpu.go:524-534)
 * are allocated against lim->memory_budget (lim NULL: the device's limits).
 * prefill_batch is the prompt chunk (PrefillBatch, gpu.go:165; 0 = 64). */
LLMHIP_API int llmhip_model_create(int ordinal, const llmhip_limits* lim, const llmhip_config* cfg, int ctx,
                                   int prefill_batch, llmhip_model** out);
/* Declare a tensor of the GGUF file (name, ggml type, dims with dims[0] the
 * contiguous one).  Every tensor the model needs must be declared before the
 * first upload; names the model does not use are accepted and ignored. */
LLMHIP_API int llmhip_model_tensor(llmhip_model* m, const char* name, uint32_t ggml_type, const uint64_t* dims,
                                   uint32_t ndims);
/* Stream raw tensor bytes [byte_offset, byte_offset+nbytes) of a declared
 * tensor (whole blocks for quantised types): streamMat / loadF32 /
 * loadGroup of gpu.go:297-407 and fused.go:108-190, with the repack, the
 * QKV and gate/up concatenation and the NEOX pairing done on the device.
 * A range overlapping bytes of the tensor uploaded before is refused
 * (LLMHIP_ERR_ARG), so that finalize sees each byte counted once. */
LLMHIP_API int llmhip_model_upload(llmhip_model* m, const char* name, const void* raw, uint64_t nbytes,
                                   uint64_t byte_offset);
/* The loader's fast path: the same upload, with the nbytes read from the open
 * file descriptor fd at file_offset (pread, which leaves the descriptor's own
 * position alone) straight into pinned staging by a pool of host threads,
 * overlapped with the DMA and repack of the pieces before.  Replaces
 * streamMat's ReadAt loop (gpu.go:356-389) when the io.ReaderAt is a file;
 * one call may cover a whole tensor. */
LLMHIP_API int llmhip_model_upload_file(llmhip_model* m, const char* name, int fd, uint64_t file_offset,
                                        uint64_t nbytes, uint64_t byte_offset);
/* The fast path for a whole file: every listed tensor (its declared size, from
 * file_offsets[i]) in one call.  Consecutive tensors are read in runs of up to
 * 8 MiB, each with one parallel pread and one DMA, and each tensor's repack
 * runs on its part of the run; the same result as one llmhip_model_upload per
 * tensor.  Replaces NewGPU's tensor-by-tensor loadMat / loadMatRows / loadF32 /
 * loadGroup calls (gpu.go:543-740, fused.go:108-190) when the io.ReaderAt is a
 * file. */
LLMHIP_API int llmhip_model_upload_file_tensors(llmhip_model* m, int fd, uint32_t n, const char* const* names,
                                                const uint64_t* file_offsets);
/* Check that every needed tensor arrived in full ("llm: missing tensor"):
 * its uploaded ranges, disjoint, cover all of its bytes. */
LLMHIP_API int llmhip_model_finalize(llmhip_model* m);
/* Run a prompt from position 0 (prefill, gpu.go:853-900) in chunks of
 * prefill_batch tokens; optionally copy out the last token's logits (vocab
 * floats, PrefillLogits gpu.go:904-927) and the greedy token it samples.
 * Requires 1 <= n <= ctx and ids in [0, vocab). */
LLMHIP_API int llmhip_model_prefill(llmhip_model* m, const int32_t* ids, int n, float* logits, int32_t* first);
/* cnt greedy decode steps (one hipGraph launch each; gpu.go:987-1009): each
 * embeds the last sampled token, runs the layers and the head and samples on
 * the GPU.  out receives the cnt sampled ids.  Requires pos + cnt <= ctx. */
LLMHIP_API int llmhip_model_decode(llmhip_model* m, int cnt, int32_t* out);
/* The first n 4-byte words of a named buffer as float32 (Peek, gpu.go:1018-1043):
 * x, q, att (the merged attention output), gate (the SwiGLU activations),
 * up (the up product W_up h), h (the head's normed row: RMSNorm of the last
 * token's residual with output_norm, formed at the call), k and v (the K and V
 * rows the latest pass appended last, in the last layer run: K after bias and
 * RoPE, as the cache holds them),
 * logits, state, tokens, outb, and
 * kvblk.N. (layer N's cache [2][ctx][kvd]). */
LLMHIP_API int llmhip_model_peek(llmhip_model* m, const char* name, float* out, uint64_t n);
LLMHIP_API uint64_t llmhip_model_memory_used(const llmhip_model* m);
LLMHIP_API int llmhip_model_stats(const llmhip_model* m, llmhip_stats* out);
LLMHIP_API int llmhip_model_config(const llmhip_model* m, llmhip_config* out, int* ctx);
/* Store the KV cache in binary16, each K and V element rounded to nearest even
 * (the F16KV mode of the reference's CPU path, cpu.go:22-24 and 298-299; its
 * GPU path keeps f32).  Halves the cache and the attention's reads.  Call
 * before the first llmhip_model_upload / finalize. */
LLMHIP_API int llmhip_model_set_kv_f16(llmhip_model* m, int on);
/* The ExactGGML mode of the reference's CPU path (cpu.go:15-21): every matrix
 * input (the normed residual, the attention output, the SwiGLU activations)
 * is quantised to Q8_0 blocks (Q8_1 for Q4_1 weights) as quantizeQ8 does
 * (cpu.go:117-140), each block product is ggml's integer dot product scaled
 * by d_w * d_x (+ m_w * s_x) (cpu.go:166-214), and the KV cache is binary16.
 * Results match the CPU path with ExactGGML set, not the f32 path.  Call
 * before the first upload. */
LLMHIP_API int llmhip_model_set_exact_ggml(llmhip_model* m, int on);
/* The fused decode pass: a decode step's layers in one persistent launch
 * whose phases (QKV, attention, output projection, gate/up, down) hand their
 * results to each other through flag-carrying words instead of kernel
 * boundaries (3 dispatches per token with the head and the sampling kernel,
 * against five per layer in the reference, fused.go:259-265).  Taken by every
 * decode step of a model that fits it (finalize decides: head size 64 or 128,
 * embedding <= 1024, feed-forward <= 6144, fused QKV and gate/up groups, f32
 * activations; positions past 256 (head size 64) while 16 chunks of 256 rows
 * of every query head fit the grid, past 128 (head size 128) never), else the
 * steps run one launch per kernel; results agree with
 * the CPU path within the same bounds either way.  on = 0 turns it off, 1 on;
 * poll_limit > 0 makes a hand-off wait give up after that many polls (0: the
 * default, about a second), after which the decode call fails with
 * LLMHIP_ERR_DEVICE and later steps take one launch per kernel.  Returns 1
 * when decode steps take the fused launch, 0 when not (why, if not null,
 * receives the reason, cap bytes at most), < 0 on error. */
LLMHIP_API int llmhip_model_set_fused(llmhip_model* m, int on, uint32_t poll_limit, char* why, uint64_t cap);
/* Run only the first `layers` layers (no head, no sampling; Layers, gpu.go:143-146). 0 = all. */
LLMHIP_API int llmhip_model_set_layers(llmhip_model* m, int layers);
/* Leave kernel classes out of every pass, comma-separated (Skip, gpu.go:769-784):
 * embed, k1, k2, k3, k4, k5, head, argmax, adv, or all; a prefill chunk's activation
 * staging for k1, k3, k4 and k5 also as p1, p3, p4 and p5.  Output is garbage then. */
LLMHIP_API int llmhip_model_set_skip(llmhip_model* m, const char* classes);
/* Average device microseconds of one launch of a kernel of the decode step,
 * launched `iters` times back-to-back on the model's stream between hipEvents
 * with the arguments it has in the decode graph: "head", or "k1".."k5", launch
 * i using layer i % layers (so consecutive launches read different weights).
 * bytes receives its algorithmic bytes per launch (GGUF weight bytes; k2: the
 * KV bytes read at the current position).  It overwrites the activations and
 * the cache row at the current position: run it between generations. */
LLMHIP_API int llmhip_model_bench_kernel(llmhip_model* m, const char* kernel, int iters, float* avg_us,
                                         uint64_t* bytes);
/* One kernel launch timed by llmhip_model_profile. */
typedef struct llmhip_kernel_time {
  char cls[8];    /* embed, k1..k5, head, argmax */
  int32_t layer;  /* -1 outside the layers */
  uint64_t bytes; /* algorithmic bytes: GGUF weight bytes, or KV bytes read (k2) */
  float us;       /* device time between HIP events around the launch */
} llmhip_kernel_time;
/* Run `tokens` decode steps (>= 1) launching each kernel directly, with HIP
 * events recorded on the model's stream around every launch, and return the
 * launches of the last step (at most cap; *n their count).  Advances the
 * model like llmhip_model_decode(tokens).  The times include each launch's
 * dispatch latency (~2-3 us), so they rank kernels; llmhip_model_bench_kernel
 * measures durations. */
LLMHIP_API int llmhip_model_profile(llmhip_model* m, int tokens, llmhip_kernel_time* out, int cap, int* n);
LLMHIP_API void llmhip_model_free(llmhip_model* m);

/* ====================================================================
 * Layer 2: the reference's host package in C++ (llm_*).
 * ==================================================================== */

/* Which error a GGUF parse returned (gguf/gguf.go:29-34 plus I/O). */
enum { LLM_GGUF_OK = 0, LLM_GGUF_MAGIC = 1, LLM_GGUF_VERSION = 2, LLM_GGUF_BOUND = 3, LLM_GGUF_FORMAT = 4,
       LLM_GGUF_IO = 5 };

typedef struct llm_gguf llm_gguf;

/* gguf.Parse (gguf/gguf.go:292-407) of a file or of bytes in memory; *kind is
 * one of LLM_GGUF_*.  Reads the header only, with the reference's bounds. */
LLMHIP_API int llm_gguf_parse_file(const char* path, llm_gguf** out, int* kind);
LLMHIP_API int llm_gguf_parse_bytes(const void* data, uint64_t size, llm_gguf** out, int* kind);
LLMHIP_API void llm_gguf_free(llm_gguf* g);
LLMHIP_API int llm_gguf_info(const llm_gguf* g, uint64_t* ntensors, uint64_t* nkv, uint64_t* data_offset,
                             uint64_t* alignment, uint32_t* version);
LLMHIP_API int llm_gguf_tensor_info(const llm_gguf* g, uint64_t i, char* name, uint64_t name_cap, uint32_t* type,
                                    uint32_t* ndims, uint64_t* dims, uint64_t* offset, uint64_t* size);
LLMHIP_API int llm_gguf_find_tensor(const llm_gguf* g, const char* name, uint64_t* index);
/* File.Uint / Float / Str (gguf/gguf.go:410-432): 1 when present with that kind. */
LLMHIP_API int llm_gguf_meta_uint(const llm_gguf* g, const char* key, uint64_t* v);
LLMHIP_API int llm_gguf_meta_float(const llm_gguf* g, const char* key, double* v);
LLMHIP_API int llm_gguf_meta_str(const llm_gguf* g, const char* key, char* buf, uint64_t cap);
/* ConfigFrom, config.go:29-73. */
LLMHIP_API int llm_config_from(const llm_gguf* g, llmhip_config* out);

/* Package tunables: DecodeBatch (gpu.go:1052, bounded by MaxBatch 16) and
 * PrefillBatch (gpu.go:165), read by the next llm_new_gpu / generate. */
LLMHIP_API int llm_set_decode_batch(int n);
LLMHIP_API int llm_set_prefill_batch(int n);
/* F16KV for the next llm_new_gpu (llmhip_model_set_kv_f16; cpu.go:22-24). */
LLMHIP_API int llm_set_f16kv(int on);
/* ExactGGML for the next llm_new_gpu (llmhip_model_set_exact_ggml; cpu.go:15-21). */
LLMHIP_API int llm_set_exact_ggml(int on);

/* Timing, gpu.go:930-939 (nanoseconds).  record_ns stays 0: the passes are
 * recorded once, as hipGraphs, not per submit. */
typedef struct llm_timing {
  int64_t prefill_ns, decode_ns;
  int64_t prompt_tokens, generated, submits, dispatches;
  int64_t record_ns, submit_ns;
} llm_timing;

/* emit(tok, user) returns nonzero to continue (the emit func of Generate). */
typedef int (*llm_emit_fn)(int32_t tok, void* user);

typedef struct llm_gpu llm_gpu;

/* NewGPU (gpu.go:465-764): parse the file at path, ConfigFrom, create the
 * model and read every tensor straight into pinned staging
 * (llmhip_model_upload_file_tensors). lim NULL: the device's limits. */
LLMHIP_API int llm_new_gpu(int ordinal, const llmhip_limits* lim, const char* path, int ctx, llm_gpu** out);
/* Generate (gpu.go:946-1014). */
LLMHIP_API int llm_gpu_generate(llm_gpu* g, const int32_t* prompt, int n_prompt, int n, int32_t eos, llm_emit_fn emit,
                                void* user, llm_timing* tm);
/* PrefillLogits (gpu.go:904-927): vocab floats of the last prompt token. */
LLMHIP_API int llm_gpu_prefill_logits(llm_gpu* g, const int32_t* prompt, int n_prompt, float* logits);
LLMHIP_API int llm_gpu_peek(llm_gpu* g, const char* name, float* out, uint64_t n);
LLMHIP_API int llm_gpu_config(const llm_gpu* g, llmhip_config* out, int* ctx);
/* The device-layer model (MemoryUsed, Stats, Layers, Skip, bench). */
LLMHIP_API llmhip_model* llm_gpu_model(llm_gpu* g);
LLMHIP_API void llm_gpu_free(llm_gpu* g);

#ifdef __cplusplus
}
#endif
#endif
