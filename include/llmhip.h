/*
 * llmhip.h — the C-ABI of the MI355X (gfx950) forward pass for llama / qwen2
 * GGUF models: the drop-in for the GPU half of go-wasmcontainers/llm.
 *
 * Two layers, both plain C (pointers, sizes, status codes; no C++ or torch
 * types):
 *
 *  1. llmhip_*  — the device layer.  This is what the Go package's cgo wrapper
 *     binds (its NewGPU keeps parsing the GGUF header and ConfigFrom in Go and
 *     streams raw tensor bytes in).  It replaces the
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
LLMHIP_API void llmhip_qmat_free(llmhip_qmat* m);

#ifdef __cplusplus
}
#endif
#endif
