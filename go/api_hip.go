//go:build hip

// The package-level API that gpu.go and fused.go declare for the WebGPU build,
// declared again for the hip build (those two files, and kernels.go and
// kernels_fused.go, carry `//go:build !hip`).  Names, types and default values
// are the reference's, so callers (examples/generate) compile unchanged; the
// tunables the HIP forward pass has no use for are kept as no-ops and say so.

package llm

import "time"

// ChunkSize is the largest single upload of the WebGPU loader (gpu.go:20).
// The HIP loader stages 8 MiB runs of its own; the value is kept for callers.
const ChunkSize = 16 << 20

// PieceSize is the size of one read from the model file while loading
// (gpu.go:23): NewGPU reads a non-file io.ReaderAt in pieces of this size.
const PieceSize = 4 << 20

// Limits are the device limits a model is created against (gpu.go:28-36).
// On HIP the kernels take raw pointers and pick their own launch shapes, so
// only MemoryBudget is enforced (every device allocation of a model counts
// against it); DeviceLimits fills the rest from hipDeviceProp_t.
type Limits struct {
	MaxInvocationsPerWorkgroup uint32
	MaxWorkgroupStorage        uint32 // bytes
	MaxWorkgroupsPerDimension  uint32
	MaxStorageBuffers          uint32
	MaxBindingSize             uint64
	MaxBufferSize              uint64
	MemoryBudget               uint64 // device memory the model may hold
}

// DefaultLimits are the WebGPU guaranteed minimum the reference defaults to
// (gpu.go:39-41), kept value for value; a HIP caller usually wants
// DeviceLimits instead (its MemoryBudget is the device's memory).
func DefaultLimits() Limits {
	return Limits{MaxInvocationsPerWorkgroup: 256, MaxWorkgroupStorage: 16384, MaxWorkgroupsPerDimension: 65535,
		MaxStorageBuffers: 8, MaxBindingSize: 128 << 20, MaxBufferSize: 256 << 20, MemoryBudget: 256 << 20}
}

// WorkgroupSize is the reference's reduction width for these limits
// (gpu.go:47-53): 64, halved while the invocation or workgroup-memory limit is
// below it.  Informational on HIP, where every kernel runs 64-wide waves.
func (l Limits) WorkgroupSize() int {
	wg := 64
	for wg > 1 && (uint32(wg) > l.MaxInvocationsPerWorkgroup || uint32(8*wg) > l.MaxWorkgroupStorage) {
		wg >>= 1
	}
	return wg
}

// Stats counts what a model did (gpu.go:56-60): submits are graph launches
// and synchronising calls, dispatches are kernel launches.
type Stats struct {
	Submits    int
	Dispatches int
	Tokens     int
}

// Timing of a generation (gpu.go:930-939).  Record stays zero on HIP: the
// passes are captured once as hipGraphs, not recorded per submit.
type Timing struct {
	Prefill, Decode time.Duration
	PromptTokens    int
	Generated       int
	Submits         int
	Dispatches      int
	Record, Submit  time.Duration
}

// PrefillBatch is the number of prompt tokens one pass processes (gpu.go:165):
// read by NewGPU, at most 64.
var PrefillBatch = 64

// NoFused selected the reference's unfused kernels for A/B runs (gpu.go:168).
// The HIP pass has one form; the flag is accepted and ignored.
var NoFused bool

// TPR was the invocations per output row of the WebGPU matrix-vector kernels
// (fused.go:17).  The HIP kernels map 16-row tiles onto 64-wide waves; the
// value is accepted and ignored.
var TPR = 8

// PrefillChunk is the prompt chunk of the reference's unfused path
// (gpu.go:851).  The HIP pass always runs PrefillBatch-token chunks.
const PrefillChunk = 8

// MaxBatch bounds DecodeBatch (gpu.go:1046).
const MaxBatch = 16

// DecodeBatch is the number of tokens one decode submit computes
// (gpu.go:1052): one llmhip_model_decode call, one read-back of the ids.
var DecodeBatch = 8

// GPUF16KV stores the KV cache in binary16, each element rounded to nearest
// even at the append, as the CPU model's F16KV does (cpu.go:22-24, 298-299).
// Read by NewGPU; results then match the CPU path with F16KV set.
var GPUF16KV bool

// GPUExactGGML selects the numerics of the CPU model's ExactGGML
// (cpu.go:15-21): matrix inputs quantised to Q8_0 / Q8_1 blocks, ggml's
// integer block products, a binary16 cache.  Read by NewGPU.
var GPUExactGGML bool

func b2i(b bool) int {
	if b {
		return 1
	}
	return 0
}
