//go:build hip

// The forward pass on an AMD MI355X through libllmhip.so (include/llmhip.h),
// behind the same API as the WebGPU gpu.go: NewGPU, Generate, PrefillLogits,
// Peek, MemoryUsed and the Cfg / Stats / Layers / Skip fields.  Go keeps the
// GGUF header (gguf.Parse) and ConfigFrom; only raw tensor bytes cross into
// the library, which repacks them on the device.  Every call copies: C never
// holds a Go pointer after it returns (cgo's pointer rule).

package llm

/*
#cgo CFLAGS: -I${SRCDIR}/third_party/llmhip/include
#cgo LDFLAGS: -L${SRCDIR}/third_party/llmhip/lib -lllmhip -Wl,-rpath,${SRCDIR}/third_party/llmhip/lib
#include <stdlib.h>
#include "llmhip.h"
*/
import "C"

import (
	"errors"
	"fmt"
	"io"
	"os"
	"time"
	"unsafe"

	"github.com/go-wasmcontainers/llm/gguf"
)

// Device is the GPU a model runs on: a HIP device ordinal (the WebGPU build
// takes a *webgpu.Device).
type Device struct {
	Ordinal int
}

// HIPDevice returns device n (0 is the first GPU); the error says "no GPU"
// when there is none, as examples/generate expects.
func HIPDevice(n int) (*Device, error) {
	var cnt C.int
	if rc := C.llmhip_device_count(&cnt); rc != 0 {
		return nil, hipErr(rc)
	}
	if n < 0 || n >= int(cnt) {
		return nil, fmt.Errorf("llm: no GPU %d (%d present)", n, int(cnt))
	}
	return &Device{Ordinal: n}, nil
}

// DeviceLimits are d's own limits from hipDeviceProp_t; MemoryBudget is the
// device's memory.
func DeviceLimits(d *Device) (Limits, error) {
	var cl C.llmhip_limits
	if rc := C.llmhip_device_limits(C.int(d.Ordinal), &cl); rc != 0 {
		return Limits{}, hipErr(rc)
	}
	return Limits{MaxInvocationsPerWorkgroup: uint32(cl.max_invocations_per_workgroup),
		MaxWorkgroupStorage: uint32(cl.max_workgroup_storage), MaxWorkgroupsPerDimension: uint32(cl.max_workgroups_per_dimension),
		MaxStorageBuffers: uint32(cl.max_storage_buffers), MaxBindingSize: uint64(cl.max_binding_size),
		MaxBufferSize: uint64(cl.max_buffer_size), MemoryBudget: uint64(cl.memory_budget)}, nil
}

// GPU is the forward pass on one device (gpu.go:116-159).  Not safe for
// concurrent use.
type GPU struct {
	m     *C.llmhip_model
	Cfg   Config
	ctx   int
	Stats Stats
	// Layers, when non-zero, runs only that many layers (no logits, no
	// sampling; gpu.go:143-146).
	Layers int
	// Skip leaves kernel classes out of every pass, for timing by difference
	// (embed, k1..k5, head, argmax, adv or all; gpu.go:769-784).
	Skip map[string]bool
}

func hipErr(rc C.int) error {
	if rc == 0 {
		return nil
	}
	return errors.New(C.GoString(C.llmhip_last_error()))
}

// NewGPU creates the model on dev and streams every tensor of f from r to it
// (gpu.go:465-764).  ctx <= 0, or above the model's context length, is the
// model's context length.  lim.MemoryBudget, when non-zero, bounds the
// device memory the model allocates.
func NewGPU(dev *Device, lim Limits, f *gguf.File, r io.ReaderAt, ctx int) (*GPU, error) {
	cfg, err := ConfigFrom(f)
	if err != nil {
		return nil, err
	}
	var cl C.llmhip_limits
	if rc := C.llmhip_device_limits(C.int(dev.Ordinal), &cl); rc != 0 {
		return nil, hipErr(rc)
	}
	if lim.MemoryBudget != 0 {
		cl.memory_budget = C.uint64_t(lim.MemoryBudget)
	}
	cc := C.llmhip_config{layers: C.int32_t(cfg.Layers), embd: C.int32_t(cfg.Embd), ff: C.int32_t(cfg.FF),
		heads: C.int32_t(cfg.Heads), kv_heads: C.int32_t(cfg.KVHeads), head_dim: C.int32_t(cfg.HeadDim),
		vocab: C.int32_t(cfg.Vocab), ctx: C.int32_t(cfg.Ctx), rope_base: C.float(cfg.RopeBase), eps: C.float(cfg.Eps),
		arch: C.int32_t(b2i(cfg.Arch == "qwen2")), rope_neox: C.int32_t(b2i(cfg.RopeNeox)),
		bias: C.int32_t(b2i(cfg.Bias)), tied_output: C.int32_t(b2i(cfg.TiedOutput))}
	g := &GPU{Cfg: cfg}
	if rc := C.llmhip_model_create(C.int(dev.Ordinal), &cl, &cc, C.int(ctx), C.int(PrefillBatch), &g.m); rc != 0 {
		return nil, hipErr(rc)
	}
	fail := func(err error) (*GPU, error) {
		g.Close()
		return nil, err
	}
	// the cache format is fixed before the first upload
	if GPUF16KV {
		if rc := C.llmhip_model_set_kv_f16(g.m, 1); rc != 0 {
			return fail(hipErr(rc))
		}
	}
	if GPUExactGGML {
		if rc := C.llmhip_model_set_exact_ggml(g.m, 1); rc != 0 {
			return fail(hipErr(rc))
		}
	}
	var got C.int
	C.llmhip_model_config(g.m, &cc, &got)
	g.ctx = int(got)
	for i := range f.Tensors {
		t := &f.Tensors[i]
		if len(t.Dims) == 0 {
			continue
		}
		name := C.CString(t.Name)
		dims := (*C.uint64_t)(C.malloc(C.size_t(8 * len(t.Dims))))
		for j, d := range t.Dims {
			unsafe.Slice(dims, len(t.Dims))[j] = C.uint64_t(d)
		}
		rc := C.llmhip_model_tensor(g.m, name, C.uint32_t(t.Type), dims, C.uint32_t(len(t.Dims)))
		C.free(unsafe.Pointer(dims))
		C.free(unsafe.Pointer(name))
		if rc != 0 {
			return fail(hipErr(rc))
		}
	}
	if osf, ok := r.(*os.File); ok {
		err = g.uploadFile(osf, f)
	} else {
		err = g.uploadPieces(r, f)
	}
	if err != nil {
		return fail(err)
	}
	if rc := C.llmhip_model_finalize(g.m); rc != 0 {
		return fail(hipErr(rc))
	}
	g.refresh()
	return g, nil
}

// uploadFile hands the library the file descriptor and every tensor's
// offset: it reads runs of consecutive tensors with parallel pread straight
// into pinned staging (no tensor byte passes through Go memory).
func (g *GPU) uploadFile(osf *os.File, f *gguf.File) error {
	n := len(f.Tensors)
	cnames := (**C.char)(C.malloc(C.size_t(n) * C.size_t(unsafe.Sizeof(uintptr(0)))))
	coffs := (*C.uint64_t)(C.malloc(C.size_t(8 * n)))
	names := unsafe.Slice(cnames, n)
	offs := unsafe.Slice(coffs, n)
	for i := range f.Tensors {
		names[i] = C.CString(f.Tensors[i].Name)
		offs[i] = C.uint64_t(f.DataOffset + f.Tensors[i].Offset)
	}
	rc := C.llmhip_model_upload_file_tensors(g.m, C.int(osf.Fd()), C.uint32_t(n), cnames, coffs)
	for _, p := range names {
		C.free(unsafe.Pointer(p))
	}
	C.free(unsafe.Pointer(cnames))
	C.free(unsafe.Pointer(coffs))
	return hipErr(rc)
}

// uploadPieces reads each tensor in PieceSize pieces of whole blocks
// (streamMat's loop, gpu.go:356-389) into C memory and uploads them.
func (g *GPU) uploadPieces(r io.ReaderAt, f *gguf.File) error {
	piece := C.malloc(PieceSize)
	defer C.free(piece)
	buf := unsafe.Slice((*byte)(piece), PieceSize)
	for i := range f.Tensors {
		t := &f.Tensors[i]
		_, bb, ok := t.Type.BlockSize()
		if !ok || bb == 0 {
			bb = 1
		}
		per := uint64(PieceSize) / bb * bb
		name := C.CString(t.Name)
		for a := uint64(0); a < t.Size; a += per {
			n := min(per, t.Size-a)
			if _, err := r.ReadAt(buf[:n], int64(f.DataOffset+t.Offset+a)); err != nil {
				C.free(unsafe.Pointer(name))
				return fmt.Errorf("llm: reading %s: %w", t.Name, err)
			}
			if rc := C.llmhip_model_upload(g.m, name, piece, C.uint64_t(n), C.uint64_t(a)); rc != 0 {
				C.free(unsafe.Pointer(name))
				return hipErr(rc)
			}
		}
		C.free(unsafe.Pointer(name))
	}
	return nil
}

// Close frees every device resource of the model (the WebGPU build leaves
// this to the collector).
func (g *GPU) Close() {
	if g.m != nil {
		C.llmhip_model_free(g.m)
		g.m = nil
	}
}

// MemoryUsed is the device memory the model holds (gpu.go:767).
func (g *GPU) MemoryUsed() uint64 { return uint64(C.llmhip_model_memory_used(g.m)) }

// refresh copies the library's counters into g.Stats.
func (g *GPU) refresh() {
	var s C.llmhip_stats
	C.llmhip_model_stats(g.m, &s)
	g.Stats = Stats{Submits: int(s.submits), Dispatches: int(s.dispatches), Tokens: int(s.tokens)}
}

// apply hands Layers and Skip to the library before a pass.
func (g *GPU) apply() error {
	if rc := C.llmhip_model_set_layers(g.m, C.int(g.Layers)); rc != 0 {
		return hipErr(rc)
	}
	skip := ""
	for k, on := range g.Skip {
		if on {
			skip += k + ","
		}
	}
	cs := C.CString(skip)
	defer C.free(unsafe.Pointer(cs))
	return hipErr(C.llmhip_model_set_skip(g.m, cs))
}

func cIDs(prompt []int32) (*C.int32_t, func()) {
	p := (*C.int32_t)(C.malloc(C.size_t(4 * max(len(prompt), 1))))
	copy(unsafe.Slice((*int32)(unsafe.Pointer(p)), len(prompt)), prompt)
	return p, func() { C.free(unsafe.Pointer(p)) }
}

// PrefillLogits runs the prompt from position 0 and returns the logits of
// its last token (gpu.go:904-927).
func (g *GPU) PrefillLogits(prompt []int32) ([]float32, error) {
	if len(prompt) >= g.ctx {
		return nil, errors.New("llm: prompt longer than the context")
	}
	if err := g.apply(); err != nil {
		return nil, err
	}
	p, done := cIDs(prompt)
	defer done()
	out := (*C.float)(C.malloc(C.size_t(4 * g.Cfg.Vocab)))
	defer C.free(unsafe.Pointer(out))
	rc := C.llmhip_model_prefill(g.m, p, C.int(len(prompt)), out, nil)
	g.refresh()
	if rc != 0 {
		return nil, hipErr(rc)
	}
	return append([]float32(nil), unsafe.Slice((*float32)(unsafe.Pointer(out)), g.Cfg.Vocab)...), nil
}

// Generate decodes greedily (gpu.go:946-1014): the first token comes from
// the prefill, the rest from submits of min(DecodeBatch, remaining) tokens
// sampled on the GPU, each one graph replay per token and one read-back of
// the ids.  emit is called with each token; Generate stops after n tokens, at
// eos (not emitted) or when emit returns false.
func (g *GPU) Generate(prompt []int32, n int, eos int32, emit func(int32) bool) (Timing, error) {
	var tm Timing
	if len(prompt)+n > g.ctx {
		return tm, fmt.Errorf("llm: prompt of %d tokens and %d new tokens exceed the context of %d", len(prompt), n,
			g.ctx)
	}
	if err := g.apply(); err != nil {
		return tm, err
	}
	s0 := g.Stats
	buf := (*C.int32_t)(C.malloc(4 * MaxBatch))
	defer C.free(unsafe.Pointer(buf))
	toks := unsafe.Slice((*int32)(unsafe.Pointer(buf)), MaxBatch)
	p, done := cIDs(prompt)
	defer done()
	t0 := time.Now()
	if rc := C.llmhip_model_prefill(g.m, p, C.int(len(prompt)), nil, buf); rc != 0 {
		g.refresh()
		return tm, hipErr(rc)
	}
	tm.Prefill, tm.PromptTokens = time.Since(t0), len(prompt)
	t1 := time.Now()
	have := 1 // ids in toks not yet emitted
	for produced := 0; produced < n; {
		for j := 0; j < have && produced < n; j++ {
			if toks[j] == eos {
				n = produced
				break
			}
			tm.Generated++
			produced++
			if !emit(toks[j]) {
				n = produced
				break
			}
		}
		if produced >= n {
			break
		}
		have = min(max(1, min(DecodeBatch, MaxBatch)), n-produced)
		ts := time.Now()
		if rc := C.llmhip_model_decode(g.m, C.int(have), buf); rc != 0 {
			g.refresh()
			return tm, hipErr(rc)
		}
		tm.Submit += time.Since(ts)
	}
	tm.Decode = time.Since(t1)
	g.refresh()
	tm.Submits, tm.Dispatches = g.Stats.Submits-s0.Submits, g.Stats.Dispatches-s0.Dispatches
	return tm, nil
}

// Peek reads the first n 4-byte words of a named buffer as float32
// (gpu.go:1018-1043): x, h, q, k, v, att, gate, up, logits, state, tokens,
// outb, and kvblk.N. (layer N's cache).  For tests and traces, never in the
// decode loop.
func (g *GPU) Peek(name string, n int) ([]float32, error) {
	cs := C.CString(name)
	defer C.free(unsafe.Pointer(cs))
	out := (*C.float)(C.malloc(C.size_t(4 * max(n, 1))))
	defer C.free(unsafe.Pointer(out))
	rc := C.llmhip_model_peek(g.m, cs, out, C.uint64_t(n))
	g.refresh()
	if rc != 0 {
		return nil, hipErr(rc)
	}
	return append([]float32(nil), unsafe.Slice((*float32)(unsafe.Pointer(out)), n)...), nil
}
