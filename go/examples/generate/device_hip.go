//go:build hip

// How examples/generate obtains its GPU in the hip build: device 0 through
// libllmhip.so, with the device's own limits.  The WebGPU build keeps the
// batchsink code of main.go:81-96 in device_webgpu.go (//go:build !hip);
// main.go calls openGPU in their place (a two-line edit of main.go).

package main

import (
	"fmt"
	"io"
	"os"

	llm "github.com/go-wasmcontainers/llm"
	"github.com/go-wasmcontainers/llm/gguf"
)

// openGPU prints the limits line and loads the model; with no GPU it prints
// "no GPU" and exits 2, as main.go:81-85 does.  The returned func releases
// the device resources.
func openGPU(f *gguf.File, r io.ReaderAt, ctx int) (*llm.GPU, llm.Limits, func(), error) {
	dev, err := llm.HIPDevice(0)
	if err != nil {
		fmt.Println("no GPU:", err)
		os.Exit(2)
	}
	lim, err := llm.DeviceLimits(dev)
	if err != nil {
		return nil, lim, nil, err
	}
	fmt.Printf("limits: workgroup size %d, %d invocations, %d B shared, %d groups/dim, binding %d, memory %d\n",
		lim.WorkgroupSize(), lim.MaxInvocationsPerWorkgroup, lim.MaxWorkgroupStorage, lim.MaxWorkgroupsPerDimension,
		lim.MaxBindingSize, lim.MemoryBudget)
	g, err := llm.NewGPU(dev, lim, f, r, ctx)
	if err != nil {
		return nil, lim, nil, err
	}
	return g, lim, g.Close, nil
}
