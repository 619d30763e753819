//go:build windows

// libgtmoe is built for Linux (ROCm) only: on Windows the GPU branch of
// Forward always answers on the CPU.  Not compiled here (no Go toolchain in
// the environment this was written in).
package mixtureofexperts

import (
	"errors"

	"github.com/javanhut/GoTransformers/vectormath"
)

// UseGPU reports that no MI355X library exists on this platform.
func UseGPU(device int) error {
	return errors.New("gtmoe: libgtmoe is not available on Windows")
}

// CloseGPU does nothing on this platform.
func CloseGPU() {}

// LastGPUError is always nil on this platform.
func (mixture *MixtureOfExperts) LastGPUError() error { return nil }

func (mixture *MixtureOfExperts) forwardOnGPU(inputs vectormath.Matrix, tokenIDs []int) (vectormath.Matrix, bool) {
	return vectormath.Matrix{}, false
}
