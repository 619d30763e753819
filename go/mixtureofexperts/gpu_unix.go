//go:build !windows

// The GPU branch of MixtureOfExperts.Forward: libgtmoe (include/gtmoe.h), the
// MI355X implementation of this package's forward pass, loaded at run time
// with purego so the build stays CGO_ENABLED=0, the way gpu/library_unix.go
// loads Vulkan.
//
// The file goes into package mixtureofexperts beside mixtureofexperts.go,
// with gpu_windows.go.  The one change outside these files is two lines at
// the head of Forward (mixtureofexperts/mixtureofexperts.go, after the
// argument checks that end at line 134, before the routing):
//
//	if outputs, ok := mixture.forwardOnGPU(inputs, tokenIDs); ok {
//		return outputs
//	}
//
// Forward keeps its checks and panics ahead of the branch; libgtmoe repeats
// them and answers GTMOE_ERR_INVALID_ARGUMENT.  A process opts in with
// UseGPU(device).  A mixture then runs on the GPU when its experts are
// compressed at lowprecision.Float32, Int8 or FP4 (one precision for all),
// are SwiGLU or clamped SwiGLU, and carry no low-rank adapters; any other
// mixture, any failure to load or open, and any non-zero status answers on
// the CPU, with the error kept for LastGPUError, as gpu.Device's
// multiplyOrUseCPU does (gpu/device.go:722-739).  Weights are uploaded from
// the layers' Rows snapshots on the first GPU forward of a mixture and again
// whenever vectormath.WeightsVersion() has moved since (the reference's own
// signal that weights changed, vectormath/weights.go:13-21).  A mixture's
// device copy lives until ReleaseGPU, CloseGPU, or the first GPU forward
// after the mixture itself was garbage-collected (the table below holds it
// by a weak pointer).
//
// This file has not been compiled: the environment it was written in has no
// Go toolchain.  tests/test_go_binding.py checks its struct layouts against
// include/gtmoe.h with a C program built by gcc, and every entry point it
// registers against the header.
package mixtureofexperts

import (
	"errors"
	"fmt"
	"os"
	"sync"
	"unsafe"
	"weak"

	"github.com/ebitengine/purego"
	"github.com/javanhut/GoTransformers/activationfunction"
	"github.com/javanhut/GoTransformers/feedforward"
	"github.com/javanhut/GoTransformers/lowprecision"
	"github.com/javanhut/GoTransformers/perceptron"
	"github.com/javanhut/GoTransformers/vectormath"
)

// Status codes, precisions and roles of include/gtmoe.h.
const (
	gtmoeOK = 0

	gtmoeFloat64 = 0
	gtmoeFloat32 = 1
	gtmoeInt8    = 2
	gtmoeFP4     = 3

	gtmoeRoleRouter      = 0
	gtmoeRoleSharedGate  = 1
	gtmoeRoleRoutedGate  = 4
	gtmoeRolesPerExpert  = 3 // gate, up, down follow each other
	gtmoePathAuto uint32 = 0
)

// gtmoeLayerDesc is gtmoe_layer_desc: eight int32 then a double (40 bytes).
type gtmoeLayerDesc struct {
	VectorSize       int32
	ExpertHiddenSize int32
	SharedExperts    int32
	RoutedExperts    int32
	ExpertsPerToken  int32
	Precision        int32
	UseHashRouting   int32
	Reserved         int32
	ClampLimit       float64
}

// gtmoeRows is gtmoe_rows: four int32, then pointer, size, pointer, size
// (48 bytes on 64-bit targets).
type gtmoeRows struct {
	Precision   int32
	Rows        int32
	Width       int32
	Reserved    int32
	Values      unsafe.Pointer
	ValuesBytes uintptr
	Scales      unsafe.Pointer
	ScaleCount  uintptr
}

var (
	libraryOnce  sync.Once
	libraryError error

	gtmoeOpen             func(device int32, context *uintptr) int32
	gtmoeContextFree      func(context uintptr) int32
	gtmoeLastError        func(context uintptr) string
	gtmoeLayerCreate      func(context uintptr, desc *gtmoeLayerDesc, layer *uintptr) int32
	gtmoeLayerDestroy     func(layer uintptr) int32
	gtmoeUploadRows       func(layer uintptr, role int32, index int32, rows *gtmoeRows, biases *float64) int32
	gtmoeSetBalanceBiases func(layer uintptr, biases *float64) int32
	gtmoeForward          func(layer uintptr, tokens int32, inputs *float64, tokenIDs *int64, outputs *float64, flags uint32) int32
	gtmoeLastRouting      func(layer uintptr, tokens *int32, chosen *int32, gates *float64, load *int32, rowsForExpert *int32, offsets *int32) int32
)

// libgtmoeNames lists where the library is looked for: GTMOE_LIBRARY when
// set, then the loader's search path.
func libgtmoeNames() []string {
	names := []string{"libgtmoe.so", "libgtmoe.so.1"}
	if path := os.Getenv("GTMOE_LIBRARY"); path != "" {
		names = append([]string{path}, names...)
	}
	return names
}

func loadLibrary() error {
	libraryOnce.Do(func() {
		var library uintptr
		var lastError error
		for _, name := range libgtmoeNames() {
			handle, err := purego.Dlopen(name, purego.RTLD_NOW|purego.RTLD_GLOBAL)
			if err == nil {
				library = handle
				break
			}
			lastError = err
		}
		if library == 0 {
			libraryError = fmt.Errorf("could not find libgtmoe (tried %v): %w", libgtmoeNames(), lastError)
			return
		}
		functions := map[string]any{
			"gtmoe_open":               &gtmoeOpen,
			"gtmoe_context_free":       &gtmoeContextFree,
			"gtmoe_last_error":         &gtmoeLastError,
			"gtmoe_layer_create":       &gtmoeLayerCreate,
			"gtmoe_layer_destroy":      &gtmoeLayerDestroy,
			"gtmoe_upload_rows":        &gtmoeUploadRows,
			"gtmoe_set_balance_biases": &gtmoeSetBalanceBiases,
			"gtmoe_forward":            &gtmoeForward,
			"gtmoe_last_routing":       &gtmoeLastRouting,
		}
		for name, function := range functions {
			address, err := purego.Dlsym(library, name)
			if err != nil || address == 0 {
				libraryError = fmt.Errorf("libgtmoe is missing %s", name)
				return
			}
			purego.RegisterFunc(function, address)
		}
	})
	return libraryError
}

// gpuState is what the GPU keeps for one mixture.
type gpuState struct {
	layer          uintptr
	desc           gtmoeLayerDesc
	weightsVersion uint64
	lastError      error
}

// deviceLock serialises every call into libgtmoe, as gpu.Device's lock does
// (gpu/device.go:40); a MixtureOfExperts itself has no lock.  gpuStates is
// keyed by weak pointers, so it keeps no mixture alive: the device layers of
// mixtures that were collected are freed by the next GPU forward.
var (
	deviceLock    sync.Mutex
	deviceContext uintptr
	gpuStates     = map[weak.Pointer[MixtureOfExperts]]*gpuState{}
)

// releaseState frees one table entry's device layer (deviceLock held).
func releaseState(key weak.Pointer[MixtureOfExperts]) {
	if state := gpuStates[key]; state != nil {
		if state.layer != 0 {
			gtmoeLayerDestroy(state.layer)
		}
		delete(gpuStates, key)
	}
}

// releaseCollected frees the device layers of mixtures the garbage
// collector has taken (deviceLock held).
func releaseCollected() {
	for key := range gpuStates {
		if key.Value() == nil {
			releaseState(key)
		}
	}
}

// ReleaseGPU frees this mixture's device layer (its weights in HBM) now; a
// later GPU forward uploads them again.  Mixtures that are simply dropped
// have theirs freed by the next GPU forward of any mixture.
func (mixture *MixtureOfExperts) ReleaseGPU() {
	deviceLock.Lock()
	defer deviceLock.Unlock()
	releaseState(weak.Make(mixture))
}

// UseGPU opens GPU `device` for every MixtureOfExperts of the process
// (gpu.Open's counterpart, gpu/device.go:90-130).  Without the library or
// the device it returns the reason and Forward stays on the CPU.
func UseGPU(device int) error {
	deviceLock.Lock()
	defer deviceLock.Unlock()
	if deviceContext != 0 {
		return nil
	}
	if err := loadLibrary(); err != nil {
		return err
	}
	var context uintptr
	if status := gtmoeOpen(int32(device), &context); status != gtmoeOK {
		return fmt.Errorf("gtmoe: opening GPU %d: %s (status %d)", device, gtmoeLastError(0), status)
	}
	deviceContext = context
	return nil
}

// CloseGPU frees every mixture's device layer and the context (Device.Close);
// Forward answers on the CPU afterwards.
func CloseGPU() {
	deviceLock.Lock()
	defer deviceLock.Unlock()
	if deviceContext == 0 {
		return
	}
	for key := range gpuStates {
		releaseState(key)
	}
	gtmoeContextFree(deviceContext)
	deviceContext = 0
}

// LastGPUError is the failure after which this mixture's last GPU attempt
// answered on the CPU (Device.LastError, gpu/device.go:749-753), or nil.
func (mixture *MixtureOfExperts) LastGPUError() error {
	deviceLock.Lock()
	defer deviceLock.Unlock()
	if state := gpuStates[weak.Make(mixture)]; state != nil {
		return state.lastError
	}
	return nil
}

// forwardOnGPU is the branch at the head of Forward.  ok is false when the
// mixture does not run on the GPU or the GPU failed; Forward then continues
// on the CPU.
func (mixture *MixtureOfExperts) forwardOnGPU(inputs vectormath.Matrix, tokenIDs []int) (vectormath.Matrix, bool) {
	deviceLock.Lock()
	defer deviceLock.Unlock()
	if deviceContext == 0 {
		return vectormath.Matrix{}, false
	}
	desc, eligible := mixture.gpuDesc()
	if !eligible {
		return vectormath.Matrix{}, false
	}
	releaseCollected()
	key := weak.Make(mixture)
	state := gpuStates[key]
	if state == nil {
		state = &gpuState{}
		gpuStates[key] = state
	}
	fail := func(err error) (vectormath.Matrix, bool) {
		state.lastError = err
		return vectormath.Matrix{}, false
	}
	if err := mixture.ensureUploaded(state, desc); err != nil {
		return fail(err)
	}
	// BalanceBiases change on this side (UpdateBalance): hand them over on
	// every forward (E float64 values)
	if status := gtmoeSetBalanceBiases(state.layer, &mixture.BalanceBiases[0]); status != gtmoeOK {
		return fail(deviceError("setting the balance biases", status))
	}
	tokens := inputs.Rows
	outputs := vectormath.NewMatrix(tokens, inputs.Columns)
	var ids *int64
	if mixture.UseHashRouting && tokens > 0 {
		converted := make([]int64, tokens)
		for i, id := range tokenIDs {
			converted[i] = int64(id)
		}
		ids = &converted[0]
	}
	var x, y *float64
	if tokens > 0 {
		x, y = &inputs.Values[0], &outputs.Values[0]
	}
	if status := gtmoeForward(state.layer, int32(tokens), x, ids, y, gtmoePathAuto); status != gtmoeOK {
		return fail(deviceError("forward", status))
	}
	if err := mixture.copyRoutingFromGPU(state, tokens); err != nil {
		return fail(err)
	}
	state.lastError = nil
	return outputs, true
}

func deviceError(what string, status int32) error {
	return fmt.Errorf("gtmoe: %s: %s (status %d)", what, gtmoeLastError(deviceContext), status)
}

// gpuDesc is the device layer's shape, and whether this mixture can run on
// the GPU at all.
func (mixture *MixtureOfExperts) gpuDesc() (gtmoeLayerDesc, bool) {
	experts := append(append([]*feedforward.GatedFeedForward{}, mixture.SharedExperts...), mixture.RoutedExperts...)
	if len(experts) == 0 || mixture.RouterLayer.Adapter != nil {
		return gtmoeLayerDesc{}, false
	}
	first := experts[0].GateLayer
	if !first.IsCompressed() {
		return gtmoeLayerDesc{}, false
	}
	precision := first.CompressedWeights.Precision
	if precision != lowprecision.Float32 && precision != lowprecision.Int8 && precision != lowprecision.FP4 {
		return gtmoeLayerDesc{}, false
	}
	clamp, ok := clampLimit(first.Activation, experts[0].UpLayer.Activation)
	if !ok {
		return gtmoeLayerDesc{}, false
	}
	for _, expert := range experts {
		for _, layer := range []*perceptron.Layer{expert.GateLayer, expert.UpLayer, expert.DownLayer} {
			if !layer.IsCompressed() || layer.CompressedWeights.Precision != precision || layer.Adapter != nil {
				return gtmoeLayerDesc{}, false
			}
		}
		if limit, same := clampLimit(expert.GateLayer.Activation, expert.UpLayer.Activation); !same || limit != clamp {
			return gtmoeLayerDesc{}, false
		}
	}
	hash := int32(0)
	if mixture.UseHashRouting {
		hash = 1
	}
	return gtmoeLayerDesc{
		VectorSize:       int32(mixture.VectorSize()),
		ExpertHiddenSize: int32(experts[0].GateLayer.NumberOfOutputs()),
		SharedExperts:    int32(len(mixture.SharedExperts)),
		RoutedExperts:    int32(len(mixture.RoutedExperts)),
		ExpertsPerToken:  int32(mixture.ExpertsPerToken),
		Precision:        int32(precision),
		UseHashRouting:   hash,
		ClampLimit:       clamp,
	}, true
}

// clampLimit reads the SwiGLU variant from the activations: SiLU and Linear
// (limit 0), or ClampedSiLU(L) and ClampedLinear(L)
// (activationfunction/moreactivationfunctions.go:207-244).
func clampLimit(gate activationfunction.Activation, up activationfunction.Activation) (float64, bool) {
	if gate.Name == activationfunction.SiLU.Name && up.Name == activationfunction.Linear.Name {
		return 0, true
	}
	var gateLimit, upLimit float64
	if _, err := fmt.Sscanf(gate.Name, "ClampedSiLU(%g)", &gateLimit); err != nil {
		return 0, false
	}
	if _, err := fmt.Sscanf(up.Name, "ClampedLinear(%g)", &upLimit); err != nil {
		return 0, false
	}
	return gateLimit, gateLimit == upLimit && gateLimit > 0
}

// ensureUploaded creates the device layer on first use and uploads every
// weight matrix and bias whenever the weights version moved since the last
// upload (or the shape changed).
func (mixture *MixtureOfExperts) ensureUploaded(state *gpuState, desc gtmoeLayerDesc) error {
	version := vectormath.WeightsVersion()
	if state.layer != 0 && state.desc == desc && state.weightsVersion == version {
		return nil
	}
	if state.layer != 0 && state.desc != desc {
		gtmoeLayerDestroy(state.layer)
		state.layer = 0
	}
	if state.layer == 0 {
		var layer uintptr
		if status := gtmoeLayerCreate(deviceContext, &desc, &layer); status != gtmoeOK {
			return deviceError("creating the layer", status)
		}
		state.layer = layer
		state.desc = desc
	}
	for kind, experts := range [][]*feedforward.GatedFeedForward{mixture.SharedExperts, mixture.RoutedExperts} {
		firstRole := int32(gtmoeRoleSharedGate)
		if kind == 1 {
			firstRole = gtmoeRoleRoutedGate
		}
		for index, expert := range experts {
			for offset, layer := range []*perceptron.Layer{expert.GateLayer, expert.UpLayer, expert.DownLayer} {
				if status := uploadCompressed(state.layer, firstRole+int32(offset), int32(index), layer); status != gtmoeOK {
					return deviceError(fmt.Sprintf("uploading %s", layer.Name), status)
				}
			}
		}
	}
	if !mixture.UseHashRouting {
		if status := uploadRouter(state.layer, mixture.RouterLayer); status != gtmoeOK {
			return deviceError("uploading the router", status)
		}
	}
	state.weightsVersion = version
	return nil
}

// uploadCompressed hands one compressed layer over from its RowsSnapshot
// arrays (lowprecision/rows.go:148-170), unchanged.
func uploadCompressed(layer uintptr, role int32, index int32, source *perceptron.Layer) int32 {
	snapshot := source.CompressedWeights.Snapshot()
	view := gtmoeRows{Precision: int32(snapshot.Precision), Rows: int32(snapshot.NumberOfRows), Width: int32(snapshot.Width)}
	switch snapshot.Precision {
	case lowprecision.Int8:
		if len(snapshot.Int8Values) > 0 {
			view.Values, view.ValuesBytes = unsafe.Pointer(&snapshot.Int8Values[0]), uintptr(len(snapshot.Int8Values))
		}
	case lowprecision.FP4:
		if len(snapshot.FP4Values) > 0 {
			view.Values, view.ValuesBytes = unsafe.Pointer(&snapshot.FP4Values[0]), uintptr(len(snapshot.FP4Values))
		}
	case lowprecision.Float32:
		if len(snapshot.Float32Values) > 0 {
			view.Values, view.ValuesBytes = unsafe.Pointer(&snapshot.Float32Values[0]), uintptr(4*len(snapshot.Float32Values))
		}
	}
	if len(snapshot.Scales) > 0 {
		view.Scales, view.ScaleCount = unsafe.Pointer(&snapshot.Scales[0]), uintptr(len(snapshot.Scales))
	}
	return gtmoeUploadRows(layer, role, index, &view, &source.Biases[0])
}

// uploadRouter hands the router over: its compressed rows when it has them
// (the model-level compression of transformer/model.go:78-82), its float64
// weights otherwise.
func uploadRouter(layer uintptr, router *perceptron.Layer) int32 {
	if router.IsCompressed() {
		return uploadCompressed(layer, gtmoeRoleRouter, 0, router)
	}
	weights := router.Weights.Values
	view := gtmoeRows{Precision: gtmoeFloat64, Rows: int32(router.Weights.Rows), Width: int32(router.Weights.Columns)}
	if len(weights) > 0 {
		view.Values, view.ValuesBytes = unsafe.Pointer(&weights[0]), uintptr(8*len(weights))
	}
	return gtmoeUploadRows(layer, gtmoeRoleRouter, 0, &view, &router.Biases[0])
}

// copyRoutingFromGPU fills the forward-state cache (mixtureofexperts.go:207-214)
// from the device's routing of the last forward: chosen experts, gates,
// rowsForExpert and the load, which LastExpertLoad, UpdateBalance and
// Backward read.  The router logits, affinities and expert outputs stay on
// the device; a mixture on the GPU has no adapters, so its Backward stops at
// the compressed experts' own panic (perceptron/layer.go:165-166) before it
// would read them.
func (mixture *MixtureOfExperts) copyRoutingFromGPU(state *gpuState, tokens int) error {
	k, experts := mixture.ExpertsPerToken, mixture.NumberOfRoutedExperts()
	chosen := make([]int32, tokens*k+1)
	gates := make([]float64, tokens*k+1)
	load := make([]int32, experts)
	rows := make([]int32, tokens*k+1)
	offsets := make([]int32, experts+1)
	var got int32
	if status := gtmoeLastRouting(state.layer, &got, &chosen[0], &gates[0], &load[0], &rows[0], &offsets[0]); status != gtmoeOK {
		return deviceError("reading the routing", status)
	}
	if int(got) != tokens {
		return errors.New("gtmoe: the routing read back is for another forward")
	}
	chosenExperts := make([][]int, tokens)
	tokenGates := make([][]float64, tokens)
	for token := range tokens {
		chosenExperts[token] = make([]int, k)
		tokenGates[token] = make([]float64, k)
		for i := range k {
			chosenExperts[token][i] = int(chosen[token*k+i])
			tokenGates[token][i] = gates[token*k+i]
		}
	}
	rowsForExpert := make([][]int, experts)
	expertLoad := make([]int, experts)
	for expert := range experts {
		expertLoad[expert] = int(load[expert])
		for _, token := range rows[offsets[expert]:offsets[expert+1]] {
			rowsForExpert[expert] = append(rowsForExpert[expert], int(token))
		}
	}
	mixture.lastNumberOfTokens = tokens
	mixture.lastRouterLogits = vectormath.Matrix{}
	mixture.lastAffinities = vectormath.Matrix{}
	mixture.lastChosenExperts = chosenExperts
	mixture.lastGates = tokenGates
	mixture.lastRowsForExpert = rowsForExpert
	mixture.lastExpertOutputs = nil
	mixture.lastExpertLoad = expertLoad
	return nil
}
