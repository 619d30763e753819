/*
 * gtmoe.h -- C ABI of libgtmoe, the MI355X (gfx950) implementation of
 * GoTransformers' mixture-of-experts forward pass over lowprecision expert
 * weights.
 *
 * The ABI is plain C: opaque handles, plain pointers and sizes, int32 status
 * codes.  A CGO_ENABLED=0 Go host binds it with purego Dlopen/Dlsym/
 * RegisterFunc, the way gpu/library_unix.go:19-33 and gpu/vulkan.go:443-519
 * bind Vulkan.  Every call that takes host buffers copies what it needs and
 * blocks until its results are back in host memory (the contract of
 * gpu/device.go:636-654).  Calls on one context are serialised by a mutex
 * (gpu/device.go:40); a layer must not be used from two threads at once,
 * just as mixtureofexperts.MixtureOfExperts has no lock.
 *
 * Status codes: 0 is success.  On failure the call returns a non-zero code
 * and gtmoe_last_error() describes it; the Go side then answers on the CPU
 * and records the error, as gpu/device.go:723-739 does for Vulkan.
 */
#ifndef GTMOE_H
#define GTMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GTMOE_ABI_VERSION 1

enum gtmoe_status {
    GTMOE_OK = 0,
    GTMOE_ERR_INVALID_ARGUMENT = 1, /* the reference would panic */
    GTMOE_ERR_UNSUPPORTED = 2,      /* valid for the reference, not offered on the GPU */
    GTMOE_ERR_DEVICE = 3,           /* a HIP call failed */
    GTMOE_ERR_NOT_READY = 4,        /* weights missing, or no Forward yet */
    GTMOE_ERR_OUT_OF_MEMORY = 5
};

/* lowprecision.Precision (lowprecision/lowprecision.go:9-16) */
enum gtmoe_precision { GTMOE_FLOAT64 = 0, GTMOE_FLOAT32 = 1, GTMOE_INT8 = 2, GTMOE_FP4 = 3 };

/* Which weight matrix an upload fills.  Gate, Up and Down are the three
 * perceptron.Layers of feedforward.GatedFeedForward
 * (feedforward/gatedfeedforward.go:11-19); ROUTER is
 * MixtureOfExperts.RouterLayer (mixtureofexperts/mixtureofexperts.go:19). */
enum gtmoe_role {
    GTMOE_ROLE_ROUTER = 0,
    GTMOE_ROLE_SHARED_GATE = 1,
    GTMOE_ROLE_SHARED_UP = 2,
    GTMOE_ROLE_SHARED_DOWN = 3,
    GTMOE_ROLE_ROUTED_GATE = 4,
    GTMOE_ROLE_ROUTED_UP = 5,
    GTMOE_ROLE_ROUTED_DOWN = 6
};

/* Forward flags: which expert kernels run.  AUTO takes the fp32 dequant-GEMV
 * path while tokens per expert are few (decode) and the bf16 MFMA grouped GEMM
 * otherwise (prefill).  FP32 and BF16 force one path. */
enum gtmoe_path { GTMOE_PATH_AUTO = 0, GTMOE_PATH_FP32 = 1, GTMOE_PATH_BF16 = 2 };

typedef struct gtmoe_context gtmoe_context;
typedef struct gtmoe_layer gtmoe_layer;
typedef struct gtmoe_graph gtmoe_graph;
typedef struct gtmoe_weights_file gtmoe_weights_file;

/* The shape of one MixtureOfExperts.  Mirrors the arguments of
 * NewMixtureOfExperts / NewClampedMixtureOfExperts
 * (mixtureofexperts/mixtureofexperts.go:33-45) plus the fields
 * UseHashRouting (:16) and the expert weight precision
 * (transformer.Settings.WeightPrecision, transformer/settings.go:23). */
typedef struct gtmoe_layer_desc {
    int32_t vector_size;        /* d: RouterLayer.NumberOfInputs() */
    int32_t expert_hidden_size; /* h */
    int32_t shared_experts;     /* S >= 0 */
    int32_t routed_experts;     /* E in [1, 256] */
    int32_t experts_per_token;  /* k in [1, min(E, 8)] */
    int32_t precision;          /* expert weights: GTMOE_FLOAT32, GTMOE_INT8 or GTMOE_FP4
                                   (FLOAT32 rows also keep a bf16 copy on the device, for the
                                   many-token path: 6 bytes per weight in all) */
    int32_t use_hash_routing;   /* MixtureOfExperts.UseHashRouting */
    int32_t reserved;
    double clamp_limit;         /* > 0: clamped SwiGLU (feedforward.NewClampedSwiGLU); 0: SwiGLU */
} gtmoe_layer_desc;

/* One weight matrix in the reference's Rows storage (lowprecision/rows.go:8-18,
 * RowsSnapshot at :148-170): `rows` output neurons of `width` inputs.
 *   FLOAT64  values = double[rows*width]
 *   FLOAT32  values = float[rows*width]
 *   INT8     values = int8_t[rows*width], scales = float[rows*ceil(width/16)]
 *   FP4      values = uint8_t[rows*ceil(width/2)] (even index in the low
 *            nibble), scales = float[rows*ceil(width/16)]
 * values_bytes and scale_count are the lengths of the two arrays and are
 * checked like RowsFromSnapshot (rows.go:172-203). */
typedef struct gtmoe_rows {
    int32_t precision;
    int32_t rows;
    int32_t width;
    int32_t reserved;
    const void *values;
    size_t values_bytes;
    const float *scales;
    size_t scale_count;
} gtmoe_rows;

/* ---- library and context -------------------------------------------------
 * gtmoe_open replaces the device bring-up of gpu.Open/openDevice
 * (gpu/device.go:90-130); without a gfx950 device it fails (GTMOE_ERR_DEVICE
 * or GTMOE_ERR_UNSUPPORTED, text in gtmoe_last_error(NULL)) and the caller
 * answers on the CPU.  gtmoe_close replaces Device.Close: it waits for the
 * device and releases the context's stream and events, but the handle stays
 * readable, as a closed gpu.Device does (gpu/device.go:729-731,
 * gpu/gpu_test.go:145-154): a second gtmoe_close does nothing, any other call
 * on the context or its layers answers GTMOE_ERR_INVALID_ARGUMENT with "the
 * context is closed" in gtmoe_last_error, and gtmoe_layer_destroy still frees
 * a layer.  A closed context's own few hundred bytes stay allocated until
 * gtmoe_context_free. */
int32_t gtmoe_abi_version(void);
int32_t gtmoe_device_count(int32_t *count);
int32_t gtmoe_open(int32_t device, gtmoe_context **out);
int32_t gtmoe_close(gtmoe_context *ctx);
/* No counterpart in the reference (a gpu.Device is garbage-collected):
 * closes the context if it is open and gives up the caller's handle, which
 * must not be used again.  The context's memory goes once the handle and
 * every layer and graph made on it are gone (gtmoe_layer_destroy,
 * gtmoe_graph_destroy); until then those still answer "the context is
 * closed". */
int32_t gtmoe_context_free(gtmoe_context *ctx);
/* Text of the last failure on this context (Device.LastError,
 * gpu/device.go:749-753).  With ctx NULL: the last failure of gtmoe_open. */
const char *gtmoe_last_error(const gtmoe_context *ctx);

/* Test hook, no counterpart in the reference: the next call of the entry
 * point named `entry_point` (e.g. "gtmoe_forward") made on this thread
 * answers `status` with the text "injected failure in <entry point>" instead
 * of running, as a failing HIP call would; later calls run normally.  For
 * testing a caller's fallback (the CPU answer and lastError of
 * gpu/device.go:733-737).  Armed per thread; one failure at a time. */
int32_t gtmoe_test_inject_failure(const char *entry_point, int32_t status);

/* Test hook, no counterpart in the reference: how many device allocations
 * (hipMalloc) and frees (hipFree) the library has made since it was loaded,
 * over all contexts and threads (either pointer may be NULL).  For tests that
 * a call allocates nothing, e.g. gtmoe_forward_device_noalloc. */
int32_t gtmoe_test_device_allocations(int64_t *allocations, int64_t *frees);

/* ---- quantization ---------------------------------------------------------
 * Rows.Append over `rows` rows of float64 values (lowprecision/rows.go:38-79,
 * encoders lowprecision/lowprecision.go:56-104), bit-exact.  values_out is
 * float/int8/packed-FP4 storage as in gtmoe_rows; scales_out is written for
 * INT8 and FP4.  Host only; no context needed. */
int32_t gtmoe_encode_rows(int32_t precision, int32_t rows, int32_t width, const double *values,
                          void *values_out, float *scales_out);

/* ---- layers ------------------------------------------------------------------
 * A layer is one MixtureOfExperts with its weights resident in HBM.  It
 * replaces buildMixtureOfExperts (mixtureofexperts.go:47-70) on the device. */
int32_t gtmoe_layer_create(gtmoe_context *ctx, const gtmoe_layer_desc *desc, gtmoe_layer **out);
int32_t gtmoe_layer_destroy(gtmoe_layer *layer);

/* Upload one weight matrix and its float64 biases (perceptron.Layer.Weights /
 * CompressedWeights and Biases, perceptron/layer.go:12-25).  index is the
 * expert within its role (ignored for ROUTER).  Expert matrices must use the
 * layer's precision; the router may be FLOAT64 or FLOAT32 (logits are
 * computed in fp32 on the device).  Shapes: gate/up h x d, down d x h,
 * router E x d.  Re-uploading replaces the matrix, as Layer.SetWeights does
 * (layer.go:234-246). */
int32_t gtmoe_upload_rows(gtmoe_layer *layer, int32_t role, int32_t index, const gtmoe_rows *rows,
                          const double *biases);

/* MixtureOfExperts.BalanceBiases (mixtureofexperts.go:20), E values. */
int32_t gtmoe_set_balance_biases(gtmoe_layer *layer, const double *biases);
int32_t gtmoe_get_balance_biases(const gtmoe_layer *layer, double *biases);

/* RMSNorm weights applied before this layer by gtmoe_stack_forward
 * (Block.FeedForwardNorm, transformer/block.go:59-60; epsilon 1e-6 as
 * normalization.NewRMSNorm, normalization/rmsnorm.go:20-31). */
int32_t gtmoe_set_norm_weights(gtmoe_layer *layer, const double *weights);

/* ---- forward ---------------------------------------------------------------
 * MixtureOfExperts.Forward (mixtureofexperts.go:122-216): inputs T x d
 * float64 row-major, token_ids T values (required with hash routing, may be
 * NULL otherwise), outputs T x d float64.  tokens may be 0.  flags is a
 * gtmoe_path.  The routing, gates, dispatch and per-expert load of the call
 * stay cached on the layer (the lastChosenExperts/lastGates/lastRowsForExpert/
 * lastExpertLoad state, :207-214) and are read back with gtmoe_last_routing.
 * A negative token id with hash routing returns GTMOE_ERR_INVALID_ARGUMENT
 * (the reference panics, :144-146). */
int32_t gtmoe_forward(gtmoe_layer *layer, int32_t tokens, const double *inputs, const int64_t *token_ids,
                      double *outputs, uint32_t flags);

/* Forward over device-resident fp32 activations (inputs and outputs T x d in
 * HBM, row-major, any 4-byte-aligned addresses; token_ids T int64 in HBM or
 * NULL), enqueued on `stream` without synchronising.  `stream` is a
 * hipStream_t; NULL is the device's null stream, which orders this forward
 * after work the caller enqueued on the null stream (torch's default stream,
 * for example) and before work enqueued there later.  Inputs and outputs must
 * not overlap (GTMOE_ERR_INVALID_ARGUMENT): a forward does not run in place.
 * Hash routing ids must be non-negative: the device cannot panic.  For callers
 * that keep activations on the GPU between layers; no reference counterpart
 * beyond Forward itself. */
int32_t gtmoe_forward_device(gtmoe_layer *layer, int32_t tokens, const float *inputs,
                             const int64_t *token_ids, float *outputs, uint32_t flags, void *stream);

/* ---- a forward that allocates nothing -----------------------------------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  The forward of gtmoe_forward_device (same arguments,
 * kernels and results), with every intermediate buffer taken from a fixed
 * scratch area inside the library instead of the layer's workspace: the call
 * allocates and frees nothing.  The area is GTMOE_NOALLOC_SCRATCH_BYTES on
 * each GPU, held from the library's load until the process ends.  A call
 * whose intermediates do not fit returns GTMOE_ERR_INVALID_ARGUMENT: a layer
 * of d = 2048, h = 1024 and 1 + 4 experts per token fits 792 tokens, one of
 * d = 1024, h = 2048 and 2 experts per token 1715.  Every call on
 * one GPU shares that GPU's area and finds there what the last call left:
 * calls enqueued on one stream are ordered, but calls that overlap in time on
 * one GPU (other streams, other threads) race.  The call keeps no routing
 * state on the layer: gtmoe_last_routing, gtmoe_last_expert_load and
 * gtmoe_relaunch answer GTMOE_ERR_NOT_READY until the next forward of another
 * kind, and per-kernel timing leaves its kernels out. */
#define GTMOE_NOALLOC_SCRATCH_BYTES (64u << 20)
int32_t gtmoe_forward_device_noalloc(gtmoe_layer *layer, int32_t tokens, const float *inputs,
                                     const int64_t *token_ids, float *outputs, uint32_t flags, void *stream);

/* The routing state of the last forward on this layer, any pointer may be
 * NULL: chosen T x k expert indices and gates T x k (lastChosenExperts,
 * lastGates), load E (lastExpertLoad), rows_for_expert T*k token indices with
 * expert_offsets E+1 (lastRowsForExpert flattened: experts ascending, tokens
 * ascending inside an expert).  tokens_out receives T.  Synchronises. */
int32_t gtmoe_last_routing(gtmoe_layer *layer, int32_t *tokens_out, int32_t *chosen, double *gates,
                           int32_t *load, int32_t *rows_for_expert, int32_t *expert_offsets);

/* MixtureOfExperts.LastExpertLoad (mixtureofexperts.go:287-291): E counts. */
int32_t gtmoe_last_expert_load(gtmoe_layer *layer, int32_t *load);

/* MixtureOfExperts.UpdateBalance (mixtureofexperts.go:293-310): moves every
 * balance bias by +-rate against the last forward's mean load.  Does
 * nothing before the first forward or with hash routing. */
int32_t gtmoe_update_balance(gtmoe_layer *layer, double rate);

/* Routing alone from given float64 router logits (pre-activation plus bias,
 * T x E): affinity sqrt(softplus), top-k with the balance biases and the
 * reference's tie-break, gates, then dispatch (mixtureofexperts.go:153-180).
 * Runs the same device kernels as the forward; outputs as in
 * gtmoe_last_routing (any may be NULL).  Bit-exact against the CPU
 * restatement for any logits. */
int32_t gtmoe_route_from_logits(gtmoe_layer *layer, int32_t tokens, const double *logits, int32_t *chosen,
                                double *gates, int32_t *load, int32_t *rows_for_expert,
                                int32_t *expert_offsets);

/* A stack of blocks without attention, x <- x + MoE_l(RMSNorm_l(x)) for
 * l = 0..n_layers-1 (the residual of transformer.Block.Forward,
 * transformer/block.go:71-77).  x is T x d float64, updated in place; every
 * layer needs gtmoe_set_norm_weights and the same d.  When chosen/gates are
 * given they receive [n_layers][T][k] of each layer's routing; every layer
 * must then have the same k (GTMOE_ERR_INVALID_ARGUMENT otherwise). */
int32_t gtmoe_stack_forward(gtmoe_layer *const *layers, int32_t n_layers, int32_t tokens, double *x,
                            const int64_t *token_ids, uint32_t flags, int32_t *chosen, double *gates);

/* The same stack over a device-resident fp32 x (T x d in HBM, updated in
 * place), enqueued on `stream` without synchronising (NULL: the null stream,
 * as for gtmoe_forward_device). */
int32_t gtmoe_stack_forward_device(gtmoe_layer *const *layers, int32_t n_layers, int32_t tokens, float *x,
                                   const int64_t *token_ids, uint32_t flags, void *stream);

/* ---- one forward as a HIP graph ----------------------------------------------
 * The decode step replayed without per-kernel launches: the kernels of
 * gtmoe_forward_device (one layer) or gtmoe_stack_forward_device (a stack)
 * for a fixed token count are recorded once into an instantiated hipGraph
 * and replayed by gtmoe_graph_launch on any stream (NULL: the null stream).
 * The graph keeps the device pointers it was recorded with: the caller
 * refills the same buffers between replays and keeps them alive.  While a
 * graph exists, its layers keep their workspace in place: a forward on one
 * of them with more tokens than any earlier call needed, and
 * gtmoe_layer_destroy, return GTMOE_ERR_INVALID_ARGUMENT until the graph is
 * destroyed.  Each replay counts
 * as a forward of every recorded layer (gtmoe_last_routing etc. read it).
 * Workspace is sized before recording; no replay allocates.  There is no
 * reference counterpart (the reference has no device graph); this serves
 * the block step of transformer/block.go:76-77,117 for decode. */
int32_t gtmoe_graph_capture_forward(gtmoe_layer *layer, int32_t tokens, const float *inputs,
                                    const int64_t *token_ids, float *outputs, uint32_t flags, gtmoe_graph **graph);
int32_t gtmoe_graph_capture_stack(gtmoe_layer *const *layers, int32_t n_layers, int32_t tokens, float *x,
                                  const int64_t *token_ids, uint32_t flags, gtmoe_graph **graph);
int32_t gtmoe_graph_launch(gtmoe_graph *graph, void *stream);
int32_t gtmoe_graph_destroy(gtmoe_graph *graph);

/* ---- measurement -----------------------------------------------------------
 * Per-kernel timing with HIP events, the counterpart of the Vulkan
 * timestamps behind Recorder.MeasureTime / DispatchTimes
 * (gpu/compute.go:54-57,670-694).  While enabled, every kernel the context
 * launches is bracketed by events on its stream; gtmoe_timing_read sums the
 * elapsed milliseconds per kernel name since the last reset.  Reading
 * synchronises.  names is a buffer of `capacity` entries of 64 bytes. */
int32_t gtmoe_timing_enable(gtmoe_context *ctx, int32_t enabled);
int32_t gtmoe_timing_reset(gtmoe_context *ctx);
int32_t gtmoe_timing_read(gtmoe_context *ctx, int32_t capacity, char *names, double *total_ms,
                          int32_t *launches, int32_t *count);

/* The expert path the last forward on this layer took (a gtmoe_path other
 * than AUTO). */
int32_t gtmoe_last_path(const gtmoe_layer *layer, int32_t *path);

/* Launch one expert kernel of the last forward on this layer again, with the
 * same arguments and workspace, on `stream` (a hipStream_t; NULL = the null
 * stream), without synchronising.  Bracketing a burst of these with
 * events gives the kernel's duration free of per-launch event skew -- the
 * per-dispatch timing of Recorder.MeasureTime (gpu/compute.go:670-694) for a
 * single program.  kernel: GTMOE_KERNEL_GATEUP (gate/up + SwiGLU) or
 * GTMOE_KERNEL_DOWN of the path the last forward took.  When the last
 * forward was a gtmoe_forward_device on the fp32 path of a layer with at
 * most two experts per token in all (shared + routed), its down kernel adds
 * the weighted rows straight into the caller's outputs (the combine is
 * folded into it), so launching it again adds them once more. */
enum gtmoe_kernel { GTMOE_KERNEL_GATEUP = 0, GTMOE_KERNEL_DOWN = 1 };
int32_t gtmoe_relaunch(gtmoe_layer *layer, int32_t kernel, void *stream);

/* ---- binary weights files ----------------------------------------------------
 * Reading GoTransformers binary weights files, "GOTRANSFORMERS-WEIGHTS-1" and
 * "-2" (weightfile/binaryfile.go:13-21, layout written at :63-138).  Opening
 * indexes the file and checks it as ReadBinaryKeepingCompressed does
 * (binaryfile.go:157-372, with RowsFromSnapshot, lowprecision/rows.go:172-203);
 * values are read from the file when asked for.  These are host calls and need
 * no context.  On failure gtmoe_weights_file_open writes the reference's
 * message, prefixed by the path, into `error` (when error_capacity > 0) and
 * returns GTMOE_ERR_INVALID_ARGUMENT; later calls leave theirs in
 * gtmoe_weights_file_error. */
enum gtmoe_stored_as {
    GTMOE_STORED_FLOAT64 = 1,
    GTMOE_STORED_FLOAT32 = 2,
    GTMOE_STORED_BFLOAT16 = 3,
    GTMOE_STORED_ROWS = 4 /* lowprecision.Rows: precision, rows, width */
};
int32_t gtmoe_weights_file_open(const char *path, gtmoe_weights_file **out, char *error, int32_t error_capacity);
int32_t gtmoe_weights_file_close(gtmoe_weights_file *file);
const char *gtmoe_weights_file_error(const gtmoe_weights_file *file);
/* Parameters in file order.  entry: name (NUL-terminated, cut to capacity),
 * stored_as, precision (-1 unless ROWS), rows and width (0 unless ROWS), and
 * count = values, or rows*width.  Any output may be NULL.  find: index of a
 * name, -1 when absent. */
int32_t gtmoe_weights_file_count(const gtmoe_weights_file *file, int32_t *count);
int32_t gtmoe_weights_file_entry(const gtmoe_weights_file *file, int32_t index, char *name, int32_t name_capacity,
                                 int32_t *stored_as, int32_t *precision, int64_t *rows, int64_t *width,
                                 int64_t *count);
int32_t gtmoe_weights_file_find(const gtmoe_weights_file *file, const char *name, int32_t *index);
/* A plain parameter's `count` values as float64, float32 and bfloat16
 * widened as readFloat32Values / readBFloat16Values do (binaryfile.go:309-331,
 * weightfile/precision.go:73-75).  The savedValues map of ReadBinary. */
int32_t gtmoe_weights_file_values(gtmoe_weights_file *file, int32_t index, double *out, int64_t count);
/* A compressed parameter's storage as in gtmoe_rows: the list its precision
 * reads (float64, float32, int8 or packed FP4 bytes; values_bytes long) and its
 * scale_count float32 scales.  The savedCompressedValues map of
 * ReadBinaryKeepingCompressed. */
int32_t gtmoe_weights_file_rows(gtmoe_weights_file *file, int32_t index, void *values, int64_t values_bytes,
                                float *scales, int64_t scale_count);

/* LoadBinary into one MixtureOfExperts (weightfile/weightfile.go:118-124 over
 * MixtureOfExperts.Parameters, mixtureofexperts.go:312-324): the parameters
 * "<name>.shared<i>.{gate,up,down}.{weights,biases}",
 * "<name>.expert<i>.{gate,up,down}.{weights,biases}" (i from 1,
 * mixtureofexperts.go:60-67) and, without hash routing,
 * "<name>.router.{weights,biases}" are moved from the file into the layer's
 * device buffers.  Every parameter is checked before any is uploaded, with
 * the messages of checkSavedParameterFits (weightfile.go:69-87): expert
 * weights must be compressed rows of the layer's shape; the router takes
 * plain values or compressed rows of as many values.  Expert rows at a
 * precision other than the layer's return GTMOE_ERR_UNSUPPORTED (the
 * reference would switch the layer's precision). */
int32_t gtmoe_layer_load_weights(gtmoe_layer *layer, gtmoe_weights_file *file, const char *name);

/* ---------------------------------------------------------------------------
 * Low-rank adapters and the backward (training around frozen compressed
 * experts).
 *
 * A layer with adapters runs gtmoe_forward through the adapter path: every
 * layer of the mixture (shared and routed experts' gate, up and down, and
 * the router) computes pre = (x W^T + s (x Down^T) Up^T) + b with s =
 * alpha / rank (perceptron/layer.go:133-162, perceptron/adapter.go:66-76),
 * in fp32, and keeps what gtmoe_backward needs.  gtmoe_forward_device, the
 * stack and graph entry points refuse such a layer.  Adapter dropout is not
 * supported (rate 0).
 * ------------------------------------------------------------------------- */

/* Model.AddLowRankAdapters over MixtureOfExperts.Layers
 * (transformer/adapters.go:24-38, mixtureofexperts.go:326-335): each layer
 * gets Layer.AddLowRankAdapter (adapter.go:28-44) with rank min(rank, inputs,
 * outputs): Down uniform in +-1/sqrt(inputs) from `seed` (not the
 * reference's random source; set the values with gtmoe_layer_set_adapter to
 * match a Go-side adapter), Up zero, gradients zero.  The router's adapter
 * exists with hash routing too and then stays unused. */
int32_t gtmoe_layer_add_adapters(gtmoe_layer *layer, int32_t rank, double alpha, uint64_t seed);
/* Model.RemoveAdapters (adapters.go:40-46). */
int32_t gtmoe_layer_remove_adapters(gtmoe_layer *layer);
/* Rank of one layer's adapter (LowRankAdapter.Rank); role/index as in
 * gtmoe_upload_rows. */
int32_t gtmoe_layer_adapter_rank(gtmoe_layer *layer, int32_t role, int32_t index, int32_t *rank);
/* Adapter.Down [rank][inputs] and Adapter.Up [outputs][rank], float64
 * row-major; either may be null to leave it. */
int32_t gtmoe_layer_set_adapter(gtmoe_layer *layer, int32_t role, int32_t index, const double *down,
                                const double *up);
int32_t gtmoe_layer_get_adapter(gtmoe_layer *layer, int32_t role, int32_t index, double *down, double *up);
/* Adapter.DownGradients and Adapter.UpGradients (the sums every Backward
 * adds to), same shapes as Down and Up. */
int32_t gtmoe_layer_adapter_gradients(gtmoe_layer *layer, int32_t role, int32_t index, double *down_grad,
                                      double *up_grad);
/* parameter.ZeroGradients over the adapters. */
int32_t gtmoe_layer_zero_adapter_gradients(gtmoe_layer *layer);
/* MixtureOfExperts.Backward (mixtureofexperts.go:227-285) after a
 * gtmoe_forward of the same `tokens` rows: output_gradients [tokens][d] in,
 * input_gradients [tokens][d] out (float64); every adapter's gradients are
 * added to.  Base weights are frozen (Layer.Backward with FreezeBase,
 * layer.go:164-210): input gradients go through them with
 * Rows.AddScaledRowTo (lowprecision/rows.go:285-324).  Without adapters it
 * fails as the reference panics for compressed weights. */
int32_t gtmoe_backward(gtmoe_layer *layer, int32_t tokens, const double *output_gradients,
                       double *input_gradients);

#ifdef __cplusplus
}
#endif

#endif /* GTMOE_H */
