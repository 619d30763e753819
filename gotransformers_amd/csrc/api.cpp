// C ABI of libgtmoe: contexts, layers resident in HBM, and the forward
// orchestration.  The host-side object mirrors mixtureofexperts.MixtureOfExperts
// (mixtureofexperts/mixtureofexperts.go:14-31): weights per role, balance
// biases, and the routing state of the last forward for LastExpertLoad and
// UpdateBalance.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <functional>
#include <initializer_list>
#include <map>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include "kernels.h"
#include "gtmoe.h"
#include "weightfile.h"

using namespace gtmoe;

namespace {

constexpr int kMaxExperts = 256;
constexpr int kMaxK = 8;
constexpr int kMaxGemvK = 4096;
// AUTO takes the dequant-GEMV path while routed tokens per expert stay at or
// below this many (decode batches); above it the MFMA grouped GEMM.
constexpr int kGemvTokensPerExpert = 8;
// The decode routing's read-ahead of the next kernel's gate/up rows: bytes
// (whole expert groups) and workgroups.
constexpr size_t kReadAheadBytes = 16u << 20;
constexpr int kReadAheadBlocks = 128;

thread_local std::string g_open_error;

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Every device allocation and free the library makes goes through these two,
// which count them for gtmoe_test_device_allocations.
std::atomic<long long> g_device_allocations{0}, g_device_frees{0};

template <class T>
hipError_t dev_malloc(T **p, size_t bytes)
{
    g_device_allocations.fetch_add(1, std::memory_order_relaxed);
    return hipMalloc(reinterpret_cast<void **>(p), bytes);
}

hipError_t dev_free(void *p)
{
    g_device_frees.fetch_add(1, std::memory_order_relaxed);
    return hipFree(p);
}

// Pinned host memory (the host API's staging) is counted with them.
hipError_t pinned_malloc(void **p, size_t bytes)
{
    g_device_allocations.fetch_add(1, std::memory_order_relaxed);
    return hipHostMalloc(p, bytes, hipHostMallocDefault);
}

hipError_t pinned_free(void *p)
{
    g_device_frees.fetch_add(1, std::memory_order_relaxed);
    return hipHostFree(p);
}

}  // namespace

struct TimingRecord {
    std::string name;
    hipEvent_t start;
    hipEvent_t stop;
};

struct gtmoe_context {
    int device = 0;
    int compute_units = 256;
    hipStream_t stream = nullptr;
    std::recursive_mutex mu;
    std::string error;
    bool timing = false;
    std::vector<TimingRecord> pending;
    std::vector<hipEvent_t> spare_events;
    std::map<std::string, std::pair<double, int>> totals;
    bool closed = false;      // gtmoe_close ran: the handle stays readable, every call answers an error
    // references: the caller's handle (until gtmoe_context_free), every layer
    // and every recorded graph; the last one to go frees the context
    int refs = 1;
    void *scratch = nullptr;  // device address of the no-allocation forward's scratch area on this device
    std::string scratch_error;
};

namespace {

int32_t fail(gtmoe_context *ctx, int32_t code, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (ctx) ctx->error = buf;
    else g_open_error = buf;
    return code;
}

#define HIP_TRY(ctx, call)                                                                              \
    do {                                                                                                \
        hipError_t e_ = (call);                                                                         \
        if (e_ != hipSuccess)                                                                           \
            return fail((ctx), e_ == hipErrorOutOfMemory ? GTMOE_ERR_OUT_OF_MEMORY : GTMOE_ERR_DEVICE, \
                        "%s: %s", #call, hipGetErrorString(e_));                                        \
    } while (0)

hipEvent_t take_event(gtmoe_context *ctx)
{
    if (!ctx->spare_events.empty()) {
        hipEvent_t e = ctx->spare_events.back();
        ctx->spare_events.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// Drops one reference to ctx (the caller holds no lock on it); the last frees it.
void release_context(gtmoe_context *ctx)
{
    bool last;
    {
        std::lock_guard<std::recursive_mutex> lock(ctx->mu);
        last = --ctx->refs == 0;
    }
    if (last) delete ctx;
}

// Launch one kernel through `fn`, bracketed by events when timing is on.
template <class F>
int32_t run(gtmoe_context *ctx, hipStream_t s, const char *name, F &&fn)
{
    hipEvent_t a = nullptr, b = nullptr;
    if (ctx->timing) {
        a = take_event(ctx);
        if (a) (void)hipEventRecord(a, s);
    }
    hipError_t e = fn();
    if (ctx->timing && a) {
        b = take_event(ctx);
        if (b) {
            (void)hipEventRecord(b, s);
            ctx->pending.push_back({name, a, b});
        } else {
            ctx->spare_events.push_back(a);
        }
    }
    if (e != hipSuccess) return fail(ctx, GTMOE_ERR_DEVICE, "kernel %s: %s", name, hipGetErrorString(e));
    return GTMOE_OK;
}

#define RUN(ctx, s, name, expr)                                      \
    do {                                                             \
        int32_t rc_ = run((ctx), (s), (name), [&]() { return (expr); }); \
        if (rc_ != GTMOE_OK) return rc_;                             \
    } while (0)

// One failure armed by gtmoe_test_inject_failure on this thread: the next
// call of the named entry point answers `status` instead of running.
thread_local std::string g_inject_entry;
thread_local int32_t g_inject_status = GTMOE_OK;

bool take_injection(const char *entry, int32_t *status)
{
    if (g_inject_status == GTMOE_OK || g_inject_entry != entry) return false;
    *status = g_inject_status;
    g_inject_status = GTMOE_OK;
    g_inject_entry.clear();
    return true;
}

// Entry into a call on a context: its lock, then the refusals every call
// shares (a closed context, an injected failure), then its device current.
#define ENTER_NODEV(c)                                                                                     \
    std::lock_guard<std::recursive_mutex> lock_((c)->mu);                                                  \
    do {                                                                                                   \
        if ((c)->closed) return fail((c), GTMOE_ERR_INVALID_ARGUMENT, "the context is closed");           \
        int32_t inj_ = GTMOE_OK;                                                                           \
        if (take_injection(__func__, &inj_)) return fail((c), inj_, "injected failure in %s", __func__);  \
    } while (0)
#define ENTER(c)      \
    ENTER_NODEV(c);   \
    HIP_TRY((c), hipSetDevice((c)->device))

}  // namespace

// Device buffers a forward needs, sized for `cap` tokens.
struct Workspace {
    int cap = -1;
    void *base = nullptr;
    double *x64 = nullptr;   // [T][d] host-API staging
    double *y64 = nullptr;   // [T][d]
    float *xf = nullptr;     // [T][dp]
    uint16_t *xb = nullptr;  // [T][dp] bf16
    float *xs = nullptr;     // [T][d] residual stream of a host-API stack
    double *logits = nullptr;
    int32_t *chosen = nullptr;
    double *gates = nullptr;
    float *gates32 = nullptr;
    int64_t *ids = nullptr;
    int32_t *load = nullptr;
    int32_t *offsets = nullptr;
    int32_t *rows = nullptr;
    int32_t *pos = nullptr;
    int32_t *goff = nullptr;
    int32_t *tile_off = nullptr;
    int4 *tile_desc = nullptr;    // (group, first position, positions) of every tile / slice
    int32_t *tok = nullptr;
    float *hidden32 = nullptr;    // [P][hp]
    uint16_t *hidden16 = nullptr;  // [P][hp] bf16
    float *slot_out = nullptr;    // [P][d] fp32 (fp32 path) or bf16 (MFMA path)
    int32_t *chunk_cnt = nullptr;  // [chunks][E] scratch of the many-token dispatch
    // a layer's own workspace only (not the no-allocation forward's area):
    int32_t *part_cnt = nullptr;   // [cap] arrival counts of a token's routing workgroups (kept zero)
    float *xalt = nullptr;         // [min(cap, kMaxSplitRouteTokens)][d] a stack's second residual buffer
    float *inv = nullptr;          // [T] inverse RMS of rows the previous stack layer's combine normalised
};

// Low-rank adapters of one weight role over all groups (G = S + E), or of
// the router (G = 1): A [G][R][kin], B [G][rows][R] fp32, zero beyond each
// layer's rank and widths; dA, dB their float64 gradient sums.
struct AdapterSet {
    int R = 0, kin = 0, width = 0, rows = 0, G = 0;
    float *A = nullptr, *B = nullptr, *scale = nullptr;
    double *dA = nullptr, *dB = nullptr;
};

// What the adapter path's forward keeps for the backward, sized for `cap`
// tokens (P = cap * (S + k) positions).
struct TrainWorkspace {
    int cap = -1;
    std::vector<void *> blocks;
    float *gpre = nullptr, *upre = nullptr;  // [P][hp] pre-activations of gate and up
    float *u_gate = nullptr, *u_up = nullptr, *u_down = nullptr, *u_router = nullptr;  // x A^T per position / token
    double *og = nullptr;    // [T][d] output gradients
    float *eg = nullptr;     // [P][d] expert output gradients
    float *hgrad = nullptr;  // [P][hp]
    float *ggrad = nullptr, *ugrad = nullptr;  // [P][hp]
    float *dxg = nullptr, *dxu = nullptr;      // [P][dp]
    float *t = nullptr;      // [max(P, T)][R]
    double *dx = nullptr;    // [T][d]
    double *lg = nullptr;    // [T][E]
    float *lgf = nullptr;    // [T][E]
    float *dxr = nullptr;    // [T][dp]
    int32_t *pgroup = nullptr;  // [P]
    int4 *tiles_tr = nullptr;  // [P + G]
    int32_t *goff_router = nullptr;  // {0, T}
    double *zero_bias = nullptr;     // [E]
    float *partial = nullptr;        // [chunks][P][max(dp, hp)] row-chunk sums of the transposed product
    int chunks = 1;                  // row chunks the partial buffer holds
    // position tiles of the adapter gradients (LoraArgs::otiles) of the
    // experts' groups and of the router's one group of tokens
    struct OuterTiles {
        int4 *tiles = nullptr;     // [P/64 + G]
        int32_t *toff = nullptr;   // [G + 1] first tile of every group
        int32_t *multi = nullptr;  // [G] groups of more than one tile
        int n = 0, nmulti = 0;
        std::vector<int4> host_tiles;  // sources of the uploads
        std::vector<int32_t> host_toff, host_multi;
    } ot, rt;
    float *outer = nullptr;  // [P/64 + G][R][max(dp, hp, E)] tile sums of the adapter gradients
    int P = 0, ntiles_tr = 0, tile_tr = 4;
};

struct gtmoe_layer {
    gtmoe_context *ctx = nullptr;
    gtmoe_layer_desc desc{};
    int d = 0, h = 0, S = 0, E = 0, k = 0, G = 0, dp = 0, hp = 0;
    DeviceMatrix gate, up, down;
    float *router_w = nullptr;  // [E][dp]
    double *router_b = nullptr;  // [E]
    double *balance = nullptr;   // [E]
    std::vector<double> balance_host;
    float *norm_w = nullptr;  // [d]
    bool has_norm = false;
    float *router_wn = nullptr;        // [E][dp] router rows times the norm weights
    std::vector<float> router_host;    // [E][dp] fp32 router rows
    std::vector<float> norm_host;      // [d]
    // launch arguments of the expert kernels of the last forward
    GemvArgs last_gemv[2]{};
    MfmaArgs last_mfma[2]{};
    int last_max_tiles = 0;
    bool relaunch_ready = false;  // the expert kernels of the last forward can be launched again
    std::vector<char> uploaded;  // per (role, index)
    Workspace ws;
    // state of the last forward
    int last_T = -1;
    int last_path = GTMOE_PATH_FP32;
    hipStream_t last_stream = nullptr;
    // kernels of a device-API call (forward, stack, graph replay, relaunch)
    // were enqueued on a caller's stream and may still run: a host-API call
    // waits for them before it touches the workspace or the weights
    bool device_work_pending = false;
    std::vector<int32_t> last_load;
    bool load_on_host = false;
    // the decode path's expert kernels found their own tokens: the dispatch
    // tables (load, rows_for_expert, offsets) are built only when read
    bool skipped_dispatch = false;  // by the forward being enqueued
    bool dispatch_pending = false;  // by the last forward
    // low-rank adapters on every layer (Model.AddLowRankAdapters over
    // MixtureOfExperts.Layers); the last forward's kept state for Backward
    bool has_adapters = false;
    AdapterSet ad_gate, ad_up, ad_down, ad_router;
    TrainWorkspace tw;
    int adapter_T = -1;  // tokens of the last forward through the adapter path, -1: none
    // recorded graphs that hold pointers into this layer's workspace: while
    // any exists the workspace is never reallocated
    int live_graphs = 0;
    // pinned host staging of the host-API calls: their float64 rows and the
    // routing state they copy back, so that every copy is one asynchronous
    // DMA on the stream and a call waits for the device once
    char *stage = nullptr;
    char *stage_dev = nullptr;  // the same memory as the device addresses it
    size_t stage_bytes = 0;
    // the routing state of the last gtmoe_forward, copied back with its
    // outputs: gtmoe_last_routing then answers from host memory
    bool routing_on_host = false;
    std::vector<int32_t> host_chosen, host_rows, host_offsets;
    std::vector<double> host_gates;
};

namespace {

int role_slot(const gtmoe_layer *L, int role, int index)
{
    switch (role) {
    case GTMOE_ROLE_ROUTER: return 0;
    case GTMOE_ROLE_SHARED_GATE:
    case GTMOE_ROLE_SHARED_UP:
    case GTMOE_ROLE_SHARED_DOWN: return 1 + (role - GTMOE_ROLE_SHARED_GATE) * L->G + index;
    default: return 1 + (role - GTMOE_ROLE_ROUTED_GATE) * L->G + L->S + index;
    }
}

int32_t alloc_matrix(gtmoe_context *ctx, DeviceMatrix &m, int precision, int rows, int width, int groups)
{
    m.precision = precision;
    m.rows = rows;
    m.rows_p = pad_rows(rows);
    m.width = width;
    m.kp = pad_k(width);
    m.nblocks = m.kp / kValuesPerScale;
    m.row_bytes = precision == kInt8 ? m.kp : precision == kFP4 ? m.kp / 2 : m.kp * 4;
    m.groups = groups;
    const size_t vb = (size_t)groups * m.group_value_bytes();
    HIP_TRY(ctx, dev_malloc(&m.values, vb));
    HIP_TRY(ctx, hipMemset(m.values, 0, vb));
    if (precision != kFloat32) {
        const size_t sb = (size_t)groups * m.group_scales() * sizeof(float);
        HIP_TRY(ctx, dev_malloc(&m.scales, sb));
        HIP_TRY(ctx, hipMemset(m.scales, 0, sb));
    } else {
        const size_t hb = (size_t)groups * m.group_bf16_bytes();
        HIP_TRY(ctx, dev_malloc(&m.bf16, hb));
        HIP_TRY(ctx, hipMemset(m.bf16, 0, hb));
    }
    const size_t bb = (size_t)groups * rows * sizeof(float);
    HIP_TRY(ctx, dev_malloc(&m.biases, bb));
    HIP_TRY(ctx, hipMemset(m.biases, 0, bb));
    return GTMOE_OK;
}

void free_matrix(DeviceMatrix &m)
{
    if (m.values) (void)dev_free(m.values);
    if (m.scales) (void)dev_free(m.scales);
    if (m.biases) (void)dev_free(m.biases);
    if (m.bf16) (void)dev_free(m.bf16);
    m.values = nullptr;
    m.scales = nullptr;
    m.biases = nullptr;
    m.bf16 = nullptr;
}

// Check a Rows snapshot like RowsFromSnapshot (lowprecision/rows.go:172-203).
int32_t check_rows(gtmoe_context *ctx, const gtmoe_rows *r, int rows, int width)
{
    if (!r) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "rows are null");
    if (r->rows != rows || r->width != width)
        return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "got %dx%d weights but the layer holds %dx%d", r->rows, r->width,
                    rows, width);
    const size_t blocks = (size_t)(width + 15) / 16;
    size_t want_values = 0, want_scales = 0;
    switch (r->precision) {
    case GTMOE_FLOAT64: want_values = (size_t)rows * width * 8; break;
    case GTMOE_FLOAT32: want_values = (size_t)rows * width * 4; break;
    case GTMOE_INT8:
        want_values = (size_t)rows * width;
        want_scales = (size_t)rows * blocks;
        break;
    case GTMOE_FP4:
        want_values = (size_t)rows * ((width + 1) / 2);
        want_scales = (size_t)rows * blocks;
        break;
    default: return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "unknown precision %d", r->precision);
    }
    if (r->values_bytes != want_values || r->scale_count != want_scales)
        return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT,
                    "rows snapshot for %d rows of width %d at precision %d has the wrong amount of data", rows, width,
                    r->precision);
    if (want_values && !r->values) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "values are null");
    if (want_scales && !r->scales) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "scales are null");
    return GTMOE_OK;
}

// Decoded float64 value i of row `row` (Rows.Row, lowprecision/rows.go:87-119).
double decoded_value(const gtmoe_rows *r, int row, int i)
{
    static const double kFp4[16] = {0, 0.5, 1, 1.5, 2, 3, 4, 6, 0, -0.5, -1, -1.5, -2, -3, -4, -6};
    const size_t blocks = (size_t)(r->width + 15) / 16;
    switch (r->precision) {
    case GTMOE_FLOAT64: return ((const double *)r->values)[(size_t)row * r->width + i];
    case GTMOE_FLOAT32: return (double)((const float *)r->values)[(size_t)row * r->width + i];
    case GTMOE_INT8:
        return (double)((const int8_t *)r->values)[(size_t)row * r->width + i] *
               (double)r->scales[row * blocks + i / 16];
    default: {
        const uint8_t byte = ((const uint8_t *)r->values)[(size_t)row * ((r->width + 1) / 2) + i / 2];
        const uint8_t code = (i % 2) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 15);
        return kFp4[code] * (double)r->scales[row * blocks + i / 16];
    }
    }
}

// The buffers of a forward for `cap` tokens laid out from `base` (256-byte
// aligned parts); returns the bytes they take.  With base null only the size
// is computed.  Without host staging the float64 rows of the host-API calls,
// the stack-only buffers (a host-API stack's residual, the rows' inverse
// RMS, the second residual buffer) and the split routing's arrival counts
// are left out (single-layer device forwards only; their routing then runs
// one workgroup per token).
size_t layout_workspace(const gtmoe_layer *L, int cap, bool host_staging, char *base, Workspace &w)
{
    const size_t P = (size_t)cap * (L->S + L->k);
    const size_t TK = (size_t)cap * L->k;
    const size_t hs = host_staging ? 1 : 0;
    struct Part {
        void **ptr;
        size_t bytes;
    };
    Part parts[] = {
        {(void **)&w.x64, hs * cap * L->d * 8},         {(void **)&w.y64, hs * cap * L->d * 8},
        {(void **)&w.xf, (size_t)cap * L->dp * 4},      {(void **)&w.xb, (size_t)cap * L->dp * 2},
        {(void **)&w.xs, hs * cap * L->d * 4},          {(void **)&w.logits, (size_t)cap * L->E * 8},
        {(void **)&w.chosen, TK * 4},                   {(void **)&w.gates, TK * 8},
        {(void **)&w.gates32, TK * 4},                  {(void **)&w.ids, hs * cap * 8},
        {(void **)&w.load, (size_t)L->E * 4},           {(void **)&w.offsets, (size_t)(L->E + 1) * 4},
        {(void **)&w.rows, TK * 4},                     {(void **)&w.pos, TK * 4},
        {(void **)&w.goff, (size_t)(L->G + 1) * 4},     {(void **)&w.tile_off, (size_t)(L->G + 1) * 4},
        {(void **)&w.tile_desc, ((size_t)L->S * cap + TK + L->G + 1 + 8) * sizeof(int4)},
        {(void **)&w.tok, P * 4},                       {(void **)&w.hidden32, P * L->hp * 4},
        {(void **)&w.hidden16, P * L->hp * 2},          {(void **)&w.slot_out, P * L->d * 4},
        {(void **)&w.chunk_cnt, (size_t)dispatch_chunks(cap) * L->E * 4},
        {(void **)&w.inv, hs * cap * 4},               {(void **)&w.part_cnt, hs * cap * 4},
        {(void **)&w.xalt, hs * std::min(cap, kMaxSplitRouteTokens) * L->d * 4},
    };
    size_t off = 0;
    for (const Part &p : parts) {
        if (base) *p.ptr = p.bytes ? base + off : nullptr;
        off += align_up(p.bytes, 256);
    }
    if (base) {
        w.base = base;
        w.cap = cap;
    }
    return off;
}

int32_t ensure_workspace(gtmoe_layer *L, int T)
{
    gtmoe_context *ctx = L->ctx;
    if (T <= L->ws.cap) return GTMOE_OK;
    if (L->live_graphs > 0)
        return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT,
                    "a forward of %d tokens needs a larger workspace than the %d tokens this layer's %d recorded "
                    "graph(s) use; destroy the graphs first",
                    T, L->ws.cap, L->live_graphs);
    int cap = T < 64 ? 64 : T;
    if (L->ws.base) {
        HIP_TRY(ctx, hipDeviceSynchronize());
        (void)dev_free(L->ws.base);
        L->ws = Workspace{};
    }
    Workspace w{};
    const size_t total = layout_workspace(L, cap, true, nullptr, w);
    void *base = nullptr;
    HIP_TRY(ctx, dev_malloc(&base, total));
    // zero once: padding columns of the activation buffers are never written.
    // hipMemset runs on the null stream, which does not order against the
    // non-blocking streams the forward runs on: wait for it here.
    HIP_TRY(ctx, hipMemset(base, 0, total));
    HIP_TRY(ctx, hipDeviceSynchronize());
    layout_workspace(L, cap, true, (char *)base, L->ws);
    return GTMOE_OK;
}

bool layer_ready(const gtmoe_layer *L, std::string &missing)
{
    for (int role = GTMOE_ROLE_ROUTER; role <= GTMOE_ROLE_ROUTED_DOWN; ++role) {
        if (role == GTMOE_ROLE_ROUTER && L->desc.use_hash_routing) continue;
        const int n = role == GTMOE_ROLE_ROUTER ? 1 : role <= GTMOE_ROLE_SHARED_DOWN ? L->S : L->E;
        for (int i = 0; i < n; ++i)
            if (!L->uploaded[role_slot(L, role, i)]) {
                char buf[96];
                snprintf(buf, sizeof buf, "role %d index %d", role, i);
                missing = buf;
                return false;
            }
    }
    return true;
}

int choose_path(const gtmoe_layer *L, int T, uint32_t flags)
{
    if (flags == GTMOE_PATH_FP32 || flags == GTMOE_PATH_BF16) return (int)flags;
    const long long routed = (long long)T * L->k;
    const bool few = routed <= (long long)kGemvTokensPerExpert * L->E;
    const bool fits = L->dp <= kMaxGemvK && L->hp <= kMaxGemvK;
    return (few && fits) ? GTMOE_PATH_FP32 : GTMOE_PATH_BF16;
}

// Where a forward's input rows come from: raw rows [T][d] as float or
// double, optionally passed through the layer's RMSNorm first.
struct Inputs {
    const void *x;
    bool f64;
    bool norm;
    bool host = false;  // the rows are in pinned host memory: converted once, never read in place
};

// A stack layer's combine left for the next layer's routing kernel to do.
struct PendingCombine {
    const float *slot;
    const int32_t *pos;
    const float *gates;
    int S, k, d;
};

// Input preparation, routing and dispatch.  Few tokens: one fused launch.
// Otherwise: convert or RMSNorm into ws.xf / ws.xb, router and top-k (or hash
// routing), then the dispatch.  token_ids: device pointer (hash routing).
int32_t prepare_and_route(gtmoe_layer *L, int T, const Inputs &in, const int64_t *token_ids, int path, hipStream_t s,
                          float *zero_out = nullptr, const PendingCombine *pend = nullptr, bool prenormed = false,
                          float *x_out = nullptr)
{
    gtmoe_context *ctx = L->ctx;
    Workspace &w = L->ws;
    const bool hash = L->desc.use_hash_routing != 0;
    const bool need_f32 = path == GTMOE_PATH_FP32 || !hash;
    float *xf = need_f32 ? w.xf : nullptr;
    uint16_t *xb = path == GTMOE_PATH_BF16 ? w.xb : nullptr;
    // fp32 rows for the router: an fp32 input whose rows are already a
    // multiple of 64 wide is read in place on the bf16 path
    const float *xr = w.xf;
    if (path == GTMOE_PATH_BF16 && !in.f64 && !in.norm && !in.host && L->d == L->dp) {
        xf = nullptr;
        xr = (const float *)in.x;
    }
    // the dispatch's per-group tile prefix counts MFMA m-tiles on the bf16
    // path and token slices on the fp32 path
    const int bm = path == GTMOE_PATH_BF16 ? mfma_tile_m() : kGemvSlice;
    if (fused_route_fits(T, L->k, L->dp)) {
        FusedArgs f{};
        f.x = in.x;
        f.norm = in.norm ? L->norm_w : nullptr;
        f.w = in.norm ? L->router_wn : L->router_w;
        f.bias = L->router_b;
        f.balance = L->balance;
        f.ids = token_ids;
        f.T = T;
        f.d = L->d;
        f.kp = L->dp;
        f.E = L->E;
        f.k = L->k;
        f.S = L->S;
        f.bm = bm;
        f.xf = xf;
        f.xb = xb;
        f.logits = w.logits;
        f.chosen = w.chosen;
        f.gates = w.gates;
        f.gates32 = w.gates32;
        f.load = w.load;
        f.offsets = w.offsets;
        f.rows = w.rows;
        f.pos = w.pos;
        f.goff = w.goff;
        f.tok = w.tok;
        f.tile_off = w.tile_off;
        f.tile_desc = w.tile_desc;
        f.zero_out = zero_out;
        // split routing where the workspace has the arrival counts
        f.parts = w.part_cnt ? route_fused_parts(T, L->E, hash) : 1;
        f.part_cnt = w.part_cnt;
        f.x_out = x_out;
        if (pend) {  // x is the fp32 residual stream, combined first (into x_out, or in place)
            f.pend_slot = pend->slot;
            f.pend_pos = pend->pos;
            f.pend_gates = pend->gates;
            f.pend_S = pend->S;
            f.pend_k = pend->k;
        }
        // the fp32 path's kernels find their own tokens from the choices
        L->skipped_dispatch = path == GTMOE_PATH_FP32 && T <= kSelfDispatchMaxTokens;
        // When the batch holds at least one entry per expert, the gate/up
        // kernel that follows streams most groups' rows, shared groups first
        // and then routed experts in order: the routing launch reads the
        // first groups ahead while its own work leaves HBM idle.
        if (L->skipped_dispatch && !hash && T * L->k >= L->E) {
            const DeviceMatrix &gm = L->gate, &um = L->up;
            const size_t per_group = gm.group_value_bytes() + um.group_value_bytes() +
                                     (gm.scales ? gm.group_scales() * sizeof(float) : 0) +
                                     (um.scales ? um.group_scales() * sizeof(float) : 0);
            const size_t groups = std::min<size_t>(gm.groups, kReadAheadBytes / per_group);
            if (groups > 0) {
                f.ra[0] = gm.values;
                f.ra_bytes[0] = groups * gm.group_value_bytes();
                f.ra[1] = um.values;
                f.ra_bytes[1] = groups * um.group_value_bytes();
                f.ra[2] = gm.scales;
                f.ra_bytes[2] = gm.scales ? groups * gm.group_scales() * sizeof(float) : 0;
                f.ra[3] = um.scales;
                f.ra_bytes[3] = um.scales ? groups * um.group_scales() * sizeof(float) : 0;
                f.ra_blocks = kReadAheadBlocks;
            }
        }
        RUN(ctx, s, "route_small", launch_route_fused(f, in.f64, hash, !L->skipped_dispatch, s));
        return GTMOE_OK;
    }
    L->skipped_dispatch = false;
    if (pend)
        RUN(ctx, s, "combine",
            launch_combine(T, pend->d, pend->S, pend->k, pend->slot, false, pend->pos, pend->gates,
                           (const float *)in.x, (float *)in.x, nullptr, s));
    if (zero_out) RUN(ctx, s, "zero_out", launch_fill_i32(reinterpret_cast<int32_t *>(zero_out), T * L->d, 0, s));
    // the chunked dispatch's counts: cleared by the router, added up by the
    // top-k (no count launch)
    const bool counted = !hash && dispatch_chunked(T);
    int32_t *cnt = counted ? w.chunk_cnt : nullptr;
    const int ncnt = counted ? dispatch_chunks(T) * L->E : 0;
    if (prenormed) {
        // the previous layer's combine wrote the bf16 normalised rows and each
        // row's inverse RMS; the router reads the raw rows (stride d == dp)
        // against its rows times the norm weights
        if (!hash) {
            RUN(ctx, s, "router",
                launch_router((const float *)in.x, L->d, T, L->d, L->router_wn, L->dp, L->router_b, L->E, w.logits,
                              s, w.inv, nullptr, 0, cnt, ncnt));
            RUN(ctx, s, "topk",
                launch_topk(w.logits, T, L->E, L->k, L->balance, w.chosen, w.gates, w.gates32, s, cnt));
        } else {
            RUN(ctx, s, "hash_route",
                launch_hash_route(token_ids, T, L->E, L->k, w.chosen, w.gates, w.gates32, s));
        }
        RUN(ctx, s, "dispatch",
            launch_dispatch(w.chosen, T, L->k, L->E, L->S, bm, w.load, w.offsets, w.rows, w.pos, w.goff, w.tok,
                            w.tile_off, w.tile_desc, w.chunk_cnt, s, counted));
        return GTMOE_OK;
    }
    if (in.norm) {
        RUN(ctx, s, "rmsnorm", launch_rmsnorm((const float *)in.x, T, L->d, L->norm_w, xf, L->dp, xb, L->dp, s));
    } else if (in.f64) {
        RUN(ctx, s, "convert_inputs",
            launch_convert_inputs_f64((const double *)in.x, T, L->d, xf, L->dp, xb, L->dp, s));
    } else if (xf != nullptr || hash) {
        RUN(ctx, s, "convert_inputs",
            launch_convert_inputs_f32((const float *)in.x, T, L->d, xf, L->dp, xb, L->dp, s));
    }
    // an fp32 input read in place by the router: the router writes its bf16 rows
    uint16_t *router_xb = xf == nullptr && !in.f64 && !in.norm && !hash ? xb : nullptr;
    if (hash) {
        RUN(ctx, s, "hash_route", launch_hash_route(token_ids, T, L->E, L->k, w.chosen, w.gates, w.gates32, s));
    } else {
        RUN(ctx, s, "router", launch_router(xr, L->dp, T, L->d, L->router_w, L->dp, L->router_b, L->E, w.logits, s,
                                            nullptr, router_xb, L->dp, cnt, ncnt));
        RUN(ctx, s, "topk", launch_topk(w.logits, T, L->E, L->k, L->balance, w.chosen, w.gates, w.gates32, s, cnt));
    }
    RUN(ctx, s, "dispatch",
        launch_dispatch(w.chosen, T, L->k, L->E, L->S, bm, w.load, w.offsets, w.rows, w.pos, w.goff, w.tok,
                        w.tile_off, w.tile_desc, w.chunk_cnt, s, counted));
    return GTMOE_OK;
}

// The expert kernels over the dispatched positions, reading ws.xf (fp32
// path) or ws.xb (bf16 path); leaves the slot outputs in ws.slot_out.
int32_t run_experts(gtmoe_layer *L, int T, int path, hipStream_t s, float *final_out = nullptr)
{
    gtmoe_context *ctx = L->ctx;
    Workspace &w = L->ws;
    const int bm = path == GTMOE_PATH_BF16 ? mfma_tile_m() : kGemvSlice;
    // upper bound of the tiles / slices over all groups; without dispatch
    // tables, the shared slices plus two workgroups per routed expert
    const bool self = path == GTMOE_PATH_FP32 && L->skipped_dispatch;
    const int max_tiles = self ? L->S * ((T + bm - 1) / bm) + 2 * L->E
                               : L->S * ((T + bm - 1) / bm) + (T * L->k + bm - 1) / bm + L->E;
    auto set_self = [&](GemvArgs &g) {
        g.self_dispatch = 1;
        g.shared_slices = (T + kGemvSlice - 1) / kGemvSlice;
        g.T = T;
        g.k = L->k;
        g.S = L->S;
        g.E = L->E;
        g.chosen = w.chosen;
        g.gates32 = w.gates32;
    };
    if (path == GTMOE_PATH_FP32) {
        GemvArgs a{};
        a.w0 = L->gate.values;
        a.s0 = L->gate.scales;
        a.b0 = L->gate.biases;
        a.w1 = L->up.values;
        a.s1 = L->up.scales;
        a.b1 = L->up.biases;
        a.w_group_stride = (long long)L->gate.group_value_bytes();
        a.s_group_stride = (long long)L->gate.group_scales();
        a.rows = L->h;
        a.nblocks = L->gate.nblocks;
        a.row_bytes = L->gate.row_bytes;
        a.in = w.xf;
        a.ld_in = L->dp;
        a.in_rows = w.cap;
        a.tok = w.tok;
        a.count = w.tile_off + L->G;
        a.desc = w.tile_desc;
        a.out = w.hidden32;
        a.ld_out = L->hp;
        a.clamp = (float)L->desc.clamp_limit;
        if (self) set_self(a);
        L->last_gemv[0] = a;
        L->last_max_tiles = max_tiles;
        L->relaunch_ready = true;
        RUN(ctx, s, "gemv_gateup", launch_gemv_gateup(a, L->gate.precision, max_tiles, s));
        GemvArgs b{};
        b.w0 = L->down.values;
        b.s0 = L->down.scales;
        b.b0 = L->down.biases;
        b.w_group_stride = (long long)L->down.group_value_bytes();
        b.s_group_stride = (long long)L->down.group_scales();
        b.rows = L->d;
        b.nblocks = L->down.nblocks;
        b.row_bytes = L->down.row_bytes;
        b.in = w.hidden32;
        b.ld_in = L->hp;
        b.in_rows = (long long)w.cap * (L->S + L->k);
        b.tok = nullptr;
        b.count = w.tile_off + L->G;
        b.desc = w.tile_desc;
        b.out = w.slot_out;
        b.ld_out = L->d;
        if (final_out) {
            b.final_out = final_out;
            b.tok_all = w.tok;
            b.chosen = w.chosen;
            b.gates32 = w.gates32;
            b.T = T;
            b.k = L->k;
            b.S = L->S;
        }
        if (self) set_self(b);
        L->last_gemv[1] = b;
        RUN(ctx, s, "gemv_down", launch_gemv_down(b, L->down.precision, max_tiles, s));
    } else {
        MfmaArgs a{};
        a.w0 = L->gate.values;
        a.s0 = L->gate.scales;
        a.b0 = L->gate.biases;
        a.w1 = L->up.values;
        a.s1 = L->up.scales;
        a.b1 = L->up.biases;
        a.w_group_stride = (long long)L->gate.group_value_bytes();
        a.s_group_stride = (long long)L->gate.group_scales();
        a.n = L->h;
        a.kp = L->dp;
        a.row_bytes = L->gate.row_bytes;
        a.nblocks = L->gate.nblocks;
        a.a = w.xb;
        a.lda = L->dp;
        a.a_rows = w.cap;
        a.tok = w.tok;
        a.count = w.tile_off + L->G;
        a.desc = w.tile_desc;
        a.out = w.hidden16;
        a.ldo = L->hp;
        a.clamp = (float)L->desc.clamp_limit;
        if (L->gate.precision == kFloat32) {  // Float32 experts: their rows' bf16 copies
            a.w0 = L->gate.bf16;
            a.w1 = L->up.bf16;
            a.w_group_stride = (long long)L->gate.group_bf16_bytes();
            a.row_bytes = L->gate.bf16_row_bytes();
        }
        L->last_mfma[0] = a;
        L->last_max_tiles = max_tiles;
        L->relaunch_ready = true;
        RUN(ctx, s, "mfma_gateup", launch_mfma_gateup(a, L->gate.precision, max_tiles, s));
        MfmaArgs b{};
        b.w0 = L->down.values;
        b.s0 = L->down.scales;
        b.b0 = L->down.biases;
        b.w_group_stride = (long long)L->down.group_value_bytes();
        b.s_group_stride = (long long)L->down.group_scales();
        b.n = L->d;
        b.kp = L->hp;
        b.row_bytes = L->down.row_bytes;
        b.nblocks = L->down.nblocks;
        b.a = w.hidden16;
        b.lda = L->hp;
        b.a_rows = (long long)w.cap * (L->S + L->k);
        b.tok = nullptr;
        b.count = w.tile_off + L->G;
        b.desc = w.tile_desc;
        b.out = w.slot_out;
        b.ldo = L->d;
        if (L->down.precision == kFloat32) {
            b.w0 = L->down.bf16;
            b.w_group_stride = (long long)L->down.group_bf16_bytes();
            b.row_bytes = L->down.bf16_row_bytes();
        }
        L->last_mfma[1] = b;
        RUN(ctx, s, "mfma_down", launch_mfma_down(b, L->down.precision, max_tiles, s));
    }
    return GTMOE_OK;
}

void mark_forward(gtmoe_layer *L, int T, int path, hipStream_t s)
{
    L->last_T = T;
    L->last_path = path;
    L->last_stream = s;
    L->device_work_pending = s != L->ctx->stream;
    L->routing_on_host = false;
    L->load_on_host = false;
    L->dispatch_pending = T > 0 && L->skipped_dispatch;
    L->adapter_T = -1;  // set again by the adapter path's forward
}

// Pinned staging of at least `bytes` for a host-API call.
int32_t ensure_stage(gtmoe_layer *L, size_t bytes)
{
    if (bytes <= L->stage_bytes) return GTMOE_OK;
    if (L->stage) {
        HIP_TRY(L->ctx, hipDeviceSynchronize());  // no copy into the old block is in flight
        (void)pinned_free(L->stage);
        L->stage = nullptr;
        L->stage_bytes = 0;
    }
    bytes = std::max(bytes, (size_t)64 << 10);
    void *p = nullptr, *dp = nullptr;
    HIP_TRY(L->ctx, pinned_malloc(&p, bytes));
    L->stage = static_cast<char *>(p);
    L->stage_bytes = bytes;
    HIP_TRY(L->ctx, hipHostGetDevicePointer(&dp, p, 0));
    L->stage_dev = static_cast<char *>(dp);
    return GTMOE_OK;
}

// Before a host-API call enqueues work on the context's stream, which does
// not synchronise with a caller's streams: wait for any device-API work on
// this layer (its kernels use the same workspace, routing state and weights).
// The device is synchronised as a whole: the caller's stream may be gone.
int32_t settle_device_work(gtmoe_layer *L)
{
    if (!L->device_work_pending) return GTMOE_OK;
    HIP_TRY(L->ctx, hipDeviceSynchronize());
    L->device_work_pending = false;
    return GTMOE_OK;
}

// Build the dispatch tables of the last forward if its kernels skipped them
// (the same kernel as a forward's dispatch, so the tables are identical).
int32_t ensure_dispatch(gtmoe_layer *L)
{
    if (!L->dispatch_pending) return GTMOE_OK;
    gtmoe_context *ctx = L->ctx;
    Workspace &w = L->ws;
    hipStream_t s = L->last_stream;
    RUN(ctx, s, "dispatch",
        launch_dispatch(w.chosen, L->last_T, L->k, L->E, L->S, kGemvSlice, w.load, w.offsets, w.rows, w.pos, w.goff,
                        w.tok, w.tile_off, w.tile_desc, w.chunk_cnt, s));
    L->dispatch_pending = false;
    return GTMOE_OK;
}

int32_t fetch_load(gtmoe_layer *L)
{
    gtmoe_context *ctx = L->ctx;
    if (L->last_T < 0) return fail(ctx, GTMOE_ERR_NOT_READY, "call Forward before reading the expert load");
    if (L->load_on_host) return GTMOE_OK;
    int32_t rc = ensure_dispatch(L);
    if (rc != GTMOE_OK) return rc;
    L->last_load.assign(L->E, 0);
    if (L->last_T > 0) {
        HIP_TRY(ctx, hipStreamSynchronize(L->last_stream));
        HIP_TRY(ctx, hipMemcpy(L->last_load.data(), L->ws.load, sizeof(int32_t) * L->E, hipMemcpyDeviceToHost));
    }
    L->load_on_host = true;
    return GTMOE_OK;
}

// Router rows with the RMSNorm weights folded in, for the fused routing of
// a normalised input: logit = inv_rms * sum_i x_i * (w_ei * norm_i) + b_e.
int32_t refresh_folded_router(gtmoe_layer *L)
{
    if (L->router_host.empty() || L->norm_host.empty()) return GTMOE_OK;
    std::vector<float> wn(L->router_host.size(), 0.f);
    for (int e = 0; e < L->E; ++e)
        for (int i = 0; i < L->d; ++i)
            wn[(size_t)e * L->dp + i] = L->router_host[(size_t)e * L->dp + i] * L->norm_host[i];
    HIP_TRY(L->ctx, hipMemcpy(L->router_wn, wn.data(), wn.size() * sizeof(float), hipMemcpyHostToDevice));
    return GTMOE_OK;
}

int32_t check_layer_call(gtmoe_layer *L)
{
    if (!L || !L->ctx) return GTMOE_ERR_INVALID_ARGUMENT;
    std::string missing;
    if (!layer_ready(L, missing))
        return fail(L->ctx, GTMOE_ERR_NOT_READY, "mixture of experts: weights not uploaded (%s)", missing.c_str());
    return GTMOE_OK;
}

}  // namespace

// ---- HIP graphs of a whole forward ------------------------------------------

struct gtmoe_graph {
    gtmoe_context *ctx = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    std::vector<gtmoe_layer *> layers;
    std::vector<int> paths;
    std::vector<char> skipped;  // per layer: its recorded forward builds no dispatch tables
    int T = 0;
};

namespace {

void free_graph(gtmoe_graph *g)
{
    if (!g) return;
    if (g->exec)
        for (gtmoe_layer *L : g->layers) --L->live_graphs;
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
}

// Records `record(s)` on a private capture stream into an instantiated graph.
template <class F>
int32_t capture(gtmoe_context *ctx, F &&record, gtmoe_graph *g)
{
    hipStream_t cs = nullptr;
    HIP_TRY(ctx, hipStreamCreateWithFlags(&cs, hipStreamNonBlocking));
    const bool timing = ctx->timing;
    ctx->timing = false;  // no event nodes in the graph
    hipError_t e = hipStreamBeginCapture(cs, hipStreamCaptureModeRelaxed);
    int32_t rc = e == hipSuccess ? record(cs) : fail(ctx, GTMOE_ERR_DEVICE, "hipStreamBeginCapture: %s",
                                                      hipGetErrorString(e));
    hipGraph_t graph = nullptr;
    if (e == hipSuccess) {
        const hipError_t e2 = hipStreamEndCapture(cs, &graph);
        if (rc == GTMOE_OK && e2 != hipSuccess)
            rc = fail(ctx, GTMOE_ERR_DEVICE, "hipStreamEndCapture: %s", hipGetErrorString(e2));
    }
    ctx->timing = timing;
    (void)hipStreamDestroy(cs);
    if (rc != GTMOE_OK) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
    }
    g->graph = graph;
    e = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        g->exec = nullptr;
        return fail(ctx, GTMOE_ERR_DEVICE, "hipGraphInstantiate: %s", hipGetErrorString(e));
    }
    for (gtmoe_layer *L : g->layers) ++L->live_graphs;
    return GTMOE_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Scratch area of gtmoe_forward_device_noalloc: the intermediates of that
// forward live here instead of in a layer's workspace.  Each GPU the library
// runs on holds its own copy from the library's load until the process ends.
// In host code `scratch` names a host-side stand-in, not device memory: the
// device address on each GPU comes from hipGetSymbolAddress, queried once per
// device with that device current, and only that address is ever handed to
// kernels.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[GTMOE_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
bool g_scratch_queried[kMaxScratchDevices] = {};
void *g_scratch_ptr[kMaxScratchDevices] = {};
hipError_t g_scratch_status[kMaxScratchDevices] = {};

// The device address of `scratch` on `device`, which must be current; null
// with `err` set when it cannot be had.
void *scratch_address(int device, std::string &err)
{
    if (device < 0 || device >= kMaxScratchDevices) {
        err = "device index beyond the scratch table";
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_queried[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch_status[device] = e;
        g_scratch_ptr[device] = e == hipSuccess ? p : nullptr;
        g_scratch_queried[device] = true;
    }
    if (!g_scratch_ptr[device]) err = std::string("hipGetSymbolAddress: ") + hipGetErrorString(g_scratch_status[device]);
    return g_scratch_ptr[device];
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// Low-rank adapters (perceptron/adapter.go) and the adapter path: a forward
// that keeps what the backward needs, and MixtureOfExperts.Backward
// (mixtureofexperts.go:227-285) over frozen base weights.
// ---------------------------------------------------------------------------
namespace {

void free_adapter(AdapterSet &a)
{
    for (void *p : {(void *)a.A, (void *)a.B, (void *)a.scale, (void *)a.dA, (void *)a.dB})
        if (p) (void)dev_free(p);
    a = AdapterSet{};
}

void free_train_workspace(TrainWorkspace &tw)
{
    for (void *p : tw.blocks) (void)dev_free(p);
    tw = TrainWorkspace{};
}

void free_adapters(gtmoe_layer *L)
{
    free_adapter(L->ad_gate);
    free_adapter(L->ad_up);
    free_adapter(L->ad_down);
    free_adapter(L->ad_router);
    free_train_workspace(L->tw);
    L->has_adapters = false;
    L->adapter_T = -1;
}

// Uniform in [-limit, limit) from a seeded splitmix64 stream (the device
// cannot follow the reference's random source; callers that need its exact
// values set them with gtmoe_layer_set_adapter).
double seeded_uniform(uint64_t &state, double limit)
{
    uint64_t z = (state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    z ^= z >> 31;
    const double u = (double)(z >> 11) * (1.0 / 9007199254740992.0);
    return -limit + 2.0 * limit * u;
}

// AddLowRankAdapter (adapter.go:28-44) on every group of one role: rank
// min(rank, inputs, outputs) as Model.AddLowRankAdapters picks it
// (transformer/adapters.go:24-38), Down uniform in +-1/sqrt(inputs), Up zero.
int32_t alloc_adapter(gtmoe_context *ctx, AdapterSet &a, int G, int width, int kin, int rows, int rank, double alpha,
                      uint64_t &seed)
{
    a.G = G;
    a.width = width;
    a.kin = kin;
    a.rows = rows;
    a.R = std::min(rank, std::min(width, rows));
    const size_t na = (size_t)G * a.R * kin, nb = (size_t)G * rows * a.R;
    HIP_TRY(ctx, dev_malloc(&a.A, na * sizeof(float)));
    HIP_TRY(ctx, dev_malloc(&a.B, nb * sizeof(float)));
    HIP_TRY(ctx, dev_malloc(&a.scale, G * sizeof(float)));
    HIP_TRY(ctx, dev_malloc(&a.dA, na * sizeof(double)));
    HIP_TRY(ctx, dev_malloc(&a.dB, nb * sizeof(double)));
    std::vector<float> A(na, 0.f);
    const double limit = 1.0 / std::sqrt((double)width);
    for (int g = 0; g < G; ++g)
        for (int j = 0; j < a.R; ++j)
            for (int i = 0; i < width; ++i)
                A[((size_t)g * a.R + j) * kin + i] = (float)seeded_uniform(seed, limit);
    const std::vector<float> sc(G, (float)(alpha / a.R));
    HIP_TRY(ctx, hipMemcpy(a.A, A.data(), na * sizeof(float), hipMemcpyHostToDevice));
    HIP_TRY(ctx, hipMemset(a.B, 0, nb * sizeof(float)));
    HIP_TRY(ctx, hipMemcpy(a.scale, sc.data(), G * sizeof(float), hipMemcpyHostToDevice));
    HIP_TRY(ctx, hipMemset(a.dA, 0, na * sizeof(double)));
    HIP_TRY(ctx, hipMemset(a.dB, 0, nb * sizeof(double)));
    return GTMOE_OK;
}

// The adapter of (role, index) and its group, or null with an error.
AdapterSet *adapter_of(gtmoe_layer *L, int role, int index, int *group)
{
    gtmoe_context *ctx = L->ctx;
    if (!L->has_adapters) {
        fail(ctx, GTMOE_ERR_NOT_READY, "the layer has no low-rank adapters");
        return nullptr;
    }
    if (role == GTMOE_ROLE_ROUTER) {
        if (index != 0) {
            fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "the router is index 0, got %d", index);
            return nullptr;
        }
        *group = 0;
        return &L->ad_router;
    }
    const bool shared = role >= GTMOE_ROLE_SHARED_GATE && role <= GTMOE_ROLE_SHARED_DOWN;
    const bool routed = role >= GTMOE_ROLE_ROUTED_GATE && role <= GTMOE_ROLE_ROUTED_DOWN;
    if (!shared && !routed) {
        fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "unknown role %d", role);
        return nullptr;
    }
    const int n = shared ? L->S : L->E;
    if (index < 0 || index >= n) {
        fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "%s expert %d of %d", shared ? "shared" : "routed", index, n);
        return nullptr;
    }
    *group = shared ? index : L->S + index;
    const int which = shared ? role - GTMOE_ROLE_SHARED_GATE : role - GTMOE_ROLE_ROUTED_GATE;
    return which == 0 ? &L->ad_gate : which == 1 ? &L->ad_up : &L->ad_down;
}

int32_t ensure_train_workspace(gtmoe_layer *L, int T)
{
    TrainWorkspace &tw = L->tw;
    if (tw.cap >= T && tw.cap > 0) return GTMOE_OK;
    gtmoe_context *ctx = L->ctx;
    free_train_workspace(tw);
    const int cap = std::max(T, 1);
    const size_t P = (size_t)cap * (L->S + L->k);
    const size_t R = std::max({L->ad_gate.R, L->ad_up.R, L->ad_down.R, L->ad_router.R, 1});
    auto get = [&](auto *&ptr, size_t count) -> int32_t {
        void *p = nullptr;
        HIP_TRY(ctx, dev_malloc(&p, std::max<size_t>(count, 1) * sizeof(*ptr)));
        tw.blocks.push_back(p);
        ptr = static_cast<std::remove_reference_t<decltype(ptr)>>(p);
        return GTMOE_OK;
    };
    int32_t rc = GTMOE_OK;
    const size_t hp = L->hp, dp = L->dp, d = L->d, E = L->E;
    // row chunks of the transposed product: enough workgroups at decode
    // sizes, scratch bounded by 256 MB
    const size_t per_chunk = P * std::max(hp, dp) * sizeof(float);
    tw.chunks = (int)std::max<size_t>(1, std::min<size_t>(64, (256u << 20) / per_chunk));
    for (auto step : std::initializer_list<std::function<int32_t()>>{
             [&] { return get(tw.gpre, P * hp); }, [&] { return get(tw.upre, P * hp); },
             [&] { return get(tw.u_gate, P * R); }, [&] { return get(tw.u_up, P * R); },
             [&] { return get(tw.u_down, P * R); }, [&] { return get(tw.u_router, (size_t)cap * R); },
             [&] { return get(tw.og, (size_t)cap * d); }, [&] { return get(tw.eg, P * d); },
             [&] { return get(tw.hgrad, P * hp); }, [&] { return get(tw.ggrad, P * hp); },
             [&] { return get(tw.ugrad, P * hp); }, [&] { return get(tw.dxg, P * dp); },
             [&] { return get(tw.dxu, P * dp); }, [&] { return get(tw.t, std::max(P, (size_t)cap) * R); },
             [&] { return get(tw.dx, (size_t)cap * d); }, [&] { return get(tw.lg, (size_t)cap * E); },
             [&] { return get(tw.lgf, (size_t)cap * E); }, [&] { return get(tw.dxr, (size_t)cap * dp); },
             [&] { return get(tw.pgroup, P); }, [&] { return get(tw.tiles_tr, P + L->G); },
             [&] { return get(tw.goff_router, (size_t)2); }, [&] { return get(tw.zero_bias, E); },
             [&] { return get(tw.partial, (size_t)tw.chunks * P * std::max(hp, dp)); },
             [&] { return get(tw.ot.tiles, P / lora_outer_tile_positions() + L->G); },
             [&] { return get(tw.ot.toff, (size_t)L->G + 1); }, [&] { return get(tw.ot.multi, (size_t)L->G); },
             [&] { return get(tw.rt.tiles, (size_t)cap / lora_outer_tile_positions() + 1); },
             [&] { return get(tw.rt.toff, (size_t)2); }, [&] { return get(tw.rt.multi, (size_t)1); },
             [&] { return get(tw.outer, (P / lora_outer_tile_positions() + L->G) * R * std::max({hp, dp, E})); }}) {
        rc = step();
        if (rc != GTMOE_OK) {
            free_train_workspace(tw);
            return rc;
        }
    }
    HIP_TRY(ctx, hipMemset(tw.zero_bias, 0, E * sizeof(double)));
    HIP_TRY(ctx, hipDeviceSynchronize());  // the memset runs on the null stream
    tw.cap = cap;
    return GTMOE_OK;
}

LoraArgs lora_args(const AdapterSet &a, int P, const int32_t *pgroup, const int32_t *goff,
                   const TrainWorkspace::OuterTiles *ot = nullptr)
{
    LoraArgs l{};
    l.A = a.A;
    l.B = a.B;
    l.scale = a.scale;
    l.R = a.R;
    l.kin = a.kin;
    l.width = a.width;
    l.rows = a.rows;
    l.G = a.G;
    l.P = P;
    l.pgroup = pgroup;
    l.goff = goff;
    if (ot) {
        l.otiles = ot->tiles;
        l.otoff = ot->toff;
        l.notiles = ot->n;
        l.omulti = ot->multi;
        l.nomulti = ot->nmulti;
    }
    return l;
}

RowsArgs rows_args(const DeviceMatrix &m, const float *in, int ld_in, const int32_t *in_tok, float *out, int ld_out,
                   const int4 *tiles)
{
    RowsArgs r{};
    r.values = m.values;
    r.scales = m.scales;
    r.w_group_stride = (long long)m.group_value_bytes();
    r.s_group_stride = (long long)m.group_scales();
    r.rows = m.rows;
    r.rows_p = m.rows_p;
    r.kp = m.kp;
    r.row_bytes = m.row_bytes;
    r.nblocks = m.nblocks;
    r.in = in;
    r.ld_in = ld_in;
    r.in_tok = in_tok;
    r.out = out;
    r.ld_out = ld_out;
    r.tiles = tiles;
    return r;
}

// Tiles of the adapter gradients over groups whose positions start at goff
// (goff.size() - 1 groups), uploaded to `ot` (the host copies stay alive
// until the stream has read them: the caller synchronizes before returning).
int32_t upload_outer_tiles(gtmoe_context *ctx, const std::vector<int32_t> &goff, TrainWorkspace::OuterTiles &ot,
                           hipStream_t s)
{
    const int G = (int)goff.size() - 1, n = lora_outer_tile_positions();
    ot.host_tiles.clear();
    ot.host_toff.assign(G + 1, 0);
    ot.host_multi.clear();
    for (int g = 0; g < G; ++g) {
        ot.host_toff[g] = (int32_t)ot.host_tiles.size();
        const int many = goff[g + 1] - goff[g] > n ? 1 : 0;
        if (many) ot.host_multi.push_back(g);
        for (int p = goff[g]; p < goff[g + 1]; p += n)
            ot.host_tiles.push_back(make_int4(g, p, std::min(n, goff[g + 1] - p), many));
    }
    ot.host_toff[G] = (int32_t)ot.host_tiles.size();
    ot.n = (int)ot.host_tiles.size();
    ot.nmulti = (int)ot.host_multi.size();
    HIP_TRY(ctx, hipMemcpyAsync(ot.tiles, ot.host_tiles.data(), sizeof(int4) * ot.n, hipMemcpyHostToDevice, s));
    HIP_TRY(ctx, hipMemcpyAsync(ot.toff, ot.host_toff.data(), sizeof(int32_t) * (G + 1), hipMemcpyHostToDevice, s));
    if (ot.nmulti)
        HIP_TRY(ctx, hipMemcpyAsync(ot.multi, ot.host_multi.data(), sizeof(int32_t) * ot.nmulti, hipMemcpyHostToDevice, s));
    return GTMOE_OK;
}

// Row chunks for the transposed product over `rows` rows: enough four-wave
// workgroups for about four waves per SIMD (one chunk when the tiles alone
// do that).
int transposed_chunks(const gtmoe_layer *L, int rows, int ntiles, int nblocks, int tile)
{
    const int busy = ntiles * rows_transposed_colblocks(nblocks, tile);
    const int unit = rows_transposed_chunk_rows(tile);
    int want = (4 * L->ctx->compute_units + busy - 1) / std::max(busy, 1);
    want = std::min(want, (rows + unit - 1) / unit);
    return std::max(1, std::min(want, L->tw.chunks));
}

// Forward through the adapter path (host float64 in and out).  Each layer:
// pre = (x W^T + s (x A^T) B^T) + b in fp32, kept with x A^T for Backward.
int32_t adapter_forward(gtmoe_layer *L, int T, const double *inputs, const int64_t *token_ids, double *outputs)
{
    gtmoe_context *ctx = L->ctx;
    Workspace &w = L->ws;
    hipStream_t s = ctx->stream;
    int32_t rc = ensure_train_workspace(L, T);
    if (rc != GTMOE_OK) return rc;
    TrainWorkspace &tw = L->tw;
    const int d = L->d, dp = L->dp, hp = L->hp, E = L->E, S = L->S, k = L->k, G = L->G;
    const bool hash = L->desc.use_hash_routing != 0;
    HIP_TRY(ctx, hipMemcpyAsync(w.x64, inputs, sizeof(double) * T * d, hipMemcpyHostToDevice, s));
    if (hash) HIP_TRY(ctx, hipMemcpyAsync(w.ids, token_ids, sizeof(int64_t) * T, hipMemcpyHostToDevice, s));
    RUN(ctx, s, "convert_inputs", launch_convert_inputs_f64(w.x64, T, d, w.xf, dp, nullptr, dp, s));
    if (hash) {
        RUN(ctx, s, "hash_route", launch_hash_route(w.ids, T, E, k, w.chosen, w.gates, w.gates32, s));
    } else {
        const int32_t goff_r[2] = {0, T};
        HIP_TRY(ctx, hipMemcpyAsync(tw.goff_router, goff_r, sizeof goff_r, hipMemcpyHostToDevice, s));
        RUN(ctx, s, "router", launch_router(w.xf, dp, T, d, L->router_w, dp, tw.zero_bias, E, w.logits, s));
        const LoraArgs ar = lora_args(L->ad_router, T, nullptr, tw.goff_router);
        RUN(ctx, s, "lora_down", launch_lora_down(ar, w.xf, dp, nullptr, tw.u_router, s));
        RUN(ctx, s, "lora_up_bias", launch_lora_up_bias_f64(ar, tw.u_router, w.logits, E, L->router_b, s));
        RUN(ctx, s, "topk", launch_topk(w.logits, T, E, k, L->balance, w.chosen, w.gates, w.gates32, s));
    }
    L->skipped_dispatch = false;
    RUN(ctx, s, "dispatch",
        launch_dispatch(w.chosen, T, k, E, S, kGemvSlice, w.load, w.offsets, w.rows, w.pos, w.goff, w.tok,
                        w.tile_off, w.tile_desc, w.chunk_cnt, s));
    // positions of every group, and work tiles over them
    std::vector<int32_t> goff(G + 1);
    HIP_TRY(ctx, hipMemcpyAsync(goff.data(), w.goff, sizeof(int32_t) * (G + 1), hipMemcpyDeviceToHost, s));
    HIP_TRY(ctx, hipStreamSynchronize(s));
    const int P = goff[G];
    if (P != T * (S + k)) return fail(ctx, GTMOE_ERR_DEVICE, "dispatch placed %d positions, expected %d", P, T * (S + k));
    std::vector<int32_t> pgroup(P);
    std::vector<int4> ttr;
    const int bt = rows_transposed_tile(P, G);
    for (int g = 0; g < G; ++g) {
        for (int p = goff[g]; p < goff[g + 1]; ++p) pgroup[p] = g;
        for (int p = goff[g]; p < goff[g + 1]; p += bt) ttr.push_back(make_int4(g, p, std::min(bt, goff[g + 1] - p), 0));
    }
    HIP_TRY(ctx, hipMemcpyAsync(tw.pgroup, pgroup.data(), sizeof(int32_t) * P, hipMemcpyHostToDevice, s));
    HIP_TRY(ctx, hipMemcpyAsync(tw.tiles_tr, ttr.data(), sizeof(int4) * ttr.size(), hipMemcpyHostToDevice, s));
    tw.P = P;
    tw.ntiles_tr = (int)ttr.size();
    tw.tile_tr = bt;
    rc = upload_outer_tiles(ctx, goff, tw.ot, s);
    if (rc == GTMOE_OK) rc = upload_outer_tiles(ctx, {0, T}, tw.rt, s);
    if (rc != GTMOE_OK) return rc;

    // the bare products x W^T by the decode GEMV kernels (raw mode, over the
    // dispatch's slices), then the adapter terms and the biases
    const int slices = S * ((T + kGemvSlice - 1) / kGemvSlice) + (T * k + kGemvSlice - 1) / kGemvSlice + E;
    GemvArgs a{};
    a.w0 = L->gate.values;
    a.s0 = L->gate.scales;
    a.b0 = L->gate.biases;
    a.w1 = L->up.values;
    a.s1 = L->up.scales;
    a.b1 = L->up.biases;
    a.w_group_stride = (long long)L->gate.group_value_bytes();
    a.s_group_stride = (long long)L->gate.group_scales();
    a.rows = L->h;
    a.nblocks = L->gate.nblocks;
    a.row_bytes = L->gate.row_bytes;
    a.in = w.xf;
    a.ld_in = dp;
    a.in_rows = w.cap;
    a.tok = w.tok;
    a.count = w.tile_off + G;
    a.desc = w.tile_desc;
    a.out = tw.gpre;
    a.ld_out = hp;
    a.raw = 1;
    a.raw_up = tw.upre;
    RUN(ctx, s, "gemv_gateup", launch_gemv_gateup(a, L->gate.precision, slices, s));
    const float limit = (float)L->desc.clamp_limit;
    struct Role {
        const DeviceMatrix &m;
        const AdapterSet &a;
        float *pre, *u;
    };
    for (const Role &r : {Role{L->gate, L->ad_gate, tw.gpre, tw.u_gate}, Role{L->up, L->ad_up, tw.upre, tw.u_up}}) {
        const LoraArgs la = lora_args(r.a, P, tw.pgroup, w.goff);
        RUN(ctx, s, "lora_down", launch_lora_down(la, w.xf, dp, w.tok, r.u, s));
        RUN(ctx, s, "lora_up_bias", launch_lora_up_bias(la, r.u, r.pre, hp, r.m.biases, s));
    }
    RUN(ctx, s, "swiglu", launch_swiglu_forward(tw.gpre, tw.upre, P, L->h, hp, limit, w.hidden32, s));
    GemvArgs b{};
    b.w0 = L->down.values;
    b.s0 = L->down.scales;
    b.b0 = L->down.biases;
    b.w_group_stride = (long long)L->down.group_value_bytes();
    b.s_group_stride = (long long)L->down.group_scales();
    b.rows = d;
    b.nblocks = L->down.nblocks;
    b.row_bytes = L->down.row_bytes;
    b.in = w.hidden32;
    b.ld_in = hp;
    b.in_rows = (long long)w.cap * (S + k);
    b.count = w.tile_off + G;
    b.desc = w.tile_desc;
    b.out = w.slot_out;
    b.ld_out = d;
    b.raw = 1;
    RUN(ctx, s, "gemv_down", launch_gemv_down(b, L->down.precision, slices, s));
    const LoraArgs ld = lora_args(L->ad_down, P, tw.pgroup, w.goff);
    RUN(ctx, s, "lora_down", launch_lora_down(ld, w.hidden32, hp, nullptr, tw.u_down, s));
    RUN(ctx, s, "lora_up_bias", launch_lora_up_bias(ld, tw.u_down, w.slot_out, d, L->down.biases, s));
    RUN(ctx, s, "combine",
        launch_combine(T, d, S, k, w.slot_out, false, w.pos, w.gates32, nullptr, nullptr, w.y64, s));
    HIP_TRY(ctx, hipMemcpyAsync(outputs, w.y64, sizeof(double) * T * d, hipMemcpyDeviceToHost, s));
    L->last_load.assign(E, 0);
    HIP_TRY(ctx, hipMemcpyAsync(L->last_load.data(), w.load, sizeof(int32_t) * E, hipMemcpyDeviceToHost, s));
    HIP_TRY(ctx, hipStreamSynchronize(s));
    mark_forward(L, T, GTMOE_PATH_FP32, s);
    L->load_on_host = true;
    L->relaunch_ready = false;
    L->adapter_T = T;
    return GTMOE_OK;
}

// MixtureOfExperts.Backward (mixtureofexperts.go:227-285) after an adapter
// path forward of T tokens: adapter gradients are added to dA / dB, the
// input gradients returned (host float64).
int32_t adapter_backward(gtmoe_layer *L, int T, const double *output_grads, double *input_grads)
{
    gtmoe_context *ctx = L->ctx;
    Workspace &w = L->ws;
    TrainWorkspace &tw = L->tw;
    hipStream_t s = ctx->stream;
    const int d = L->d, dp = L->dp, hp = L->hp, E = L->E, S = L->S, k = L->k, P = tw.P;
    const float limit = (float)L->desc.clamp_limit;
    HIP_TRY(ctx, hipMemcpyAsync(tw.og, output_grads, sizeof(double) * T * d, hipMemcpyHostToDevice, s));
    // down layer: its pre-activation gradient is the expert output gradient
    RUN(ctx, s, "expert_output_grad",
        launch_expert_output_grad(tw.og, d, d, w.tok, tw.pgroup, S, T, k, w.chosen, w.gates, P, tw.eg, s));
    auto transposed = [&](const DeviceMatrix &m, const float *in, int ld_in, float *out, int ld_out) {
        RowsArgs r = rows_args(m, in, ld_in, nullptr, out, ld_out, tw.tiles_tr);
        r.tiles_positions = P;
        const int chunks = transposed_chunks(L, m.rows, tw.ntiles_tr, m.nblocks, tw.tile_tr);
        return launch_rows_transposed(r, m.precision, tw.ntiles_tr, tw.tile_tr, chunks, tw.partial, s);
    };
    RUN(ctx, s, "rows_transposed", transposed(L->down, tw.eg, d, tw.hgrad, hp));
    RUN(ctx, s, "lora_backward",
        launch_lora_backward(lora_args(L->ad_down, P, tw.pgroup, w.goff, &tw.ot), tw.eg, d,
                             tw.u_down, w.hidden32, hp, nullptr, tw.t, tw.hgrad, hp, L->ad_down.dA, L->ad_down.dB,
                             tw.outer, s));
    RUN(ctx, s, "swiglu_backward",
        launch_swiglu_backward(tw.hgrad, tw.gpre, tw.upre, P, L->h, hp, limit, tw.ggrad, tw.ugrad, s));
    struct Role {
        const DeviceMatrix &m;
        AdapterSet &a;
        float *grad, *u, *dx;
    };
    for (const Role &r : {Role{L->gate, L->ad_gate, tw.ggrad, tw.u_gate, tw.dxg},
                          Role{L->up, L->ad_up, tw.ugrad, tw.u_up, tw.dxu}}) {
        RUN(ctx, s, "rows_transposed", transposed(r.m, r.grad, hp, r.dx, dp));
        RUN(ctx, s, "lora_backward",
            launch_lora_backward(lora_args(r.a, P, tw.pgroup, w.goff, &tw.ot), r.grad, hp,
                                 r.u, w.xf, dp, w.tok, tw.t, r.dx, dp, r.a.dA, r.a.dB, tw.outer, s));
    }
    RUN(ctx, s, "gather_input_grad", launch_gather_input_grad(tw.dxg, tw.dxu, dp, d, T, S, k, w.pos, tw.dx, s));
    if (!L->desc.use_hash_routing) {
        RUN(ctx, s, "router_backward",
            launch_router_backward(tw.og, d, w.slot_out, d, w.chosen, w.gates, w.logits, w.pos, S, T, E, k, tw.lg,
                                   tw.lgf, s));
        RUN(ctx, s, "router_input_grad", launch_router_input_grad(tw.lgf, T, E, L->router_w, dp, d, tw.dxr, dp, s));
        RUN(ctx, s, "lora_backward",
            launch_lora_backward(lora_args(L->ad_router, T, nullptr, tw.goff_router, &tw.rt),
                                 tw.lgf, E, tw.u_router, w.xf, dp, nullptr, tw.t, tw.dxr, dp, L->ad_router.dA,
                                 L->ad_router.dB, tw.outer, s));
        RUN(ctx, s, "add_rows", launch_add_rows_f64(tw.dxr, dp, d, T, tw.dx, s));
    }
    HIP_TRY(ctx, hipMemcpyAsync(input_grads, tw.dx, sizeof(double) * T * d, hipMemcpyDeviceToHost, s));
    HIP_TRY(ctx, hipStreamSynchronize(s));
    return GTMOE_OK;
}

}  // namespace

extern "C" {

int32_t gtmoe_abi_version(void) { return GTMOE_ABI_VERSION; }

int32_t gtmoe_device_count(int32_t *count)
{
    if (!count) return GTMOE_ERR_INVALID_ARGUMENT;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    *count = n;
    return GTMOE_OK;
}

int32_t gtmoe_open(int32_t device, gtmoe_context **out)
{
    if (!out) return fail(nullptr, GTMOE_ERR_INVALID_ARGUMENT, "out is null");
    *out = nullptr;
    int32_t injected = GTMOE_OK;
    if (take_injection(__func__, &injected)) return fail(nullptr, injected, "injected failure in %s", __func__);
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) return fail(nullptr, GTMOE_ERR_DEVICE, "no HIP device: %s", hipGetErrorString(e));
    if (device < 0 || device >= n) return fail(nullptr, GTMOE_ERR_INVALID_ARGUMENT, "device %d of %d", device, n);
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess)
        return fail(nullptr, GTMOE_ERR_DEVICE, "cannot read properties of device %d", device);
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(nullptr, GTMOE_ERR_UNSUPPORTED, "device %d is %s; this library is built for gfx950", device,
                    prop.gcnArchName);
    if (hipSetDevice(device) != hipSuccess) return fail(nullptr, GTMOE_ERR_DEVICE, "hipSetDevice(%d) failed", device);
    gtmoe_context *ctx = new gtmoe_context;
    ctx->device = device;
    ctx->scratch = scratch_address(device, ctx->scratch_error);
    if (prop.multiProcessorCount > 0) ctx->compute_units = prop.multiProcessorCount;
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return fail(nullptr, GTMOE_ERR_DEVICE, "cannot create a stream");
    }
    *out = ctx;
    return GTMOE_OK;
}

static void close_locked(gtmoe_context *ctx)
{
    if (ctx->closed) return;  // closing twice does nothing (gpu/gpu_test.go:145-154)
    (void)hipSetDevice(ctx->device);
    (void)hipDeviceSynchronize();
    for (auto &r : ctx->pending) {
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
    }
    ctx->pending.clear();
    for (auto e : ctx->spare_events) (void)hipEventDestroy(e);
    ctx->spare_events.clear();
    (void)hipStreamDestroy(ctx->stream);
    ctx->stream = nullptr;
    ctx->totals.clear();
    // The handle is not freed: a closed context keeps answering, as a closed
    // gpu.Device does (gpu/device.go:729-731), with an error instead of work,
    // until gtmoe_context_free lets it go.
    ctx->closed = true;
}

int32_t gtmoe_close(gtmoe_context *ctx)
{
    if (!ctx) return GTMOE_ERR_INVALID_ARGUMENT;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    close_locked(ctx);
    return GTMOE_OK;
}

int32_t gtmoe_context_free(gtmoe_context *ctx)
{
    if (!ctx) return GTMOE_ERR_INVALID_ARGUMENT;
    {
        std::lock_guard<std::recursive_mutex> lock(ctx->mu);
        close_locked(ctx);
    }
    release_context(ctx);  // the handle's reference
    return GTMOE_OK;
}

const char *gtmoe_last_error(const gtmoe_context *ctx)
{
    return ctx ? ctx->error.c_str() : g_open_error.c_str();
}

int32_t gtmoe_test_device_allocations(int64_t *allocations, int64_t *frees)
{
    if (allocations) *allocations = g_device_allocations.load(std::memory_order_relaxed);
    if (frees) *frees = g_device_frees.load(std::memory_order_relaxed);
    return GTMOE_OK;
}

int32_t gtmoe_test_inject_failure(const char *entry_point, int32_t status)
{
    if (!entry_point || status < GTMOE_OK || status > GTMOE_ERR_OUT_OF_MEMORY) return GTMOE_ERR_INVALID_ARGUMENT;
    g_inject_entry = entry_point;
    g_inject_status = status;
    return GTMOE_OK;
}

int32_t gtmoe_layer_create(gtmoe_context *ctx, const gtmoe_layer_desc *desc, gtmoe_layer **out)
{
    if (!ctx || !desc || !out) return GTMOE_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    ENTER(ctx);
    const gtmoe_layer_desc &D = *desc;
    // buildMixtureOfExperts checks (mixtureofexperts.go:47-56) and NewLayer's
    if (D.shared_experts < 0)
        return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "number of shared experts can't be negative, got %d",
                    D.shared_experts);
    if (D.routed_experts < 1)
        return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "needs at least 1 routed expert, got %d", D.routed_experts);
    if (D.experts_per_token < 1 || D.experts_per_token > D.routed_experts)
        return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "experts per token must be between 1 and %d, got %d",
                    D.routed_experts, D.experts_per_token);
    if (D.vector_size < 1 || D.expert_hidden_size < 1)
        return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "vector size and hidden size must be at least 1");
    if (D.clamp_limit < 0) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "clamp limit must be above 0");
    if (D.routed_experts > kMaxExperts)
        return fail(ctx, GTMOE_ERR_UNSUPPORTED, "at most %d routed experts on the GPU, got %d", kMaxExperts,
                    D.routed_experts);
    if (D.shared_experts + D.routed_experts > 1024)
        return fail(ctx, GTMOE_ERR_UNSUPPORTED, "at most 1024 experts in all on the GPU, got %d",
                    D.shared_experts + D.routed_experts);
    if (D.experts_per_token > kMaxK)
        return fail(ctx, GTMOE_ERR_UNSUPPORTED, "at most %d experts per token on the GPU, got %d", kMaxK,
                    D.experts_per_token);
    if (D.precision != GTMOE_FLOAT32 && D.precision != GTMOE_INT8 && D.precision != GTMOE_FP4)
        return fail(ctx, GTMOE_ERR_UNSUPPORTED, "expert weights at precision %d are not offered on the GPU",
                    D.precision);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    gtmoe_layer *L = new gtmoe_layer;
    L->ctx = ctx;
    ++ctx->refs;  // dropped by gtmoe_layer_destroy
    L->desc = D;
    L->d = D.vector_size;
    L->h = D.expert_hidden_size;
    L->S = D.shared_experts;
    L->E = D.routed_experts;
    L->k = D.experts_per_token;
    L->G = L->S + L->E;
    L->dp = pad_k(L->d);
    L->hp = pad_k(L->h);
    L->balance_host.assign(L->E, 0.0);
    L->uploaded.assign(1 + 3 * L->G, 0);
    int32_t rc = GTMOE_OK;
    if (rc == GTMOE_OK) rc = alloc_matrix(ctx, L->gate, D.precision, L->h, L->d, L->G);
    if (rc == GTMOE_OK) rc = alloc_matrix(ctx, L->up, D.precision, L->h, L->d, L->G);
    if (rc == GTMOE_OK) rc = alloc_matrix(ctx, L->down, D.precision, L->d, L->h, L->G);
    if (rc == GTMOE_OK) {
        const size_t rw = (size_t)L->E * L->dp * sizeof(float);
        if (dev_malloc(&L->router_w, rw) != hipSuccess || hipMemset(L->router_w, 0, rw) != hipSuccess ||
            dev_malloc(&L->router_b, sizeof(double) * L->E) != hipSuccess ||
            hipMemset(L->router_b, 0, sizeof(double) * L->E) != hipSuccess ||
            dev_malloc(&L->balance, sizeof(double) * L->E) != hipSuccess ||
            hipMemset(L->balance, 0, sizeof(double) * L->E) != hipSuccess ||
            dev_malloc(&L->norm_w, sizeof(float) * L->d) != hipSuccess ||
            dev_malloc(&L->router_wn, rw) != hipSuccess || hipMemset(L->router_wn, 0, rw) != hipSuccess)
            rc = fail(ctx, GTMOE_ERR_OUT_OF_MEMORY, "cannot allocate the router");
    }
    // the zeroing memsets above run on the null stream (see ensure_workspace)
    if (rc == GTMOE_OK && hipDeviceSynchronize() != hipSuccess) rc = fail(ctx, GTMOE_ERR_DEVICE, "device sync failed");
    if (rc != GTMOE_OK) {
        gtmoe_layer_destroy(L);
        return rc;
    }
    *out = L;
    return GTMOE_OK;
}

int32_t gtmoe_layer_destroy(gtmoe_layer *L)
{
    if (!L) return GTMOE_ERR_INVALID_ARGUMENT;
    gtmoe_context *ctx = L->ctx;
    {
        std::lock_guard<std::recursive_mutex> lock(ctx->mu);
        if (L->live_graphs > 0)
            return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT,
                        "the layer is part of %d recorded graph(s); destroy them first", L->live_graphs);
        (void)hipSetDevice(ctx->device);
        (void)hipDeviceSynchronize();
        free_adapters(L);
        free_matrix(L->gate);
        free_matrix(L->up);
        free_matrix(L->down);
        for (void *p : {(void *)L->router_w, (void *)L->router_b, (void *)L->balance, (void *)L->norm_w,
                        (void *)L->router_wn, L->ws.base})
            if (p) (void)dev_free(p);
        if (L->stage) (void)pinned_free(L->stage);
        delete L;
    }
    release_context(ctx);  // the layer's reference
    return GTMOE_OK;
}

int32_t gtmoe_upload_rows(gtmoe_layer *L, int32_t role, int32_t index, const gtmoe_rows *rows, const double *biases)
{
    if (!L) return GTMOE_ERR_INVALID_ARGUMENT;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    if (!biases) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "biases are null");
    if (role < GTMOE_ROLE_ROUTER || role > GTMOE_ROLE_ROUTED_DOWN)
        return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "unknown role %d", role);
    {
        const int32_t rc0 = settle_device_work(L);  // a forward may still read the matrix
        if (rc0 != GTMOE_OK) return rc0;
    }

    if (role == GTMOE_ROLE_ROUTER) {
        int32_t rc = check_rows(ctx, rows, L->E, L->d);
        if (rc != GTMOE_OK) return rc;
        // the router runs in fp32: decode the rows and round to float
        std::vector<float> w((size_t)L->E * L->dp, 0.f);
        for (int r = 0; r < L->E; ++r)
            for (int i = 0; i < L->d; ++i) w[(size_t)r * L->dp + i] = (float)decoded_value(rows, r, i);
        HIP_TRY(ctx, hipMemcpy(L->router_w, w.data(), w.size() * sizeof(float), hipMemcpyHostToDevice));
        HIP_TRY(ctx, hipMemcpy(L->router_b, biases, sizeof(double) * L->E, hipMemcpyHostToDevice));
        L->router_host.swap(w);
        L->uploaded[role_slot(L, role, 0)] = 1;
        return refresh_folded_router(L);
    }

    const bool shared = role <= GTMOE_ROLE_SHARED_DOWN;
    const int n = shared ? L->S : L->E;
    if (index < 0 || index >= n)
        return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "%s expert %d of %d", shared ? "shared" : "routed", index, n);
    const int which = shared ? role - GTMOE_ROLE_SHARED_GATE : role - GTMOE_ROLE_ROUTED_GATE;
    DeviceMatrix &m = which == 0 ? L->gate : which == 1 ? L->up : L->down;
    int32_t rc = check_rows(ctx, rows, m.rows, m.width);
    if (rc != GTMOE_OK) return rc;
    if (rows->precision != m.precision)
        return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "expert weights at precision %d, the layer holds %d",
                    rows->precision, m.precision);
    const int group = shared ? index : L->S + index;
    // repack into the panel layout (16-byte units of 64 rows side by side)
    std::vector<uint8_t> vals(m.group_value_bytes(), 0);
    const int src_row_bytes = m.precision == kInt8 ? m.width : m.precision == kFP4 ? (m.width + 1) / 2 : m.width * 4;
    for (int r = 0; r < m.rows; ++r) {
        const uint8_t *src = (const uint8_t *)rows->values + (size_t)r * src_row_bytes;
        for (int u = 0; u * 16 < src_row_bytes; ++u)
            memcpy(vals.data() + panel_unit_offset(r, u, m.row_bytes), src + (size_t)u * 16,
                   (size_t)std::min(16, src_row_bytes - u * 16));
    }
    HIP_TRY(ctx, hipMemcpy((char *)m.values + (size_t)group * m.group_value_bytes(), vals.data(), vals.size(),
                           hipMemcpyHostToDevice));
    if (m.precision == kFloat32) {  // and the group's bf16 copy for the prefill GEMM
        HIP_TRY(ctx, launch_bf16_rows((char *)m.values + (size_t)group * m.group_value_bytes(),
                                      (char *)m.bf16 + (size_t)group * m.group_bf16_bytes(), m.rows_p, m.kp, nullptr));
        HIP_TRY(ctx, hipStreamSynchronize(nullptr));
    }
    if (m.precision != kFloat32) {
        const int src_blocks = (m.width + 15) / 16;
        std::vector<float> sc(m.group_scales(), 0.f);
        for (int r = 0; r < m.rows; ++r)
            for (int b = 0; b < src_blocks; ++b)
                sc[panel_scale_index(r, b, m.nblocks)] = rows->scales[(size_t)r * src_blocks + b];
        HIP_TRY(ctx, hipMemcpy(m.scales + (size_t)group * m.group_scales(), sc.data(), sc.size() * sizeof(float),
                               hipMemcpyHostToDevice));
    }
    std::vector<float> b(m.rows);
    for (int r = 0; r < m.rows; ++r) b[r] = (float)biases[r];
    HIP_TRY(ctx, hipMemcpy(m.biases + (size_t)group * m.rows, b.data(), sizeof(float) * m.rows, hipMemcpyHostToDevice));
    L->uploaded[role_slot(L, role, index)] = 1;
    return GTMOE_OK;
}

int32_t gtmoe_set_balance_biases(gtmoe_layer *L, const double *biases)
{
    if (!L || !biases) return GTMOE_ERR_INVALID_ARGUMENT;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    // the Go side hands the biases over on every forward: unchanged values
    // (bit for bit) need no copy
    if (memcmp(L->balance_host.data(), biases, sizeof(double) * L->E) == 0) return GTMOE_OK;
    int32_t rc = settle_device_work(L);
    if (rc != GTMOE_OK) return rc;
    L->balance_host.assign(biases, biases + L->E);
    HIP_TRY(ctx, hipMemcpy(L->balance, biases, sizeof(double) * L->E, hipMemcpyHostToDevice));
    return GTMOE_OK;
}

int32_t gtmoe_get_balance_biases(const gtmoe_layer *L, double *biases)
{
    if (!L || !biases) return GTMOE_ERR_INVALID_ARGUMENT;
    memcpy(biases, L->balance_host.data(), sizeof(double) * L->E);
    return GTMOE_OK;
}

int32_t gtmoe_set_norm_weights(gtmoe_layer *L, const double *weights)
{
    if (!L || !weights) return GTMOE_ERR_INVALID_ARGUMENT;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    int32_t rc = settle_device_work(L);
    if (rc != GTMOE_OK) return rc;
    std::vector<float> w(weights, weights + L->d);
    HIP_TRY(ctx, hipMemcpy(L->norm_w, w.data(), sizeof(float) * L->d, hipMemcpyHostToDevice));
    L->norm_host.swap(w);
    L->has_norm = true;
    return refresh_folded_router(L);
}

int32_t gtmoe_forward(gtmoe_layer *L, int32_t tokens, const double *inputs, const int64_t *token_ids,
                      double *outputs, uint32_t flags)
{
    int32_t rc = check_layer_call(L);
    if (rc != GTMOE_OK) return rc;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    const int T = tokens;
    if (T < 0) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "negative number of tokens");
    if (T > 0 && (!inputs || !outputs)) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "inputs or outputs are null");
    if (flags > GTMOE_PATH_BF16) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "unknown flags %u", flags);
    if (L->desc.use_hash_routing) {
        if (T > 0 && !token_ids)
            return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "mixture of experts: hash routing needs one token ID per row");
        for (int t = 0; t < T; ++t)
            if (token_ids[t] < 0)
                return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "mixture of experts: token ID %lld at row %d is negative",
                            (long long)token_ids[t], t);
    }
    const int path = choose_path(L, T, flags);
    if (path == GTMOE_PATH_FP32 && (L->dp > kMaxGemvK || L->hp > kMaxGemvK))
        return fail(ctx, GTMOE_ERR_UNSUPPORTED, "the fp32 path takes vector and hidden sizes up to %d", kMaxGemvK);
    rc = settle_device_work(L);
    if (rc == GTMOE_OK) rc = ensure_workspace(L, T);
    if (rc != GTMOE_OK) return rc;
    hipStream_t s = ctx->stream;
    if (T == 0) {
        mark_forward(L, 0, path, s);
        L->last_load.assign(L->E, 0);
        L->load_on_host = true;
        if (L->has_adapters) L->adapter_T = 0;
        return GTMOE_OK;
    }
    if (L->has_adapters) return adapter_forward(L, T, inputs, token_ids, outputs);
    Workspace &w = L->ws;
    // The host buffers are bridged by pinned staging that the kernels read
    // and write across the bus themselves.  The CPU rounds the float64 rows
    // to fp32 into it (every kernel's first step for float64 rows, so the
    // results are the same, and half the bytes cross the bus) and copies the
    // ids; the routing kernel reads the rows there.  The combine, which adds
    // in fp32, writes the fp32 output rows there and the CPU widens them
    // (exactly); the routing state is gathered there by the one-workgroup
    // dispatch when that runs here, else by a pack kernel; the call waits
    // for the device once.  The routing state comes back with the outputs
    // because the reference keeps it (LastExpertLoad, UpdateBalance,
    // Backward) and the Go side reads it after every forward; the dispatch
    // tables, which the few-token kernels did without, are built behind the
    // expert kernels first.
    const size_t nvals = (size_t)T * L->d;
    const size_t rows_bytes = align_up(sizeof(float) * nvals, 64);
    const size_t tk = (size_t)T * L->k;
    const int words[] = {L->E, (int)tk, (int)(2 * tk), (int)tk, L->E + 1};  // load, chosen, gates, rows, offsets
    size_t route_bytes = 0;
    for (int n : words) route_bytes += (size_t)(n + 15) / 16 * 64;
    const size_t ids_bytes = align_up(sizeof(int64_t) * T, 64);
    rc = ensure_stage(L, 2 * rows_bytes + ids_bytes + route_bytes);
    if (rc != GTMOE_OK) return rc;
    const size_t ox = 0, oy = rows_bytes, oid = 2 * rows_bytes, oroute = oid + ids_bytes;
    float *hx = reinterpret_cast<float *>(L->stage + ox);
    for (size_t i = 0; i < nvals; ++i) hx[i] = (float)inputs[i];
    const int64_t *ids = nullptr;
    if (L->desc.use_hash_routing) {
        memcpy(L->stage + oid, token_ids, sizeof(int64_t) * T);
        ids = reinterpret_cast<const int64_t *>(L->stage_dev + oid);
    }
    rc = prepare_and_route(L, T, Inputs{L->stage_dev + ox, false, false, true}, ids, path, s);
    if (rc == GTMOE_OK) rc = run_experts(L, T, path, s);
    if (rc != GTMOE_OK) return rc;
    RUN(ctx, s, "combine",
        launch_combine(T, L->d, L->S, L->k, w.slot_out, path == GTMOE_PATH_BF16, L->skipped_dispatch ? nullptr : w.pos,
                       w.gates32, nullptr, reinterpret_cast<float *>(L->stage_dev + oy), nullptr, s));
    PackParts pp{};
    const void *srcs[] = {w.load, w.chosen, w.gates, w.rows, w.offsets};
    for (int i = 0; i < 5; ++i) {
        pp.src[i] = static_cast<const uint32_t *>(srcs[i]);
        pp.words[i] = words[i];
    }
    pp.n = 5;
    uint32_t *route_dst = reinterpret_cast<uint32_t *>(L->stage_dev + oroute);
    if (L->skipped_dispatch && !dispatch_chunked(T))  // the dispatch packs the state in the same launch
        RUN(ctx, s, "dispatch",
            launch_dispatch_packed(w.chosen, T, L->k, L->E, L->S, kGemvSlice, w.load, w.offsets, w.rows, w.pos,
                                   w.goff, w.tok, w.tile_off, w.tile_desc, pp, route_dst, s));
    else {
        if (L->skipped_dispatch)
            RUN(ctx, s, "dispatch",
                launch_dispatch(w.chosen, T, L->k, L->E, L->S, kGemvSlice, w.load, w.offsets, w.rows, w.pos, w.goff,
                                w.tok, w.tile_off, w.tile_desc, w.chunk_cnt, s));
        RUN(ctx, s, "pack_routing", launch_pack_words(pp, route_dst, s));
    }
    HIP_TRY(ctx, hipStreamSynchronize(s));
    const float *hy = reinterpret_cast<const float *>(L->stage + oy);
    for (size_t i = 0; i < nvals; ++i) outputs[i] = (double)hy[i];
    mark_forward(L, T, path, s);
    L->skipped_dispatch = false;
    L->dispatch_pending = false;
    const char *part = L->stage + oroute;
    auto next = [&](int i) {
        const char *p = part;
        part += (size_t)(words[i] + 15) / 16 * 64;
        return p;
    };
    const int32_t *hload = (const int32_t *)next(0), *hchosen = (const int32_t *)next(1);
    const double *hgates = (const double *)next(2);
    const int32_t *hrows = (const int32_t *)next(3), *hoffsets = (const int32_t *)next(4);
    L->last_load.assign(hload, hload + L->E);
    L->load_on_host = true;
    L->host_chosen.assign(hchosen, hchosen + tk);
    L->host_gates.assign(hgates, hgates + tk);
    L->host_rows.assign(hrows, hrows + tk);
    L->host_offsets.assign(hoffsets, hoffsets + L->E + 1);
    L->routing_on_host = true;
    return GTMOE_OK;
}

// Checks of gtmoe_forward_device's arguments; leaves the resolved path.
static int32_t check_forward_device(gtmoe_layer *L, int32_t T, const float *inputs, const int64_t *token_ids,
                                    const float *outputs, uint32_t flags, int *path)
{
    gtmoe_context *ctx = L->ctx;
    if (T < 0) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "negative number of tokens");
    if (T > 0 && (!inputs || !outputs)) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "inputs or outputs are null");
    if (flags > GTMOE_PATH_BF16) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "unknown flags %u", flags);
    if (L->desc.use_hash_routing && T > 0 && !token_ids)
        return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "mixture of experts: hash routing needs one token ID per row");
    if (L->has_adapters)
        return fail(ctx, GTMOE_ERR_UNSUPPORTED, "a layer with low-rank adapters runs through gtmoe_forward");
    if (T > 0) {
        // the routing may clear the outputs while rows of the inputs are
        // still being read: the two buffers must not overlap
        const uintptr_t a = (uintptr_t)inputs, b = (uintptr_t)outputs;
        const uintptr_t n = (uintptr_t)T * (uintptr_t)L->d * sizeof(float);
        if (a < b + n && b < a + n)
            return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "inputs and outputs overlap; a forward cannot run in place");
    }
    *path = choose_path(L, T, flags);
    if (*path == GTMOE_PATH_FP32 && (L->dp > kMaxGemvK || L->hp > kMaxGemvK))
        return fail(ctx, GTMOE_ERR_UNSUPPORTED, "the fp32 path takes vector and hidden sizes up to %d", kMaxGemvK);
    return GTMOE_OK;
}

// The kernels of one device forward, enqueued on s.
static int32_t forward_device_run(gtmoe_layer *L, int32_t T, const float *inputs, const int64_t *token_ids,
                                  float *outputs, int path, hipStream_t s)
{
    gtmoe_context *ctx = L->ctx;
    if (T == 0) {
        mark_forward(L, 0, path, s);
        return GTMOE_OK;
    }
    Workspace &w = L->ws;
    // With at most two contributions per output row the fp32 path folds the
    // combine into the down kernel (order-independent adds onto zeroed rows).
    float *fold = path == GTMOE_PATH_FP32 && L->S + L->k <= 2 ? outputs : nullptr;
    int32_t rc = prepare_and_route(L, T, Inputs{inputs, false, false}, token_ids, path, s, fold);
    if (rc == GTMOE_OK) rc = run_experts(L, T, path, s, fold);
    if (rc != GTMOE_OK) return rc;
    if (!fold)
        RUN(ctx, s, "combine",
            launch_combine(T, L->d, L->S, L->k, w.slot_out, path == GTMOE_PATH_BF16, L->skipped_dispatch ? nullptr : w.pos, w.gates32, nullptr,
                           outputs, nullptr, s));
    mark_forward(L, T, path, s);
    return GTMOE_OK;
}

int32_t gtmoe_forward_device(gtmoe_layer *L, int32_t tokens, const float *inputs, const int64_t *token_ids,
                             float *outputs, uint32_t flags, void *stream)
{
    int32_t rc = check_layer_call(L);
    if (rc != GTMOE_OK) return rc;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    int path = 0;
    rc = check_forward_device(L, tokens, inputs, token_ids, outputs, flags, &path);
    if (rc == GTMOE_OK) rc = ensure_workspace(L, tokens);
    if (rc != GTMOE_OK) return rc;
    return forward_device_run(L, tokens, inputs, token_ids, outputs, path, (hipStream_t)stream);
}

int32_t gtmoe_forward_device_noalloc(gtmoe_layer *L, int32_t tokens, const float *inputs, const int64_t *token_ids,
                                     float *outputs, uint32_t flags, void *stream)
{
    int32_t rc = check_layer_call(L);
    if (rc != GTMOE_OK) return rc;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    int path = 0;
    rc = check_forward_device(L, tokens, inputs, token_ids, outputs, flags, &path);
    if (rc != GTMOE_OK) return rc;
    if (!ctx->scratch)
        return fail(ctx, GTMOE_ERR_DEVICE, "no scratch area on device %d (%s)", ctx->device,
                    ctx->scratch_error.c_str());
    const int T = tokens;
    Workspace w{};
    const size_t need = layout_workspace(L, T > 0 ? T : 1, false, nullptr, w);
    if (need > (size_t)GTMOE_NOALLOC_SCRATCH_BYTES)
        return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT,
                    "a forward of %d tokens on this layer needs %zu bytes of intermediates; the forward without "
                    "allocation has %zu",
                    T, need, (size_t)GTMOE_NOALLOC_SCRATCH_BYTES);
    hipStream_t s = (hipStream_t)stream;
    layout_workspace(L, T > 0 ? T : 1, false, (char *)ctx->scratch, w);
    auto enqueue = [&]() -> int32_t {
        // Padding columns of the activation rows are read (against zero
        // weights) and never written; the area holds whatever the last call
        // on this GPU left, so they are cleared here (fill kernels, no memset
        // nodes under graph capture).
        if (T > 0 && L->dp != L->d) {
            RUN(ctx, s, "clear_scratch", launch_fill_i32(reinterpret_cast<int32_t *>(w.xf), T * L->dp, 0, s));
            RUN(ctx, s, "clear_scratch", launch_fill_i32(reinterpret_cast<int32_t *>(w.xb), T * L->dp / 2, 0, s));
        }
        if (T > 0 && L->hp != L->h) {
            const int P = T * (L->S + L->k);
            RUN(ctx, s, "clear_scratch", launch_fill_i32(reinterpret_cast<int32_t *>(w.hidden32), P * L->hp, 0, s));
            RUN(ctx, s, "clear_scratch",
                launch_fill_i32(reinterpret_cast<int32_t *>(w.hidden16), P * L->hp / 2, 0, s));
        }
        return forward_device_run(L, T, inputs, token_ids, outputs, path, s);
    };
    // the layer's own workspace is left untouched; timing is off for the
    // call (its events would be created on first use)
    Workspace own = L->ws;
    L->ws = w;
    const bool timing = ctx->timing;
    ctx->timing = false;
    rc = enqueue();
    ctx->timing = timing;
    L->ws = own;
    // the call's routing lives in the shared area, which the next call on
    // this GPU overwrites: the layer keeps no state of it
    L->last_T = -1;
    L->relaunch_ready = false;
    L->dispatch_pending = false;
    L->load_on_host = false;
    return rc;
}

int32_t gtmoe_last_routing(gtmoe_layer *L, int32_t *tokens_out, int32_t *chosen, double *gates, int32_t *load,
                           int32_t *rows_for_expert, int32_t *expert_offsets)
{
    if (!L) return GTMOE_ERR_INVALID_ARGUMENT;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    if (L->last_T < 0) return fail(ctx, GTMOE_ERR_NOT_READY, "call Forward before reading its routing");
    const int T = L->last_T;
    if (tokens_out) *tokens_out = T;
    if (T == 0) {
        if (load) memset(load, 0, sizeof(int32_t) * L->E);
        if (expert_offsets) memset(expert_offsets, 0, sizeof(int32_t) * (L->E + 1));
        return GTMOE_OK;
    }
    const size_t tk = (size_t)T * L->k;
    if (L->routing_on_host) {  // copied back by gtmoe_forward
        if (chosen) memcpy(chosen, L->host_chosen.data(), tk * 4);
        if (gates) memcpy(gates, L->host_gates.data(), tk * 8);
        if (load) memcpy(load, L->last_load.data(), sizeof(int32_t) * L->E);
        if (rows_for_expert) memcpy(rows_for_expert, L->host_rows.data(), tk * 4);
        if (expert_offsets) memcpy(expert_offsets, L->host_offsets.data(), sizeof(int32_t) * (L->E + 1));
        return GTMOE_OK;
    }
    int32_t rc = ensure_dispatch(L);
    if (rc != GTMOE_OK) return rc;
    // every table asked for comes back through pinned staging in
    // asynchronous copies behind the forward's kernels, then one wait
    Workspace &w = L->ws;
    struct Part {
        void *dst;
        const void *src;
        size_t bytes;
    } parts[] = {{chosen, w.chosen, tk * 4},
                 {gates, w.gates, tk * 8},
                 {load, w.load, sizeof(int32_t) * L->E},
                 {rows_for_expert, w.rows, tk * 4},
                 {expert_offsets, w.offsets, sizeof(int32_t) * (L->E + 1)}};
    size_t need = 0;
    for (const Part &p : parts) need += p.dst ? align_up(p.bytes, 64) : 0;
    rc = ensure_stage(L, need);
    if (rc != GTMOE_OK) return rc;
    hipStream_t s = L->last_stream;
    size_t off = 0;
    for (const Part &p : parts)
        if (p.dst) {
            HIP_TRY(ctx, hipMemcpyAsync(L->stage + off, p.src, p.bytes, hipMemcpyDeviceToHost, s));
            off += align_up(p.bytes, 64);
        }
    HIP_TRY(ctx, hipStreamSynchronize(s));
    off = 0;
    for (const Part &p : parts)
        if (p.dst) {
            memcpy(p.dst, L->stage + off, p.bytes);
            off += align_up(p.bytes, 64);
        }
    return GTMOE_OK;
}

int32_t gtmoe_last_expert_load(gtmoe_layer *L, int32_t *load)
{
    if (!L || !load) return GTMOE_ERR_INVALID_ARGUMENT;
    ENTER(L->ctx);
    int32_t rc = fetch_load(L);
    if (rc != GTMOE_OK) return rc;
    memcpy(load, L->last_load.data(), sizeof(int32_t) * L->E);
    return GTMOE_OK;
}

int32_t gtmoe_update_balance(gtmoe_layer *L, double rate)
{
    if (!L) return GTMOE_ERR_INVALID_ARGUMENT;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    // mixtureofexperts.go:293-310
    if (L->last_T < 0 || L->desc.use_hash_routing) return GTMOE_OK;
    int32_t rc = fetch_load(L);
    if (rc != GTMOE_OK) return rc;
    long long total = 0;
    for (int e = 0; e < L->E; ++e) total += L->last_load[e];
    const double average = (double)total / (double)L->E;
    for (int e = 0; e < L->E; ++e) {
        if ((double)L->last_load[e] < average) L->balance_host[e] += rate;
        if ((double)L->last_load[e] > average) L->balance_host[e] -= rate;
    }
    HIP_TRY(ctx, hipMemcpy(L->balance, L->balance_host.data(), sizeof(double) * L->E, hipMemcpyHostToDevice));
    return GTMOE_OK;
}

int32_t gtmoe_route_from_logits(gtmoe_layer *L, int32_t tokens, const double *logits, int32_t *chosen, double *gates,
                                int32_t *load, int32_t *rows_for_expert, int32_t *expert_offsets)
{
    if (!L) return GTMOE_ERR_INVALID_ARGUMENT;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    const int T = tokens;
    if (T < 0 || (T > 0 && !logits)) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "bad logits");
    int32_t rc = settle_device_work(L);
    if (rc == GTMOE_OK) rc = ensure_workspace(L, T);
    if (rc != GTMOE_OK) return rc;
    hipStream_t s = ctx->stream;
    Workspace &w = L->ws;
    if (T > 0) {
        HIP_TRY(ctx, hipMemcpyAsync(w.logits, logits, sizeof(double) * T * L->E, hipMemcpyHostToDevice, s));
        RUN(ctx, s, "topk", launch_topk(w.logits, T, L->E, L->k, L->balance, w.chosen, w.gates, w.gates32, s));
    }
    RUN(ctx, s, "dispatch",
        launch_dispatch(w.chosen, T, L->k, L->E, L->S, mfma_tile_m(), w.load, w.offsets, w.rows, w.pos, w.goff,
                        w.tok, w.tile_off, w.tile_desc, w.chunk_cnt, s));
    HIP_TRY(ctx, hipStreamSynchronize(s));
    L->skipped_dispatch = false;
    mark_forward(L, T, L->last_path, s);
    L->relaunch_ready = false;
    return gtmoe_last_routing(L, nullptr, chosen, gates, load, rows_for_expert, expert_offsets);
}

static int32_t stack_common(gtmoe_layer *const *layers, int32_t n_layers, int32_t T, gtmoe_context **ctx_out)
{
    if (!layers || n_layers < 1 || T < 0) return GTMOE_ERR_INVALID_ARGUMENT;
    gtmoe_context *ctx = layers[0] ? layers[0]->ctx : nullptr;
    if (!ctx) return GTMOE_ERR_INVALID_ARGUMENT;
    for (int l = 0; l < n_layers; ++l) {
        if (!layers[l] || layers[l]->ctx != ctx || layers[l]->d != layers[0]->d)
            return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "stack layer %d differs in context or vector size", l);
        int32_t rc = check_layer_call(layers[l]);
        if (rc != GTMOE_OK) return rc;
        if (!layers[l]->has_norm) return fail(ctx, GTMOE_ERR_NOT_READY, "stack layer %d has no norm weights", l);
        if (layers[l]->has_adapters)
            return fail(ctx, GTMOE_ERR_UNSUPPORTED, "stack layer %d has low-rank adapters; it runs through gtmoe_forward",
                        l);
    }
    *ctx_out = ctx;
    return GTMOE_OK;
}

// x <- x + MoE_l(RMSNorm_l(x)) over device fp32 x (T x d) on stream s.
static int32_t stack_run(gtmoe_layer *const *layers, int32_t n_layers, int32_t T, float *x, const int64_t *ids,
                         uint32_t flags, hipStream_t s)
{
    gtmoe_context *ctx = layers[0]->ctx;
    PendingCombine pending{};
    bool have_pending = false;
    bool prenormed = false;  // this layer's norm was done by the previous layer's combine
    // Where the residual stream is: x, or, after a routing launch whose
    // workgroups split a token's experts (and so could not combine in
    // place), the first layer's second buffer.  Every combine kernel writes x.
    float *cur = x;
    for (int l = 0; l < n_layers; ++l) {
        gtmoe_layer *L = layers[l];
        const int path = choose_path(L, T, flags);
        if (path == GTMOE_PATH_FP32 && (L->dp > kMaxGemvK || L->hp > kMaxGemvK))
            return fail(ctx, GTMOE_ERR_UNSUPPORTED, "the fp32 path takes vector and hidden sizes up to %d", kMaxGemvK);
        int32_t rc = ensure_workspace(L, T);
        if (rc != GTMOE_OK) return rc;
        if (T == 0) {
            mark_forward(L, 0, path, s);
            continue;
        }
        Workspace &w = L->ws;
        // a pending combine goes to the fused routing launch (it fits, or
        // nothing would be pending); with split routing it writes the other
        // residual buffer
        // (split routing needs T <= kMaxSplitRouteTokens, the rows xalt holds)
        float *out = nullptr;
        if (have_pending && w.part_cnt && route_fused_parts(T, L->E, L->desc.use_hash_routing != 0) > 1)
            out = cur == x ? layers[0]->ws.xalt : x;
        rc = prepare_and_route(L, T, Inputs{cur, false, true}, ids, path, s, nullptr,
                               have_pending ? &pending : nullptr, prenormed, out);
        if (out) cur = out;
        have_pending = false;
        prenormed = false;
        if (rc == GTMOE_OK) rc = run_experts(L, T, path, s);
        if (rc != GTMOE_OK) return rc;
        const int32_t *pos = L->skipped_dispatch ? nullptr : w.pos;
        gtmoe_layer *N = l + 1 < n_layers ? layers[l + 1] : nullptr;
        // on the fp32 path the next layer's routing kernel, which reads x
        // anyway, does this layer's combine (one launch fewer per layer)
        if (N && path == GTMOE_PATH_FP32 && fused_route_fits(T, N->k, N->dp)) {
            pending = PendingCombine{w.slot_out, pos, w.gates32, L->S, L->k, L->d};
            have_pending = true;
        } else if (N && path == GTMOE_PATH_BF16 && choose_path(N, T, flags) == GTMOE_PATH_BF16 &&
                   !fused_route_fits(T, N->k, N->dp) && N->d == N->dp && combine_norm_fits(L->d, true)) {
            // on the bf16 path the combine, which holds whole rows, also does
            // the next layer's RMSNorm: its bf16 rows and inverse RMS
            rc = ensure_workspace(N, T);
            if (rc != GTMOE_OK) return rc;
            CombineNorm cn;
            cn.w = N->norm_w;
            cn.xb = N->ws.xb;
            cn.ldb = N->dp;
            cn.inv = N->ws.inv;
            RUN(ctx, s, "combine_norm",
                launch_combine(T, L->d, L->S, L->k, w.slot_out, true, pos, w.gates32, cur, x, nullptr, s, cn));
            prenormed = true;
            cur = x;
        } else {
            RUN(ctx, s, "combine",
                launch_combine(T, L->d, L->S, L->k, w.slot_out, path == GTMOE_PATH_BF16, pos, w.gates32, cur, x,
                               nullptr, s));
            cur = x;
        }
        mark_forward(L, T, path, s);
    }
    return GTMOE_OK;
}

int32_t gtmoe_stack_forward(gtmoe_layer *const *layers, int32_t n_layers, int32_t tokens, double *x,
                            const int64_t *token_ids, uint32_t flags, int32_t *chosen, double *gates)
{
    gtmoe_context *ctx = nullptr;
    int32_t rc = stack_common(layers, n_layers, tokens, &ctx);
    if (rc != GTMOE_OK) return rc;
    ENTER(ctx);
    const int T = tokens;
    if (flags > GTMOE_PATH_BF16) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "unknown flags %u", flags);
    if (T > 0 && !x) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "x is null");
    if (chosen || gates)  // [n_layers][T][k] needs one k
        for (int l = 1; l < n_layers; ++l)
            if (layers[l]->k != layers[0]->k)
                return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT,
                            "stack layer %d picks %d experts per token and layer 0 picks %d; the routing outputs "
                            "are [n_layers][T][k] for one k",
                            l, layers[l]->k, layers[0]->k);
    const bool hashed = [&] {
        for (int l = 0; l < n_layers; ++l)
            if (layers[l]->desc.use_hash_routing) return true;
        return false;
    }();
    if (hashed && T > 0) {
        if (!token_ids) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "hash routing needs one token ID per row");
        for (int t = 0; t < T; ++t)
            if (token_ids[t] < 0)
                return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "token ID %lld at row %d is negative",
                            (long long)token_ids[t], t);
    }
    for (int l = 0; l < n_layers; ++l) {
        rc = settle_device_work(layers[l]);
        if (rc != GTMOE_OK) return rc;
    }
    gtmoe_layer *L0 = layers[0];
    rc = ensure_workspace(L0, T);
    if (rc != GTMOE_OK) return rc;
    hipStream_t s = ctx->stream;
    Workspace &w0 = L0->ws;
    if (T > 0) {
        HIP_TRY(ctx, hipMemcpyAsync(w0.x64, x, sizeof(double) * T * L0->d, hipMemcpyHostToDevice, s));
        if (hashed) HIP_TRY(ctx, hipMemcpyAsync(w0.ids, token_ids, sizeof(int64_t) * T, hipMemcpyHostToDevice, s));
        RUN(ctx, s, "convert_inputs", launch_convert_inputs_f64(w0.x64, T, L0->d, w0.xs, L0->d, nullptr, 0, s));
    }
    rc = stack_run(layers, n_layers, T, w0.xs, w0.ids, flags, s);
    if (rc != GTMOE_OK) return rc;
    if (T > 0) {
        RUN(ctx, s, "to_f64", launch_f32_to_f64(w0.xs, w0.y64, (long long)T * L0->d, s));
        HIP_TRY(ctx, hipMemcpyAsync(x, w0.y64, sizeof(double) * T * L0->d, hipMemcpyDeviceToHost, s));
        const size_t tk = (size_t)T * L0->k;
        for (int l = 0; l < n_layers; ++l) {
            Workspace &w = layers[l]->ws;
            if (chosen)
                HIP_TRY(ctx, hipMemcpyAsync(chosen + (size_t)l * tk, w.chosen, tk * 4, hipMemcpyDeviceToHost, s));
            if (gates)
                HIP_TRY(ctx, hipMemcpyAsync(gates + (size_t)l * tk, w.gates, tk * 8, hipMemcpyDeviceToHost, s));
        }
    }
    HIP_TRY(ctx, hipStreamSynchronize(s));
    return GTMOE_OK;
}

int32_t gtmoe_stack_forward_device(gtmoe_layer *const *layers, int32_t n_layers, int32_t tokens, float *x,
                                   const int64_t *token_ids, uint32_t flags, void *stream)
{
    gtmoe_context *ctx = nullptr;
    int32_t rc = stack_common(layers, n_layers, tokens, &ctx);
    if (rc != GTMOE_OK) return rc;
    ENTER(ctx);
    if (flags > GTMOE_PATH_BF16) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "unknown flags %u", flags);
    if (tokens > 0 && !x) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "x is null");
    for (int l = 0; l < n_layers; ++l)
        if (layers[l]->desc.use_hash_routing && tokens > 0 && !token_ids)
            return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "hash routing needs one token ID per row");
    return stack_run(layers, n_layers, tokens, x, token_ids, flags, (hipStream_t)stream);
}

int32_t gtmoe_graph_capture_forward(gtmoe_layer *L, int32_t tokens, const float *inputs, const int64_t *token_ids,
                                    float *outputs, uint32_t flags, gtmoe_graph **graph)
{
    if (!graph) return GTMOE_ERR_INVALID_ARGUMENT;
    *graph = nullptr;
    int32_t rc = check_layer_call(L);
    if (rc != GTMOE_OK) return rc;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    int path = 0;
    rc = check_forward_device(L, tokens, inputs, token_ids, outputs, flags, &path);
    if (rc == GTMOE_OK) rc = ensure_workspace(L, tokens);
    if (rc != GTMOE_OK) return rc;
    gtmoe_graph *g = new gtmoe_graph;
    g->ctx = ctx;
    g->layers = {L};
    g->paths = {path};
    g->T = tokens;
    rc = capture(ctx, [&](hipStream_t cs) { return forward_device_run(L, tokens, inputs, token_ids, outputs, path, cs); },
                 g);
    if (rc != GTMOE_OK) {
        free_graph(g);
        return rc;
    }
    g->skipped = {(char)L->skipped_dispatch};
    ++ctx->refs;  // dropped by gtmoe_graph_destroy
    *graph = g;
    return GTMOE_OK;
}

int32_t gtmoe_graph_capture_stack(gtmoe_layer *const *layers, int32_t n_layers, int32_t tokens, float *x,
                                  const int64_t *token_ids, uint32_t flags, gtmoe_graph **graph)
{
    if (!graph) return GTMOE_ERR_INVALID_ARGUMENT;
    *graph = nullptr;
    gtmoe_context *ctx = nullptr;
    int32_t rc = stack_common(layers, n_layers, tokens, &ctx);
    if (rc != GTMOE_OK) return rc;
    ENTER(ctx);
    if (flags > GTMOE_PATH_BF16) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "unknown flags %u", flags);
    if (tokens > 0 && !x) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "x is null");
    gtmoe_graph *g = new gtmoe_graph;
    g->ctx = ctx;
    g->T = tokens;
    for (int l = 0; l < n_layers; ++l) {
        gtmoe_layer *L = layers[l];
        if (L->desc.use_hash_routing && tokens > 0 && !token_ids) {
            free_graph(g);
            return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "hash routing needs one token ID per row");
        }
        rc = ensure_workspace(L, tokens);  // allocations happen before the capture
        if (rc != GTMOE_OK) {
            free_graph(g);
            return rc;
        }
        g->layers.push_back(L);
        g->paths.push_back(choose_path(L, tokens, flags));
    }
    rc = capture(ctx, [&](hipStream_t cs) { return stack_run(layers, n_layers, tokens, x, token_ids, flags, cs); }, g);
    if (rc != GTMOE_OK) {
        free_graph(g);
        return rc;
    }
    for (int l = 0; l < n_layers; ++l) g->skipped.push_back((char)layers[l]->skipped_dispatch);
    ++ctx->refs;  // dropped by gtmoe_graph_destroy
    *graph = g;
    return GTMOE_OK;
}

int32_t gtmoe_graph_launch(gtmoe_graph *g, void *stream)
{
    if (!g || !g->exec) return GTMOE_ERR_INVALID_ARGUMENT;
    gtmoe_context *ctx = g->ctx;
    ENTER(ctx);
    hipStream_t s = (hipStream_t)stream;
    HIP_TRY(ctx, hipGraphLaunch(g->exec, s));
    for (size_t i = 0; i < g->layers.size(); ++i) {
        g->layers[i]->skipped_dispatch = g->skipped[i] != 0;
        mark_forward(g->layers[i], g->T, g->paths[i], s);
    }
    return GTMOE_OK;
}

int32_t gtmoe_graph_destroy(gtmoe_graph *g)
{
    if (!g) return GTMOE_OK;
    gtmoe_context *ctx = g->ctx;
    {
        std::lock_guard<std::recursive_mutex> lock(ctx->mu);
        (void)hipSetDevice(ctx->device);
        free_graph(g);
    }
    release_context(ctx);
    return GTMOE_OK;
}

int32_t gtmoe_timing_enable(gtmoe_context *ctx, int32_t enabled)
{
    if (!ctx) return GTMOE_ERR_INVALID_ARGUMENT;
    ENTER_NODEV(ctx);
    ctx->timing = enabled != 0;
    return GTMOE_OK;
}

static int32_t collect_timing(gtmoe_context *ctx)
{
    if (ctx->pending.empty()) return GTMOE_OK;
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    HIP_TRY(ctx, hipDeviceSynchronize());
    for (auto &r : ctx->pending) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, r.start, r.stop) == hipSuccess) {
            auto &slot = ctx->totals[r.name];
            slot.first += ms;
            slot.second += 1;
        }
        ctx->spare_events.push_back(r.start);
        ctx->spare_events.push_back(r.stop);
    }
    ctx->pending.clear();
    return GTMOE_OK;
}

int32_t gtmoe_timing_reset(gtmoe_context *ctx)
{
    if (!ctx) return GTMOE_ERR_INVALID_ARGUMENT;
    ENTER_NODEV(ctx);
    int32_t rc = collect_timing(ctx);
    ctx->totals.clear();
    return rc;
}

int32_t gtmoe_timing_read(gtmoe_context *ctx, int32_t capacity, char *names, double *total_ms, int32_t *launches,
                          int32_t *count)
{
    if (!ctx || !count) return GTMOE_ERR_INVALID_ARGUMENT;
    ENTER_NODEV(ctx);
    int32_t rc = collect_timing(ctx);
    if (rc != GTMOE_OK) return rc;
    int i = 0;
    for (auto &kv : ctx->totals) {
        if (i < capacity) {
            if (names) {
                strncpy(names + 64 * i, kv.first.c_str(), 63);
                names[64 * i + 63] = 0;
            }
            if (total_ms) total_ms[i] = kv.second.first;
            if (launches) launches[i] = kv.second.second;
        }
        ++i;
    }
    *count = i;
    return GTMOE_OK;
}

int32_t gtmoe_relaunch(gtmoe_layer *L, int32_t kernel, void *stream)
{
    if (!L || (kernel != GTMOE_KERNEL_GATEUP && kernel != GTMOE_KERNEL_DOWN)) return GTMOE_ERR_INVALID_ARGUMENT;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    if (L->last_T <= 0 || !L->relaunch_ready)
        return fail(ctx, GTMOE_ERR_NOT_READY, "no forward with tokens to launch again");
    hipStream_t s = (hipStream_t)stream;
    L->device_work_pending = true;
    const bool gateup = kernel == GTMOE_KERNEL_GATEUP;
    if (L->last_path == GTMOE_PATH_FP32) {
        const GemvArgs &a = L->last_gemv[gateup ? 0 : 1];
        RUN(ctx, s, gateup ? "gemv_gateup" : "gemv_down",
            gateup ? launch_gemv_gateup(a, L->gate.precision, L->last_max_tiles, s)
                   : launch_gemv_down(a, L->down.precision, L->last_max_tiles, s));
    } else {
        const MfmaArgs &a = L->last_mfma[gateup ? 0 : 1];
        RUN(ctx, s, gateup ? "mfma_gateup" : "mfma_down",
            gateup ? launch_mfma_gateup(a, L->gate.precision, L->last_max_tiles, s)
                   : launch_mfma_down(a, L->down.precision, L->last_max_tiles, s));
    }
    return GTMOE_OK;
}

int32_t gtmoe_last_path(const gtmoe_layer *L, int32_t *path)
{
    if (!L || !path) return GTMOE_ERR_INVALID_ARGUMENT;
    *path = L->last_path;
    return GTMOE_OK;
}

int32_t gtmoe_layer_load_weights(gtmoe_layer *L, gtmoe_weights_file *f, const char *name)
{
    if (!L) return GTMOE_ERR_INVALID_ARGUMENT;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    if (!f || !name) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "weights file or layer name is null");
    {
        const int32_t rc0 = settle_device_work(L);
        if (rc0 != GTMOE_OK) return rc0;
    }

    // MixtureOfExperts.Parameters order (mixtureofexperts.go:312-324):
    // shared experts, routed experts, then the router unless hash routing
    struct Item {
        std::string base;
        int role, index;
        int rows, width;
        int w, b;  // file entries of .weights and .biases
    };
    std::vector<Item> items;
    const std::string n(name);
    const char *which[3] = {"gate", "up", "down"};
    for (int kind = 0; kind < 2; ++kind) {
        const int count = kind == 0 ? L->S : L->E;
        for (int i = 0; i < count; ++i)
            for (int j = 0; j < 3; ++j) {
                const std::string base = n + (kind == 0 ? ".shared" : ".expert") + std::to_string(i + 1) + "." +
                                         which[j];
                const int role = (kind == 0 ? GTMOE_ROLE_SHARED_GATE : GTMOE_ROLE_ROUTED_GATE) + j;
                items.push_back({base, role, i, j == 2 ? L->d : L->h, j == 2 ? L->h : L->d, -1, -1});
            }
    }
    if (!L->desc.use_hash_routing) items.push_back({n + ".router", GTMOE_ROLE_ROUTER, 0, L->E, L->d, -1, -1});

    // every parameter is checked before any is uploaded, as
    // CopyIntoKeepingCompressed does (weightfile/weightfile.go:69-108)
    for (Item &it : items) {
        const std::string wn = it.base + ".weights", bn = it.base + ".biases";
        it.w = file_find(f, wn);
        it.b = file_find(f, bn);
        if (it.w < 0) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "there is no saved parameter named \"%s\"", wn.c_str());
        if (it.b < 0) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "there is no saved parameter named \"%s\"", bn.c_str());
        const FileEntryInfo bi = file_info(f, it.b), wi = file_info(f, it.w);
        if (bi.count != (uint64_t)it.rows)
            return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT,
                        "saved parameter \"%s\" has %llu values but the parameter it's loading into has %d", bn.c_str(),
                        (unsigned long long)bi.count, it.rows);
        const uint64_t want = (uint64_t)it.rows * (uint64_t)it.width;
        if (it.role == GTMOE_ROLE_ROUTER) {
            // an uncompressed layer: plain values, or compressed rows of any
            // shape with as many values (decoded, like Rows.AllValues)
            if (wi.count != want)
                return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT,
                            "saved parameter \"%s\" has %llu values but the parameter it's loading into has %llu",
                            wn.c_str(), (unsigned long long)wi.count, (unsigned long long)want);
            // compressed rows are decoded at their stored shape: the codes and
            // scales must each fit that shape, not only sum to the right total
            if (wi.stored_as == kStoredRows) {
                const uint64_t sb = (wi.width + 15) / 16;
                const uint64_t codes_need = wi.precision == GTMOE_INT8      ? wi.rows * wi.width
                                            : wi.precision == GTMOE_FP4     ? wi.rows * ((wi.width + 1) / 2)
                                            : wi.precision == GTMOE_FLOAT32 ? wi.rows * wi.width * 4
                                                                            : wi.rows * wi.width * 8;
                const uint64_t scales_need =
                    (wi.precision == GTMOE_INT8 || wi.precision == GTMOE_FP4) ? wi.rows * sb : 0;
                if (wi.code_bytes != codes_need || wi.scale_count != scales_need)
                    return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT,
                                "saved parameter \"%s\" holds %llu value bytes and %llu scales, %llux%llu rows need "
                                "%llu and %llu",
                                wn.c_str(), (unsigned long long)wi.code_bytes, (unsigned long long)wi.scale_count,
                                (unsigned long long)wi.rows, (unsigned long long)wi.width,
                                (unsigned long long)codes_need, (unsigned long long)scales_need);
            }
            continue;
        }
        if (wi.stored_as != kStoredRows)
            return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT,
                        "parameter \"%s\" is compressed but the file holds it as plain numbers, load it into an "
                        "uncompressed parameter and compress it again",
                        wn.c_str());
        if (wi.rows != (uint64_t)it.rows || wi.width != (uint64_t)it.width)
            return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT,
                        "saved parameter \"%s\" is %llux%llu compressed values but the parameter it's loading into is "
                        "%dx%d",
                        wn.c_str(), (unsigned long long)wi.rows, (unsigned long long)wi.width, it.rows, it.width);
        if (wi.precision != L->desc.precision)
            return fail(ctx, GTMOE_ERR_UNSUPPORTED,
                        "saved parameter \"%s\" is at precision %d; the layer's experts are at precision %d on the GPU",
                        wn.c_str(), wi.precision, L->desc.precision);
        const uint64_t blocks = ((uint64_t)it.width + 15) / 16;
        const uint64_t want_codes = wi.precision == GTMOE_INT8  ? want
                                    : wi.precision == GTMOE_FP4 ? (uint64_t)it.rows * (((uint64_t)it.width + 1) / 2)
                                                                : want * 4;
        const uint64_t want_scales = wi.precision == GTMOE_FLOAT32 ? 0 : (uint64_t)it.rows * blocks;
        if (wi.code_bytes != want_codes || wi.scale_count != want_scales)
            return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT,
                        "saved parameter \"%s\" holds %llu value bytes and %llu scales, %dx%d rows need %llu and %llu",
                        wn.c_str(), (unsigned long long)wi.code_bytes, (unsigned long long)wi.scale_count, it.rows,
                        it.width, (unsigned long long)want_codes, (unsigned long long)want_scales);
    }

    std::vector<double> biases, plain;
    std::vector<uint8_t> codes;
    std::vector<float> scales;
    std::string err;
    for (const Item &it : items) {
        if (file_values(f, it.b, biases, err) != GTMOE_OK) return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "%s", err.c_str());
        const FileEntryInfo wi = file_info(f, it.w);
        gtmoe_rows r{};
        r.rows = it.rows;
        r.width = it.width;
        if (wi.stored_as == kStoredRows) {
            if (file_rows(f, it.w, codes, scales, err) != GTMOE_OK)
                return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "%s", err.c_str());
            gtmoe_rows stored{};
            stored.precision = wi.precision;
            stored.rows = (int32_t)wi.rows;
            stored.width = (int32_t)wi.width;
            stored.values = codes.data();
            stored.values_bytes = codes.size();
            stored.scales = scales.data();
            stored.scale_count = scales.size();
            if (it.role == GTMOE_ROLE_ROUTER && (wi.rows != (uint64_t)it.rows || wi.width != (uint64_t)it.width)) {
                // reshape through the decoded values
                plain.resize((size_t)wi.count);
                for (uint64_t row = 0; row < wi.rows; ++row)
                    for (uint64_t i = 0; i < wi.width; ++i)
                        plain[(size_t)(row * wi.width + i)] = decoded_value(&stored, (int)row, (int)i);
                r.precision = GTMOE_FLOAT64;
                r.values = plain.data();
                r.values_bytes = plain.size() * sizeof(double);
            } else {
                r = stored;
            }
        } else {
            if (file_values(f, it.w, plain, err) != GTMOE_OK)
                return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "%s", err.c_str());
            r.precision = GTMOE_FLOAT64;
            r.values = plain.data();
            r.values_bytes = plain.size() * sizeof(double);
        }
        const int32_t rc = gtmoe_upload_rows(L, it.role, it.index, &r, biases.data());
        if (rc != GTMOE_OK) return rc;
    }
    return GTMOE_OK;
}


int32_t gtmoe_layer_add_adapters(gtmoe_layer *L, int32_t rank, double alpha, uint64_t seed)
{
    if (!L) return GTMOE_ERR_INVALID_ARGUMENT;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    if (rank < 1)
        return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "Model.AddLowRankAdapters: rank must be at least 1, got %d", rank);
    if (L->has_adapters)
        return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT,
                    "Model.AddLowRankAdapters: the model already has adapters, merge or remove them first");
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    uint64_t state = seed;
    int32_t rc = alloc_adapter(ctx, L->ad_gate, L->G, L->d, L->dp, L->h, rank, alpha, state);
    if (rc == GTMOE_OK) rc = alloc_adapter(ctx, L->ad_up, L->G, L->d, L->dp, L->h, rank, alpha, state);
    if (rc == GTMOE_OK) rc = alloc_adapter(ctx, L->ad_down, L->G, L->h, L->hp, L->d, rank, alpha, state);
    if (rc == GTMOE_OK) rc = alloc_adapter(ctx, L->ad_router, 1, L->d, L->dp, L->E, rank, alpha, state);
    if (rc != GTMOE_OK) {
        free_adapters(L);
        return rc;
    }
    HIP_TRY(ctx, hipDeviceSynchronize());  // the memsets run on the null stream
    free_train_workspace(L->tw);
    L->has_adapters = true;
    L->adapter_T = -1;
    return GTMOE_OK;
}

int32_t gtmoe_layer_remove_adapters(gtmoe_layer *L)
{
    if (!L) return GTMOE_ERR_INVALID_ARGUMENT;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    free_adapters(L);
    return GTMOE_OK;
}

int32_t gtmoe_layer_adapter_rank(gtmoe_layer *L, int32_t role, int32_t index, int32_t *rank)
{
    if (!L || !rank) return GTMOE_ERR_INVALID_ARGUMENT;
    ENTER_NODEV(L->ctx);
    int g = 0;
    const AdapterSet *a = adapter_of(L, role, index, &g);
    if (!a) return L->has_adapters ? GTMOE_ERR_INVALID_ARGUMENT : GTMOE_ERR_NOT_READY;
    *rank = a->R;
    return GTMOE_OK;
}

int32_t gtmoe_layer_set_adapter(gtmoe_layer *L, int32_t role, int32_t index, const double *down, const double *up)
{
    if (!L) return GTMOE_ERR_INVALID_ARGUMENT;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    int g = 0;
    AdapterSet *a = adapter_of(L, role, index, &g);
    if (!a) return L->has_adapters ? GTMOE_ERR_INVALID_ARGUMENT : GTMOE_ERR_NOT_READY;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    if (down) {
        std::vector<float> A((size_t)a->R * a->kin, 0.f);
        for (int j = 0; j < a->R; ++j)
            for (int i = 0; i < a->width; ++i) A[(size_t)j * a->kin + i] = (float)down[(size_t)j * a->width + i];
        HIP_TRY(ctx, hipMemcpy(a->A + (size_t)g * a->R * a->kin, A.data(), A.size() * sizeof(float),
                               hipMemcpyHostToDevice));
    }
    if (up) {
        std::vector<float> B((size_t)a->rows * a->R);
        for (size_t i = 0; i < B.size(); ++i) B[i] = (float)up[i];
        HIP_TRY(ctx, hipMemcpy(a->B + (size_t)g * a->rows * a->R, B.data(), B.size() * sizeof(float),
                               hipMemcpyHostToDevice));
    }
    return GTMOE_OK;
}

int32_t gtmoe_layer_get_adapter(gtmoe_layer *L, int32_t role, int32_t index, double *down, double *up)
{
    if (!L) return GTMOE_ERR_INVALID_ARGUMENT;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    int g = 0;
    AdapterSet *a = adapter_of(L, role, index, &g);
    if (!a) return L->has_adapters ? GTMOE_ERR_INVALID_ARGUMENT : GTMOE_ERR_NOT_READY;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    if (down) {
        std::vector<float> A((size_t)a->R * a->kin);
        HIP_TRY(ctx, hipMemcpy(A.data(), a->A + (size_t)g * a->R * a->kin, A.size() * sizeof(float),
                               hipMemcpyDeviceToHost));
        for (int j = 0; j < a->R; ++j)
            for (int i = 0; i < a->width; ++i) down[(size_t)j * a->width + i] = A[(size_t)j * a->kin + i];
    }
    if (up) {
        std::vector<float> B((size_t)a->rows * a->R);
        HIP_TRY(ctx, hipMemcpy(B.data(), a->B + (size_t)g * a->rows * a->R, B.size() * sizeof(float),
                               hipMemcpyDeviceToHost));
        for (size_t i = 0; i < B.size(); ++i) up[i] = B[i];
    }
    return GTMOE_OK;
}

int32_t gtmoe_layer_adapter_gradients(gtmoe_layer *L, int32_t role, int32_t index, double *down_grad,
                                      double *up_grad)
{
    if (!L) return GTMOE_ERR_INVALID_ARGUMENT;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    int g = 0;
    AdapterSet *a = adapter_of(L, role, index, &g);
    if (!a) return L->has_adapters ? GTMOE_ERR_INVALID_ARGUMENT : GTMOE_ERR_NOT_READY;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    if (down_grad) {
        std::vector<double> A((size_t)a->R * a->kin);
        HIP_TRY(ctx, hipMemcpy(A.data(), a->dA + (size_t)g * a->R * a->kin, A.size() * sizeof(double),
                               hipMemcpyDeviceToHost));
        for (int j = 0; j < a->R; ++j)
            for (int i = 0; i < a->width; ++i) down_grad[(size_t)j * a->width + i] = A[(size_t)j * a->kin + i];
    }
    if (up_grad)
        HIP_TRY(ctx, hipMemcpy(up_grad, a->dB + (size_t)g * a->rows * a->R, (size_t)a->rows * a->R * sizeof(double),
                               hipMemcpyDeviceToHost));
    return GTMOE_OK;
}

int32_t gtmoe_layer_zero_adapter_gradients(gtmoe_layer *L)
{
    if (!L) return GTMOE_ERR_INVALID_ARGUMENT;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    if (!L->has_adapters) return fail(ctx, GTMOE_ERR_NOT_READY, "the layer has no low-rank adapters");
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    for (AdapterSet *a : {&L->ad_gate, &L->ad_up, &L->ad_down, &L->ad_router}) {
        HIP_TRY(ctx, hipMemset(a->dA, 0, (size_t)a->G * a->R * a->kin * sizeof(double)));
        HIP_TRY(ctx, hipMemset(a->dB, 0, (size_t)a->G * a->rows * a->R * sizeof(double)));
    }
    HIP_TRY(ctx, hipDeviceSynchronize());  // the memsets run on the null stream
    return GTMOE_OK;
}

int32_t gtmoe_backward(gtmoe_layer *L, int32_t tokens, const double *output_gradients, double *input_gradients)
{
    int32_t rc = check_layer_call(L);
    if (rc != GTMOE_OK) return rc;
    gtmoe_context *ctx = L->ctx;
    ENTER(ctx);
    if (!L->has_adapters)
        return fail(ctx, GTMOE_ERR_UNSUPPORTED,
                    "mixture of experts: weights are compressed for running the model, call DecompressWeights before "
                    "training, or add a low-rank adapter to train around them");
    if (L->adapter_T < 0) return fail(ctx, GTMOE_ERR_NOT_READY, "mixture of experts: call Forward before Backward");
    if (tokens != L->adapter_T)
        return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT,
                    "mixture of experts: output gradients are %dx%d but the last Forward produced %dx%d", tokens, L->d,
                    L->adapter_T, L->d);
    if (tokens == 0) return GTMOE_OK;
    if (!output_gradients || !input_gradients)
        return fail(ctx, GTMOE_ERR_INVALID_ARGUMENT, "output or input gradients are null");
    return adapter_backward(L, tokens, output_gradients, input_gradients);
}

}  // extern "C"
