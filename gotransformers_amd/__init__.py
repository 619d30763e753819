"""gotransformers_amd: MI355X (gfx950) mixture-of-experts forward for GoTransformers.

Python bindings (ctypes) of libgtmoe.so, the C ABI declared in include/gtmoe.h.
The classes mirror the reference's mixtureofexperts.MixtureOfExperts
(mixtureofexperts/mixtureofexperts.go:14-31) and its lowprecision.Rows format
(lowprecision/rows.go:8-18).  There is no CPU fallback: if libgtmoe.so is
missing or no gfx950 device is present, the calls raise.
"""
from __future__ import annotations

import ctypes as C
import os
from types import SimpleNamespace

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgtmoe.so")

FLOAT64, FLOAT32, INT8, FP4 = 0, 1, 2, 3
PATH_AUTO, PATH_FP32, PATH_BF16 = 0, 1, 2
KERNEL_GATEUP, KERNEL_DOWN = 0, 1

ROLE_ROUTER = 0
ROLES = {("shared", "gate"): 1, ("shared", "up"): 2, ("shared", "down"): 3,
         ("routed", "gate"): 4, ("routed", "up"): 5, ("routed", "down"): 6}

OK, ERR_INVALID_ARGUMENT, ERR_UNSUPPORTED, ERR_DEVICE, ERR_NOT_READY, ERR_OUT_OF_MEMORY = range(6)

EXPORTED = [
    "gtmoe_abi_version", "gtmoe_device_count", "gtmoe_open", "gtmoe_close", "gtmoe_context_free", "gtmoe_last_error",
    "gtmoe_test_inject_failure", "gtmoe_test_device_allocations",
    "gtmoe_encode_rows", "gtmoe_layer_create", "gtmoe_layer_destroy", "gtmoe_upload_rows",
    "gtmoe_set_balance_biases", "gtmoe_get_balance_biases", "gtmoe_set_norm_weights", "gtmoe_forward",
    "gtmoe_forward_device", "gtmoe_forward_device_noalloc", "gtmoe_last_routing", "gtmoe_last_expert_load", "gtmoe_update_balance",
    "gtmoe_route_from_logits", "gtmoe_stack_forward", "gtmoe_stack_forward_device", "gtmoe_timing_enable",
    "gtmoe_timing_reset", "gtmoe_timing_read", "gtmoe_last_path", "gtmoe_relaunch",
    "gtmoe_graph_capture_forward", "gtmoe_graph_capture_stack", "gtmoe_graph_launch", "gtmoe_graph_destroy",
    "gtmoe_weights_file_open", "gtmoe_weights_file_close", "gtmoe_weights_file_error", "gtmoe_weights_file_count",
    "gtmoe_weights_file_entry", "gtmoe_weights_file_find", "gtmoe_weights_file_values", "gtmoe_weights_file_rows",
    "gtmoe_layer_load_weights", "gtmoe_layer_add_adapters", "gtmoe_layer_remove_adapters", "gtmoe_layer_adapter_rank",
    "gtmoe_layer_set_adapter", "gtmoe_layer_get_adapter", "gtmoe_layer_adapter_gradients",
    "gtmoe_layer_zero_adapter_gradients", "gtmoe_backward",
]


class GtmoeError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f"gtmoe error {code}: {message}")
        self.code = code


class InvalidArgument(GtmoeError, ValueError):
    """The reference would panic on this call."""


class LayerDesc(C.Structure):
    _fields_ = [("vector_size", C.c_int32), ("expert_hidden_size", C.c_int32), ("shared_experts", C.c_int32),
                ("routed_experts", C.c_int32), ("experts_per_token", C.c_int32), ("precision", C.c_int32),
                ("use_hash_routing", C.c_int32), ("reserved", C.c_int32), ("clamp_limit", C.c_double)]


class RowsStruct(C.Structure):
    _fields_ = [("precision", C.c_int32), ("rows", C.c_int32), ("width", C.c_int32), ("reserved", C.c_int32),
                ("values", C.c_void_p), ("values_bytes", C.c_size_t), ("scales", C.c_void_p),
                ("scale_count", C.c_size_t)]


_lib = None


def library():
    """Load libgtmoe.so (built by gotransformers_amd/build.py)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() or gotransformers_amd/build.py")
    try:
        L = C.CDLL(LIB_PATH)
    except OSError as e:
        raise ImportError(f"cannot load {LIB_PATH}: {e}") from e
    P, i32, u32, dbl = C.c_void_p, C.c_int32, C.c_uint32, C.c_double
    sig = {
        "gtmoe_abi_version": ([], i32),
        "gtmoe_device_count": ([P], i32),
        "gtmoe_open": ([i32, P], i32),
        "gtmoe_close": ([P], i32),
        "gtmoe_context_free": ([P], i32),
        "gtmoe_last_error": ([P], C.c_char_p),
        "gtmoe_test_inject_failure": ([C.c_char_p, i32], i32),
        "gtmoe_test_device_allocations": ([P, P], i32),
        "gtmoe_encode_rows": ([i32, i32, i32, P, P, P], i32),
        "gtmoe_layer_create": ([P, C.POINTER(LayerDesc), P], i32),
        "gtmoe_layer_destroy": ([P], i32),
        "gtmoe_upload_rows": ([P, i32, i32, C.POINTER(RowsStruct), P], i32),
        "gtmoe_set_balance_biases": ([P, P], i32),
        "gtmoe_get_balance_biases": ([P, P], i32),
        "gtmoe_set_norm_weights": ([P, P], i32),
        "gtmoe_forward": ([P, i32, P, P, P, u32], i32),
        "gtmoe_forward_device": ([P, i32, P, P, P, u32, P], i32),
        "gtmoe_forward_device_noalloc": ([P, i32, P, P, P, u32, P], i32),
        "gtmoe_last_routing": ([P, P, P, P, P, P, P], i32),
        "gtmoe_last_expert_load": ([P, P], i32),
        "gtmoe_update_balance": ([P, dbl], i32),
        "gtmoe_route_from_logits": ([P, i32, P, P, P, P, P, P], i32),
        "gtmoe_stack_forward": ([P, i32, i32, P, P, u32, P, P], i32),
        "gtmoe_stack_forward_device": ([P, i32, i32, P, P, u32, P], i32),
        "gtmoe_timing_enable": ([P, i32], i32),
        "gtmoe_timing_reset": ([P], i32),
        "gtmoe_timing_read": ([P, i32, P, P, P, P], i32),
        "gtmoe_last_path": ([P, P], i32),
        "gtmoe_relaunch": ([P, i32, P], i32),
        "gtmoe_graph_capture_forward": ([P, i32, P, P, P, u32, P], i32),
        "gtmoe_graph_capture_stack": ([P, i32, i32, P, P, u32, P], i32),
        "gtmoe_graph_launch": ([P, P], i32),
        "gtmoe_graph_destroy": ([P], i32),
        "gtmoe_weights_file_open": ([C.c_char_p, P, P, i32], i32),
        "gtmoe_weights_file_close": ([P], i32),
        "gtmoe_weights_file_error": ([P], C.c_char_p),
        "gtmoe_weights_file_count": ([P, P], i32),
        "gtmoe_weights_file_entry": ([P, i32, P, i32, P, P, P, P, P], i32),
        "gtmoe_weights_file_find": ([P, C.c_char_p, P], i32),
        "gtmoe_weights_file_values": ([P, i32, P, C.c_int64], i32),
        "gtmoe_weights_file_rows": ([P, i32, P, C.c_int64, P, C.c_int64], i32),
        "gtmoe_layer_load_weights": ([P, P, C.c_char_p], i32),
        "gtmoe_layer_add_adapters": ([P, i32, dbl, C.c_uint64], i32),
        "gtmoe_layer_remove_adapters": ([P], i32),
        "gtmoe_layer_adapter_rank": ([P, i32, i32, P], i32),
        "gtmoe_layer_set_adapter": ([P, i32, i32, P, P], i32),
        "gtmoe_layer_get_adapter": ([P, i32, i32, P, P], i32),
        "gtmoe_layer_adapter_gradients": ([P, i32, i32, P, P], i32),
        "gtmoe_layer_zero_adapter_gradients": ([P], i32),
        "gtmoe_backward": ([P, i32, P, P], i32),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    _lib = L
    return L


def _ptr(a):
    return None if a is None else a.ctypes.data


def _check(code, ctx_handle=None):
    if code == OK:
        return
    msg = library().gtmoe_last_error(ctx_handle)
    msg = msg.decode() if msg else ""
    if code == ERR_INVALID_ARGUMENT:
        raise InvalidArgument(code, msg)
    raise GtmoeError(code, msg)


def inject_failure(entry_point, status):
    """Test hook: the next call of `entry_point` on this thread answers
    `status` instead of running (gtmoe_test_inject_failure)."""
    _check(library().gtmoe_test_inject_failure(entry_point.encode(), status))


def device_allocations():
    """(allocations, frees): the device allocations and frees the library has
    made since it was loaded (a test hook)."""
    a, f = C.c_int64(), C.c_int64()
    _check(library().gtmoe_test_device_allocations(C.byref(a), C.byref(f)))
    return a.value, f.value


def device_count():
    n = C.c_int32(0)
    _check(library().gtmoe_device_count(C.byref(n)))
    return n.value


# --------------------------------------------------------------------------
# lowprecision rows
# --------------------------------------------------------------------------

def encode_rows(precision, values):
    """lowprecision.Rows.Append over every row of a float64 matrix
    (lowprecision/rows.go:38-79), computed by libgtmoe's host encoder.
    Returns a namespace (precision, rows, width, values, scales) in the
    reference's RowsSnapshot storage."""
    values = np.ascontiguousarray(np.atleast_2d(values), dtype=np.float64)
    rows, width = values.shape
    scales = None
    if precision == FLOAT64:
        out = np.empty((rows, width), np.float64)
    elif precision == FLOAT32:
        out = np.empty((rows, width), np.float32)
    elif precision == INT8:
        out = np.empty((rows, width), np.int8)
        scales = np.empty((rows, (width + 15) // 16), np.float32)
    elif precision == FP4:
        out = np.empty((rows, (width + 1) // 2), np.uint8)
        scales = np.empty((rows, (width + 15) // 16), np.float32)
    else:
        raise ValueError(f"unknown precision {precision}")
    _check(library().gtmoe_encode_rows(precision, rows, width, values.ctypes.data, out.ctypes.data, _ptr(scales)))
    return SimpleNamespace(precision=precision, rows=rows, width=width, values=out, scales=scales)


def _rows_struct(r):
    v = r.values
    s = r.scales
    return RowsStruct(int(r.precision), int(r.rows), int(r.width), 0, v.ctypes.data, v.nbytes,
                      None if s is None else s.ctypes.data, 0 if s is None else s.size)


# --------------------------------------------------------------------------
# context
# --------------------------------------------------------------------------

class Context:
    """One GPU: gtmoe_open / gtmoe_close (replaces gpu.Open, gpu/device.go:90-130)."""

    def __init__(self, device=0):
        h = C.c_void_p()
        _check(library().gtmoe_open(device, C.byref(h)))
        self.handle = h
        self.device = device

    def close(self):
        """gtmoe_context_free: closes the context and gives up this handle
        (layers made on it answer "the context is closed" until destroyed)."""
        if self.handle:
            library().gtmoe_context_free(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def check(self, code):
        _check(code, self.handle)

    # per-kernel HIP-event timing
    def timing(self, enabled=True):
        self.check(library().gtmoe_timing_enable(self.handle, 1 if enabled else 0))

    def timing_reset(self):
        self.check(library().gtmoe_timing_reset(self.handle))

    def timing_read(self):
        cap = 64
        names = C.create_string_buffer(64 * cap)
        ms = np.zeros(cap, np.float64)
        launches = np.zeros(cap, np.int32)
        n = C.c_int32(0)
        self.check(library().gtmoe_timing_read(self.handle, cap, names, ms.ctypes.data, launches.ctypes.data,
                                                C.byref(n)))
        out = {}
        for i in range(min(n.value, cap)):
            name = names.raw[64 * i:64 * i + 64].split(b"\0", 1)[0].decode()
            out[name] = (float(ms[i]), int(launches[i]))
        return out


# --------------------------------------------------------------------------
# MixtureOfExperts
# --------------------------------------------------------------------------

class MixtureOfExperts:
    """A mixtureofexperts.MixtureOfExperts whose weights live in HBM.

    Method names follow the reference: forward (Forward), last_expert_load
    (LastExpertLoad), update_balance (UpdateBalance), balance_biases
    (BalanceBiases)."""

    def __init__(self, ctx, vector_size, expert_hidden_size, shared_experts, routed_experts, experts_per_token,
                 precision=INT8, clamp_limit=0.0, use_hash_routing=False):
        self.ctx = ctx
        self.vector_size = vector_size
        self.expert_hidden_size = expert_hidden_size
        self.shared_experts = shared_experts
        self.routed_experts = routed_experts
        self.experts_per_token = experts_per_token
        self.precision = precision
        self.use_hash_routing = use_hash_routing
        desc = LayerDesc(vector_size, expert_hidden_size, shared_experts, routed_experts, experts_per_token,
                         precision, 1 if use_hash_routing else 0, 0, float(clamp_limit))
        h = C.c_void_p()
        ctx.check(library().gtmoe_layer_create(ctx.handle, C.byref(desc), C.byref(h)))
        self.handle = h

    @classmethod
    def from_spec(cls, ctx, spec):
        """Build and upload a layer from a namespace with the reference's
        structure (shared/routed experts with gate/up/down layers, a router
        layer and balance biases)."""
        m = cls(ctx, spec.vector_size, spec.hidden_size, len(spec.shared), len(spec.routed), spec.experts_per_token,
                spec.precision, getattr(spec, "clamp_limit", 0.0), spec.use_hash_routing)
        for kind, experts in (("shared", spec.shared), ("routed", spec.routed)):
            for i, e in enumerate(experts):
                for which in ("gate", "up", "down"):
                    layer = getattr(e, which)
                    m.upload(kind, i, which, layer.weights, layer.biases)
        if not spec.use_hash_routing:
            m.upload_router(spec.router.weights, spec.router.biases)
        m.balance_biases = spec.balance_biases
        return m

    def destroy(self):
        """Free the layer's device memory.  Refused (InvalidArgument, the
        layer kept) while a recorded Graph uses the layer."""
        if self.handle:
            code = library().gtmoe_layer_destroy(self.handle)
            if code != OK:
                self.ctx.check(code)
            self.handle = None

    def upload(self, kind, index, which, rows, biases):
        b = np.ascontiguousarray(biases, np.float64)
        s = _rows_struct(rows)
        self.ctx.check(library().gtmoe_upload_rows(self.handle, ROLES[(kind, which)], index, C.byref(s), b.ctypes.data))

    def load_weights(self, weights_file, name):
        """LoadBinary of this layer's parameters, named `name`.shared<i>...,
        `name`.expert<i>... and `name`.router..., from an open WeightsFile."""
        self.ctx.check(library().gtmoe_layer_load_weights(self.handle, weights_file.handle, name.encode()))

    def upload_router(self, rows, biases):
        b = np.ascontiguousarray(biases, np.float64)
        s = _rows_struct(rows)
        self.ctx.check(library().gtmoe_upload_rows(self.handle, ROLE_ROUTER, 0, C.byref(s), b.ctypes.data))

    @property
    def balance_biases(self):
        out = np.empty(self.routed_experts, np.float64)
        self.ctx.check(library().gtmoe_get_balance_biases(self.handle, out.ctypes.data))
        return out

    @balance_biases.setter
    def balance_biases(self, values):
        v = np.ascontiguousarray(values, np.float64)
        if v.shape != (self.routed_experts,):
            raise ValueError(f"has {self.routed_experts} routed experts but {v.size} balance biases")
        self.ctx.check(library().gtmoe_set_balance_biases(self.handle, v.ctypes.data))

    def set_norm_weights(self, weights):
        w = np.ascontiguousarray(weights, np.float64)
        self.ctx.check(library().gtmoe_set_norm_weights(self.handle, w.ctypes.data))

    def forward(self, inputs, token_ids=None, path=PATH_AUTO):
        """MixtureOfExperts.Forward: float64 T x d in, float64 T x d out."""
        x = np.ascontiguousarray(np.atleast_2d(inputs), np.float64)
        if x.shape[1] != self.vector_size:
            raise InvalidArgument(ERR_INVALID_ARGUMENT,
                                  f"each row has {x.shape[1]} values but the experts take {self.vector_size}")
        ids = None
        if token_ids is not None:
            ids = np.ascontiguousarray(token_ids, np.int64)
            if ids.shape != (x.shape[0],):
                raise InvalidArgument(ERR_INVALID_ARGUMENT, f"got {ids.size} token IDs for {x.shape[0]} rows")
        out = np.empty_like(x)
        self.ctx.check(library().gtmoe_forward(self.handle, x.shape[0], x.ctypes.data, _ptr(ids), out.ctypes.data,
                                                path))
        return out

    # ----------------------------------------------------------------- adapters

    @staticmethod
    def _role(kind, which):
        """(kind, which) as in upload(), or ("router", None)."""
        return ROLE_ROUTER if kind == "router" else ROLES[(kind, which)]

    def _adapter_shape(self, kind, which):
        if kind == "router":
            return self.vector_size, self.routed_experts
        if which == "down":
            return self.expert_hidden_size, self.vector_size
        return self.vector_size, self.expert_hidden_size

    def add_adapters(self, rank, alpha, seed=0):
        """Model.AddLowRankAdapters over this mixture's layers
        (transformer/adapters.go:24-38): rank min(rank, inputs, outputs) per
        layer, Down uniform in +-1/sqrt(inputs) (seeded here), Up zero."""
        self.ctx.check(library().gtmoe_layer_add_adapters(self.handle, int(rank), float(alpha), int(seed)))

    def remove_adapters(self):
        self.ctx.check(library().gtmoe_layer_remove_adapters(self.handle))

    def adapter_rank(self, kind, index=0, which=None):
        r = C.c_int32(0)
        self.ctx.check(library().gtmoe_layer_adapter_rank(self.handle, self._role(kind, which), index, C.byref(r)))
        return r.value

    def set_adapter(self, kind, index, which, down=None, up=None):
        """Adapter.Down [rank][inputs] and Adapter.Up [outputs][rank] of one
        layer (kind "shared"/"routed" with which "gate"/"up"/"down", or
        "router")."""
        inputs, outputs = self._adapter_shape(kind, which)
        r = self.adapter_rank(kind, index, which)
        dn = None if down is None else np.ascontiguousarray(down, np.float64).reshape(r, inputs)
        u = None if up is None else np.ascontiguousarray(up, np.float64).reshape(outputs, r)
        self.ctx.check(library().gtmoe_layer_set_adapter(self.handle, self._role(kind, which), index, _ptr(dn),
                                                          _ptr(u)))

    def adapter(self, kind, index=0, which=None):
        """(Down, Up) of one layer's adapter."""
        inputs, outputs = self._adapter_shape(kind, which)
        r = self.adapter_rank(kind, index, which)
        dn, u = np.empty((r, inputs)), np.empty((outputs, r))
        self.ctx.check(library().gtmoe_layer_get_adapter(self.handle, self._role(kind, which), index, dn.ctypes.data,
                                                          u.ctypes.data))
        return dn, u

    def adapter_gradients(self, kind, index=0, which=None):
        """(DownGradients, UpGradients) of one layer's adapter."""
        inputs, outputs = self._adapter_shape(kind, which)
        r = self.adapter_rank(kind, index, which)
        dn, u = np.empty((r, inputs)), np.empty((outputs, r))
        self.ctx.check(library().gtmoe_layer_adapter_gradients(self.handle, self._role(kind, which), index,
                                                                dn.ctypes.data, u.ctypes.data))
        return dn, u

    def zero_adapter_gradients(self):
        self.ctx.check(library().gtmoe_layer_zero_adapter_gradients(self.handle))

    def backward(self, output_gradients):
        """MixtureOfExperts.Backward after forward() of the same rows: adds
        to every adapter's gradients and returns the input gradients."""
        g = np.ascontiguousarray(np.atleast_2d(output_gradients), np.float64)
        out = np.empty_like(g)
        self.ctx.check(library().gtmoe_backward(self.handle, g.shape[0], g.ctypes.data, out.ctypes.data))
        return out

    def forward_device(self, tokens, inputs_ptr, outputs_ptr, token_ids_ptr=None, path=PATH_AUTO, stream=None):
        """Forward over device-resident fp32 buffers (raw device addresses)."""
        self.ctx.check(library().gtmoe_forward_device(self.handle, tokens, inputs_ptr, token_ids_ptr, outputs_ptr,
                                                       path, stream))

    def forward_device_noalloc(self, tokens, inputs_ptr, outputs_ptr, token_ids_ptr=None, path=PATH_AUTO,
                               stream=None):
        """forward_device with its intermediates in the library's fixed
        scratch area: the call allocates nothing (gtmoe.h)."""
        self.ctx.check(library().gtmoe_forward_device_noalloc(self.handle, tokens, inputs_ptr, token_ids_ptr,
                                                               outputs_ptr, path, stream))

    def last_routing(self):
        T = C.c_int32(0)
        self.ctx.check(library().gtmoe_last_routing(self.handle, C.byref(T), None, None, None, None, None))
        T = T.value
        k, E = self.experts_per_token, self.routed_experts
        chosen = np.empty((T, k), np.int32)
        gates = np.empty((T, k), np.float64)
        load = np.empty(E, np.int32)
        rows = np.empty(T * k, np.int32)
        offsets = np.empty(E + 1, np.int32)
        self.ctx.check(library().gtmoe_last_routing(self.handle, None, chosen.ctypes.data, gates.ctypes.data,
                                                     load.ctypes.data, rows.ctypes.data, offsets.ctypes.data))
        return SimpleNamespace(chosen=chosen, gates=gates, load=load, rows=rows, offsets=offsets)

    def last_expert_load(self):
        load = np.empty(self.routed_experts, np.int32)
        self.ctx.check(library().gtmoe_last_expert_load(self.handle, load.ctypes.data))
        return load

    def update_balance(self, rate):
        self.ctx.check(library().gtmoe_update_balance(self.handle, float(rate)))

    def route_from_logits(self, logits):
        lg = np.ascontiguousarray(np.atleast_2d(logits), np.float64)
        T = lg.shape[0]
        k, E = self.experts_per_token, self.routed_experts
        chosen = np.empty((T, k), np.int32)
        gates = np.empty((T, k), np.float64)
        load = np.empty(E, np.int32)
        rows = np.empty(T * k, np.int32)
        offsets = np.empty(E + 1, np.int32)
        self.ctx.check(library().gtmoe_route_from_logits(self.handle, T, lg.ctypes.data, chosen.ctypes.data,
                                                          gates.ctypes.data, load.ctypes.data, rows.ctypes.data,
                                                          offsets.ctypes.data))
        return SimpleNamespace(chosen=chosen, gates=gates, load=load, rows=rows, offsets=offsets)

    def relaunch(self, kernel=KERNEL_GATEUP, stream=None):
        """Launch one expert kernel of the last forward again (for timing)."""
        self.ctx.check(library().gtmoe_relaunch(self.handle, kernel, stream))

    @property
    def last_path(self):
        p = C.c_int32(0)
        self.ctx.check(library().gtmoe_last_path(self.handle, C.byref(p)))
        return p.value


def _layer_array(layers):
    arr = (C.c_void_p * len(layers))(*[m.handle.value for m in layers])
    return arr


def stack_forward(layers, x, token_ids=None, path=PATH_AUTO, with_routing=False):
    """x <- x + MoE_l(RMSNorm_l(x)) over the layers (transformer/block.go:71-77)."""
    ctx = layers[0].ctx
    x = np.ascontiguousarray(np.atleast_2d(x), np.float64).copy()
    ids = None if token_ids is None else np.ascontiguousarray(token_ids, np.int64)
    T, k = x.shape[0], layers[0].experts_per_token
    chosen = np.empty((len(layers), T, k), np.int32) if with_routing else None
    gates = np.empty((len(layers), T, k), np.float64) if with_routing else None
    ctx.check(library().gtmoe_stack_forward(_layer_array(layers), len(layers), T, x.ctypes.data, _ptr(ids), path,
                                            _ptr(chosen), _ptr(gates)))
    return (x, chosen, gates) if with_routing else x


def stack_forward_device(layers, tokens, x_ptr, token_ids_ptr=None, path=PATH_AUTO, stream=None):
    ctx = layers[0].ctx
    ctx.check(library().gtmoe_stack_forward_device(_layer_array(layers), len(layers), tokens, x_ptr, token_ids_ptr,
                                                   path, stream))


class Graph:
    """One recorded forward (a layer's forward_device or a stack's
    stack_forward_device) replayed as a HIP graph.  The recorded device
    buffers must stay alive and in place; refill them between launches."""

    def __init__(self, ctx, handle, layers):
        self.ctx, self.handle, self._layers = ctx, handle, layers

    @classmethod
    def capture_forward(cls, layer, tokens, inputs_ptr, outputs_ptr, token_ids_ptr=None, path=PATH_AUTO):
        h = C.c_void_p()
        layer.ctx.check(library().gtmoe_graph_capture_forward(layer.handle, tokens, inputs_ptr, token_ids_ptr,
                                                              outputs_ptr, path, C.byref(h)))
        return cls(layer.ctx, h, [layer])

    @classmethod
    def capture_stack(cls, layers, tokens, x_ptr, token_ids_ptr=None, path=PATH_AUTO):
        h = C.c_void_p()
        ctx = layers[0].ctx
        ctx.check(library().gtmoe_graph_capture_stack(_layer_array(layers), len(layers), tokens, x_ptr,
                                                      token_ids_ptr, path, C.byref(h)))
        return cls(ctx, h, list(layers))

    def launch(self, stream=None):
        self.ctx.check(library().gtmoe_graph_launch(self.handle, stream))

    def destroy(self):
        if self.handle:
            library().gtmoe_graph_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.destroy()


# --------------------------------------------------------------------------
# binary weights files
# --------------------------------------------------------------------------

STORED_FLOAT64, STORED_FLOAT32, STORED_BFLOAT16, STORED_ROWS = 1, 2, 3, 4


class WeightsFile:
    """An opened GoTransformers binary weights file (weightfile/binaryfile.go).

    values(name) is ReadBinary's float64 list for a plain parameter;
    rows(name) is the lowprecision.Rows of a compressed one, as a namespace
    with precision, rows, width, values and scales in gtmoe_rows storage.
    Opening raises InvalidArgument with the reference's message for a file
    ReadBinaryKeepingCompressed refuses."""

    def __init__(self, path):
        h = C.c_void_p()
        err = C.create_string_buffer(1024)
        code = library().gtmoe_weights_file_open(os.fsencode(path), C.byref(h), err, len(err))
        if code != OK:
            raise InvalidArgument(code, err.value.decode(errors="replace"))
        self.handle = h
        self.path = path

    def close(self):
        if self.handle:
            library().gtmoe_weights_file_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _check(self, code):
        if code != OK:
            msg = library().gtmoe_weights_file_error(self.handle)
            raise InvalidArgument(code, msg.decode(errors="replace") if msg else "")

    def __len__(self):
        n = C.c_int32(0)
        self._check(library().gtmoe_weights_file_count(self.handle, C.byref(n)))
        return n.value

    def entry(self, index):
        name = C.create_string_buffer(4096)
        stored, prec = C.c_int32(), C.c_int32()
        rows, width, count = C.c_int64(), C.c_int64(), C.c_int64()
        self._check(library().gtmoe_weights_file_entry(self.handle, index, name, len(name), C.byref(stored),
                                                        C.byref(prec), C.byref(rows), C.byref(width),
                                                        C.byref(count)))
        return SimpleNamespace(name=name.value.decode(errors="replace"), stored_as=stored.value,
                               precision=prec.value, rows=rows.value, width=width.value, count=count.value)

    def entries(self):
        return [self.entry(i) for i in range(len(self))]

    def names(self):
        return [e.name for e in self.entries()]

    def find(self, name):
        i = C.c_int32(-1)
        self._check(library().gtmoe_weights_file_find(self.handle, name.encode(), C.byref(i)))
        return i.value

    def _index(self, name):
        i = self.find(name)
        if i < 0:
            raise KeyError(name)
        return i

    def values(self, name):
        i = self._index(name)
        out = np.empty(self.entry(i).count, np.float64)
        self._check(library().gtmoe_weights_file_values(self.handle, i, out.ctypes.data, out.size))
        return out

    def rows(self, name):
        i = self._index(name)
        e = self.entry(i)
        if e.stored_as != STORED_ROWS:
            raise InvalidArgument(ERR_INVALID_ARGUMENT, f"parameter {name!r} holds plain values, not compressed rows")
        blocks = (e.width + 15) // 16
        if e.precision == FLOAT64:
            vals, scales = np.empty(e.rows * e.width, np.float64), None
        elif e.precision == FLOAT32:
            vals, scales = np.empty(e.rows * e.width, np.float32), None
        elif e.precision == INT8:
            vals, scales = np.empty(e.rows * e.width, np.int8), np.empty(e.rows * blocks, np.float32)
        else:
            vals, scales = np.empty(e.rows * ((e.width + 1) // 2), np.uint8), np.empty(e.rows * blocks, np.float32)
        self._check(library().gtmoe_weights_file_rows(self.handle, i, vals.ctypes.data, vals.nbytes,
                                                       None if scales is None else scales.ctypes.data,
                                                       0 if scales is None else scales.size))
        return SimpleNamespace(precision=e.precision, rows=e.rows, width=e.width, values=vals, scales=scales)
