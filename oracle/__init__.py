"""ctypes front end of the CPU oracle (oracle/gtmoe_oracle.c).

TEST INFRASTRUCTURE ONLY: the parity oracle and the timed CPU baseline.  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module; the product never does.

Weights are passed as duck-typed objects so the same arrays can be handed to
the product library and to the oracle:

* rows object: ``precision`` (0 Float64, 1 Float32, 2 Int8, 3 FP4 as in
  lowprecision/lowprecision.go:9-16), ``rows``, ``width``, ``values`` (numpy
  array in the reference's Rows storage) and ``scales`` (float32 or None);
* layer object: ``weights`` (rows object), ``biases`` (float64), ``activation``
  (0 linear, 1 SiLU, 2 clamped SiLU, 3 clamped linear) and ``clamp_limit``;
* expert object: ``gate``, ``up``, ``down`` layer objects;
* MoE object: ``vector_size``, ``hidden_size``, ``experts_per_token``,
  ``use_hash_routing``, ``shared`` and ``routed`` (lists of experts),
  ``router`` (layer object) and ``balance_biases`` (float64, one per expert).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from types import SimpleNamespace

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

FLOAT64, FLOAT32, INT8, FP4 = 0, 1, 2, 3
LINEAR, SILU, CLAMPED_SILU, CLAMPED_LINEAR = 0, 1, 2, 3


def build():
    """Compile liboracle.so with the recipe in oracle/Makefile."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


class _Rows(C.Structure):
    _fields_ = [("precision", C.c_int32), ("rows", C.c_int32), ("width", C.c_int32),
                ("pad_", C.c_int32), ("values", C.c_void_p), ("scales", C.c_void_p)]


class _Layer(C.Structure):
    _fields_ = [("weights", _Rows), ("biases", C.c_void_p), ("activation", C.c_int32),
                ("pad_", C.c_int32), ("clamp_limit", C.c_double)]


class _Expert(C.Structure):
    _fields_ = [("gate", _Layer), ("up", _Layer), ("down", _Layer)]


class _MoE(C.Structure):
    _fields_ = [("vector_size", C.c_int32), ("hidden_size", C.c_int32),
                ("shared_experts", C.c_int32), ("routed_experts", C.c_int32),
                ("experts_per_token", C.c_int32), ("use_hash_routing", C.c_int32),
                ("shared", C.c_void_p), ("routed", C.c_void_p), ("router", _Layer),
                ("balance_biases", C.c_void_p)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        i32, i64, dbl = C.c_int32, C.c_long, C.c_double
        L.gtmoe_oracle_encode_rows.argtypes = [C.c_int, C.c_int, C.c_int, P, P, P, P, P]
        L.gtmoe_oracle_decode_row.argtypes = [C.POINTER(_Rows), C.c_int, P]
        L.gtmoe_oracle_dot_row.argtypes = [C.POINTER(_Rows), C.c_int, P]
        L.gtmoe_oracle_dot_row.restype = dbl
        L.gtmoe_oracle_layer_forward.argtypes = [C.POINTER(_Layer), C.c_int, P, C.c_int, P]
        L.gtmoe_oracle_route_from_logits.argtypes = [C.c_int, C.c_int, C.c_int, P, P, P, P, P]
        L.gtmoe_oracle_go_stable_order.argtypes = [C.c_int, P, P]
        L.gtmoe_oracle_hash_route.argtypes = [C.c_int, C.c_int, C.c_int, P, P, P]
        L.gtmoe_oracle_hash_route.restype = C.c_int
        L.gtmoe_oracle_dispatch.argtypes = [C.c_int, C.c_int, C.c_int, P, P, P, P]
        L.gtmoe_oracle_moe_forward.argtypes = [C.POINTER(_MoE), C.c_int, P, P, C.c_int, P, P, P, P, P, P]
        L.gtmoe_oracle_moe_forward.restype = C.c_int
        L.gtmoe_oracle_moe_forward_routed.argtypes = [C.POINTER(_MoE), C.c_int, P, P, P, C.c_int, P, P]
        L.gtmoe_oracle_rmsnorm.argtypes = [C.c_int, C.c_int, P, P, dbl, P]
        L.gtmoe_oracle_stack_forward.argtypes = [P, P, C.c_int, C.c_int, P, P, C.c_int, P]
        L.gtmoe_oracle_stack_forward.restype = C.c_int
        L.gtmoe_oracle_stack_forward_routed.argtypes = [P, P, C.c_int, C.c_int, P, P, P, C.c_int]
        L.gtmoe_oracle_map.argtypes = [C.c_int, i64, P, P]
        _ = (i32,)
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# --------------------------------------------------------------------------
# lowprecision
# --------------------------------------------------------------------------

def blocks_of(width):
    return (width + 15) // 16


def encode_rows(precision, values):
    """Rows.Append over every row of a float64 matrix (rows.go:38-79)."""
    values = _c(np.atleast_2d(values), np.float64)
    rows, width = values.shape
    scales = None
    if precision == FLOAT64:
        out = values.copy()
    elif precision == FLOAT32:
        out = np.empty((rows, width), np.float32)
    elif precision == INT8:
        out = np.empty((rows, width), np.int8)
        scales = np.empty((rows, blocks_of(width)), np.float32)
    elif precision == FP4:
        out = np.empty((rows, (width + 1) // 2), np.uint8)
        scales = np.empty((rows, blocks_of(width)), np.float32)
    else:
        raise ValueError(f"unknown precision {precision}")
    if precision != FLOAT64:
        f32 = out if precision == FLOAT32 else None
        i8 = out if precision == INT8 else None
        f4 = out if precision == FP4 else None
        lib().gtmoe_oracle_encode_rows(precision, rows, width, values.ctypes.data, _ptr(f32), _ptr(i8),
                                       _ptr(f4), _ptr(scales))
    return SimpleNamespace(precision=precision, rows=rows, width=width, values=out, scales=scales)


def _rows_struct(r):
    return _Rows(r.precision, r.rows, r.width, 0, r.values.ctypes.data,
                 None if r.scales is None else r.scales.ctypes.data)


def decode_rows(r):
    """Rows.Row for every row (rows.go:87-119)."""
    s = _rows_struct(r)
    out = np.empty((r.rows, r.width), np.float64)
    for i in range(r.rows):
        lib().gtmoe_oracle_decode_row(C.byref(s), i, out[i].ctypes.data)
    return out


def dot_row(r, row, vector):
    v = _c(vector, np.float64)
    return lib().gtmoe_oracle_dot_row(C.byref(_rows_struct(r)), row, v.ctypes.data)


def map_fn(name, x):
    """Evaluate exp / log1p / softplus / affinity / silu element-wise."""
    fn = {"exp": 0, "log1p": 1, "softplus": 2, "affinity": 3, "silu": 4}[name]
    x = _c(x, np.float64)
    out = np.empty_like(x)
    lib().gtmoe_oracle_map(fn, x.size, x.ctypes.data, out.ctypes.data)
    return out


# --------------------------------------------------------------------------
# layers and MoE
# --------------------------------------------------------------------------

def _layer_struct(layer, keep):
    b = _c(layer.biases, np.float64)
    keep.append(b)
    keep.append(layer.weights.values)
    if layer.weights.scales is not None:
        keep.append(layer.weights.scales)
    return _Layer(_rows_struct(layer.weights), b.ctypes.data, int(layer.activation), 0,
                  float(layer.clamp_limit))


def layer_forward(layer, inputs, threads=1):
    inputs = _c(np.atleast_2d(inputs), np.float64)
    keep = []
    s = _layer_struct(layer, keep)
    out = np.empty((inputs.shape[0], layer.weights.rows), np.float64)
    lib().gtmoe_oracle_layer_forward(C.byref(s), inputs.shape[0], inputs.ctypes.data, threads, out.ctypes.data)
    return out


def _moe_struct(moe, keep):
    def experts(lst):
        arr = (_Expert * max(1, len(lst)))()
        for i, e in enumerate(lst):
            arr[i] = _Expert(_layer_struct(e.gate, keep), _layer_struct(e.up, keep), _layer_struct(e.down, keep))
        keep.append(arr)
        return arr
    shared = experts(moe.shared)
    routed = experts(moe.routed)
    bb = _c(moe.balance_biases, np.float64)
    keep.append(bb)
    router = _layer_struct(moe.router, keep) if moe.router is not None else _Layer()
    return _MoE(moe.vector_size, moe.hidden_size, len(moe.shared), len(moe.routed), moe.experts_per_token,
                int(bool(moe.use_hash_routing)), C.addressof(shared), C.addressof(routed), router, bb.ctypes.data)


def moe_forward(moe, inputs, token_ids=None, threads=1):
    """MixtureOfExperts.Forward (mixtureofexperts.go:122-216).

    Returns a namespace with outputs (T x d), chosen and gates (T x k),
    load (E) and, for learned routing, logits and affinities (T x E)."""
    inputs = _c(np.atleast_2d(inputs), np.float64)
    T = inputs.shape[0]
    E, k = len(moe.routed), moe.experts_per_token
    keep = []
    s = _moe_struct(moe, keep)
    ids = None if token_ids is None else _c(token_ids, np.int64)
    out = np.empty((T, moe.vector_size), np.float64)
    chosen = np.empty((T, k), np.int32)
    gates = np.empty((T, k), np.float64)
    load = np.empty(E, np.int32)
    logits = np.empty((T, E), np.float64)
    aff = np.empty((T, E), np.float64)
    rc = lib().gtmoe_oracle_moe_forward(C.byref(s), T, inputs.ctypes.data, _ptr(ids), threads, out.ctypes.data,
                                        chosen.ctypes.data, gates.ctypes.data, load.ctypes.data,
                                        logits.ctypes.data, aff.ctypes.data)
    if rc != 0:
        raise ValueError("mixture of experts: token ID is negative")
    if moe.use_hash_routing:
        logits = aff = None
    return SimpleNamespace(outputs=out, chosen=chosen, gates=gates, load=load, logits=logits, affinities=aff)


def moe_forward_routed(moe, inputs, chosen, gates, threads=1):
    """Experts and combine of MixtureOfExperts.Forward under a given routing."""
    inputs = _c(np.atleast_2d(inputs), np.float64)
    T = inputs.shape[0]
    keep = []
    s = _moe_struct(moe, keep)
    chosen = _c(chosen, np.int32)
    gates = _c(gates, np.float64)
    out = np.empty((T, moe.vector_size), np.float64)
    load = np.empty(len(moe.routed), np.int32)
    lib().gtmoe_oracle_moe_forward_routed(C.byref(s), T, inputs.ctypes.data, chosen.ctypes.data,
                                          gates.ctypes.data, threads, out.ctypes.data, load.ctypes.data)
    return SimpleNamespace(outputs=out, load=load)


def route_from_logits(logits, k, balance_biases=None):
    logits = _c(np.atleast_2d(logits), np.float64)
    T, E = logits.shape
    bb = np.zeros(E) if balance_biases is None else _c(balance_biases, np.float64)
    chosen = np.empty((T, k), np.int32)
    gates = np.empty((T, k), np.float64)
    aff = np.empty((T, E), np.float64)
    lib().gtmoe_oracle_route_from_logits(T, E, k, logits.ctypes.data, bb.ctypes.data, chosen.ctypes.data,
                                         gates.ctypes.data, aff.ctypes.data)
    return SimpleNamespace(chosen=chosen, gates=gates, affinities=aff)


def go_stable_order(scores):
    """The candidate order sort.SliceStable(candidates, score descending)
    leaves (mixtureofexperts.go:106), Go's block insertion sort and SymMerge
    step for step; any order of NaN scores included."""
    s = _c(scores, np.float64)
    order = np.empty(len(s), np.int32)
    lib().gtmoe_oracle_go_stable_order(len(s), s.ctypes.data, order.ctypes.data)
    return order


def hash_route(token_ids, experts, k):
    ids = _c(token_ids, np.int64)
    chosen = np.empty((len(ids), k), np.int32)
    gates = np.empty((len(ids), k), np.float64)
    if lib().gtmoe_oracle_hash_route(len(ids), experts, k, ids.ctypes.data, chosen.ctypes.data,
                                     gates.ctypes.data) != 0:
        raise ValueError("hash routing: token ID is negative")
    return SimpleNamespace(chosen=chosen, gates=gates)


def dispatch(chosen, experts):
    chosen = _c(np.atleast_2d(chosen), np.int32)
    T, k = chosen.shape
    load = np.empty(experts, np.int32)
    offsets = np.empty(experts + 1, np.int32)
    rows = np.empty(T * k, np.int32)
    lib().gtmoe_oracle_dispatch(T, experts, k, chosen.ctypes.data, load.ctypes.data, offsets.ctypes.data,
                                rows.ctypes.data)
    return SimpleNamespace(load=load, offsets=offsets, rows=rows)


def rmsnorm(inputs, weights, epsilon=1e-6):
    inputs = _c(np.atleast_2d(inputs), np.float64)
    w = _c(weights, np.float64)
    out = np.empty_like(inputs)
    lib().gtmoe_oracle_rmsnorm(inputs.shape[0], inputs.shape[1], inputs.ctypes.data, w.ctypes.data,
                               float(epsilon), out.ctypes.data)
    return out


def _stack_structs(layers, norm_weights, keep):
    arr = (_MoE * len(layers))()
    for i, m in enumerate(layers):
        arr[i] = _moe_struct(m, keep)
    norms = [_c(w, np.float64) for w in norm_weights]
    keep.extend(norms)
    nptr = (C.c_void_p * len(norms))(*[n.ctypes.data for n in norms])
    keep.extend([arr, nptr])
    return arr, nptr


def stack_forward(layers, norm_weights, x, token_ids=None, threads=1):
    """Blocks without attention, x <- x + MoE(RMSNorm(x)) (transformer/block.go:71-77)."""
    x = _c(np.atleast_2d(x), np.float64).copy()
    keep = []
    arr, nptr = _stack_structs(layers, norm_weights, keep)
    ids = None if token_ids is None else _c(token_ids, np.int64)
    k = layers[0].experts_per_token
    chosen = np.empty((len(layers), x.shape[0], k), np.int32)
    rc = lib().gtmoe_oracle_stack_forward(C.addressof(arr), C.addressof(nptr), len(layers), x.shape[0],
                                          x.ctypes.data, _ptr(ids), threads, chosen.ctypes.data)
    if rc != 0:
        raise ValueError("mixture of experts: token ID is negative")
    return x, chosen


def stack_forward_routed(layers, norm_weights, x, chosen, gates, threads=1):
    x = _c(np.atleast_2d(x), np.float64).copy()
    keep = []
    arr, nptr = _stack_structs(layers, norm_weights, keep)
    chosen = _c(chosen, np.int32)
    gates = _c(gates, np.float64)
    lib().gtmoe_oracle_stack_forward_routed(C.addressof(arr), C.addressof(nptr), len(layers), x.shape[0],
                                            x.ctypes.data, chosen.ctypes.data, gates.ctypes.data, threads)
    return x
