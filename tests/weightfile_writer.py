"""Writer of GoTransformers binary weights files for the tests: a restatement
of SaveBinary / SaveBinaryWithPrecision (weightfile/binaryfile.go:23-138),
little endian throughout.

  version 1 (nothing compressed, float64 storage; binaryfile.go:75-82):
    "GOTRANSFORMERS-WEIGHTS-1" u32 n, per parameter u32 len, name,
    u64 count, float64 values
  version 2 (binaryfile.go:84-138): "GOTRANSFORMERS-WEIGHTS-2" u32 n, per
    parameter u32 len, name, u8 stored-as, then 1/2/3 = u64 count + float64 /
    float32 / bfloat16 values, or 4 = compressed rows: u8 precision, u64 rows,
    u64 width, five lists (u64 count + values): float64, float32, int8, FP4
    bytes, float32 scales.

A parameter is (name, values) for plain float64 values, or (name, rows) with
rows a namespace in RowsSnapshot storage (precision, rows, width, values,
scales), as gotransformers_amd.encode_rows returns."""
from __future__ import annotations

import math
import struct

import numpy as np

MARKER_1 = b"GOTRANSFORMERS-WEIGHTS-1"
MARKER_2 = b"GOTRANSFORMERS-WEIGHTS-2"
STORE_FLOAT64, STORE_FLOAT32, STORE_BFLOAT16 = 0, 1, 2  # StoragePrecision (weightfile/precision.go)
FLOAT64, FLOAT32, INT8, FP4 = 0, 1, 2, 3


def float64_to_bfloat16_bits(value):
    """float64ToBFloat16Bits (weightfile/precision.go:58-71): round to the
    nearest bfloat16, ties to even, with spacing fixed below the smallest
    normal exponent; NaN -> 0x7FC0; zero and infinities keep their float32
    upper half; values past the largest bfloat16 become infinities through
    the float32 conversion."""
    if math.isnan(value):
        return 0x7FC0
    if value == 0 or math.isinf(value):
        return struct.unpack("<I", struct.pack("<f", value))[0] >> 16
    _, e = math.frexp(value)
    exponent = max(e - 1, -126)
    spacing = exponent - 7
    steps = round(math.ldexp(value, -spacing))  # Python rounds half to even
    rounded = math.ldexp(steps, spacing)
    try:
        f32 = struct.pack("<f", rounded)
    except OverflowError:
        f32 = struct.pack("<f", math.copysign(math.inf, rounded))
    return struct.unpack("<I", f32)[0] >> 16


def bfloat16_bits_to_float64(bits):
    return float(np.array([bits << 16], np.uint32).view(np.float32)[0])


def _name(out, name):
    b = name.encode()
    out += struct.pack("<I", len(b)) + b


def _list(out, arr, dtype):
    with np.errstate(over="ignore"):  # float32(1e300) is +Inf, as in Go
        a = np.ascontiguousarray(np.asarray(arr).reshape(-1), dtype)
    out += struct.pack("<Q", a.size) + a.tobytes()


def _is_rows(v):
    return hasattr(v, "precision") and hasattr(v, "rows")


def encode(params, storage=STORE_FLOAT64):
    """The bytes SaveBinaryWithPrecision writes: version 1 when nothing is
    compressed and storage is float64, else version 2."""
    out = bytearray()
    if storage == STORE_FLOAT64 and not any(_is_rows(v) for _, v in params):
        out += MARKER_1 + struct.pack("<I", len(params))
        for name, values in params:
            _name(out, name)
            _list(out, values, "<f8")
        return bytes(out)
    out += MARKER_2 + struct.pack("<I", len(params))
    empty = np.zeros(0)
    for name, v in params:
        _name(out, name)
        if _is_rows(v):
            p = int(v.precision)
            out += struct.pack("<BBQQ", 4, p, int(v.rows), int(v.width))
            _list(out, v.values if p == FLOAT64 else empty, "<f8")
            _list(out, v.values if p == FLOAT32 else empty, "<f4")
            _list(out, v.values if p == INT8 else empty, "i1")
            _list(out, v.values if p == FP4 else empty, "u1")
            _list(out, v.scales if p in (INT8, FP4) else empty, "<f4")
        elif storage == STORE_FLOAT64:
            out += b"\x01"
            _list(out, v, "<f8")
        elif storage == STORE_FLOAT32:
            out += b"\x02"
            _list(out, v, "<f4")
        else:
            out += b"\x03"
            _list(out, [float64_to_bfloat16_bits(float(x)) for x in np.asarray(v).reshape(-1)], "<u2")
    return bytes(out)


def write(path, params, storage=STORE_FLOAT64):
    with open(path, "wb") as f:
        f.write(encode(params, storage))


def moe_parameters(spec, name):
    """MixtureOfExperts.Parameters of a layer spec (mixtureofexperts.go:312-324,
    names from :60-67 and perceptron.Layer.Parameters, perceptron/layer.go:209-216)."""
    params = []
    for kind, experts in (("shared", spec.shared), ("expert", spec.routed)):
        for i, e in enumerate(experts):
            for which in ("gate", "up", "down"):
                layer = getattr(e, which)
                base = f"{name}.{kind}{i + 1}.{which}"
                params.append((base + ".weights", layer.weights))
                params.append((base + ".biases", np.asarray(layer.biases, np.float64)))
    if not spec.use_hash_routing:
        params.append((f"{name}.router.weights", spec.router.weights))
        params.append((f"{name}.router.biases", np.asarray(spec.router.biases, np.float64)))
    return params
