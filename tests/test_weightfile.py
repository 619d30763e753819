"""The weights-file reader of libgtmoe (host code, no GPU): GoTransformers
binary weights files, versions 1 and 2 (weightfile/binaryfile.go), read
through the C ABI and checked against the cases of the reference's own tests
(weightfile/precision_test.go, weightfile/weightfile_test.go).

The files are written by tests/weightfile_writer.py, a restatement of the
reference's writer.  What pins the layout beyond the two restatements
agreeing: the bfloat16 known values of TestBFloat16KnownValues (pin the
writer's rounding), the byte position of the precision byte that
TestCompressedLoadErrors corrupts (pins the parameter header), the bytes per
value of TestCompressedFileSizes (pin the list encodings), and every cut of a
file failing (pins that every field is read).  No binary weights file ships
with the reference (weightfile/testdata is absent), so the version-1 fixture
is written from the parameters TestVersionOneFixtureStillLoads names."""
import math
import os
import struct

import numpy as np
import pytest

import gotransformers_amd as gt
from tests import weightfile_writer as wfw
from tests.moe_fixtures import FLOAT32, FLOAT64, FP4, INT8


def make_parameters():
    """makeParameters (weightfile/weightfile_test.go:12-18)."""
    return [("layer1.weights", np.array([0.1, -2.5, 1e-300, math.pi, 0.0])),
            ("layer1.biases", np.array([7.0, -0.000123])),
            ("empty", np.zeros(0))]


def make_random_values(count, seed):
    """Values spread over eight decades, like makeRandomValues
    (precision_test.go:40-47)."""
    rng = np.random.default_rng(seed)
    return (rng.random(count) * 2 - 1) * 10.0 ** (rng.integers(0, 8, count) - 4)


def compressed(precision, rows, width, seed):
    return gt.encode_rows(precision, make_random_values(rows * width, seed).reshape(rows, width))


def write(tmp_path, params, storage=wfw.STORE_FLOAT64, name="weights"):
    path = str(tmp_path / name)
    wfw.write(path, params, storage)
    return path


def test_bfloat16_known_values():
    """TestBFloat16KnownValues (precision_test.go:93-124), the writer's
    float64ToBFloat16Bits."""
    cases = [
        (1.0, 0x3F80), (-2.0, 0xC000), (0.0, 0x0000), (-0.0, 0x8000),
        (1 + math.ldexp(1, -8), 0x3F80), (1 + 3 * math.ldexp(1, -8), 0x3F82),
        (1 + math.ldexp(1, -8) + math.ldexp(1, -30), 0x3F81),
        (-(1 + math.ldexp(1, -8) + math.ldexp(1, -30)), 0xBF81),
        (3.4028234663852886e38, 0x7F80), ((2 - math.ldexp(1, -7)) * math.ldexp(1, 127), 0x7F7F),
        (1e300, 0x7F80), (-math.inf, 0xFF80), (math.ldexp(1, -133), 0x0001), (math.ldexp(1, -134), 0x0000),
        (1.5 * math.ldexp(1, -134), 0x0001), (math.ldexp(1, -126), 0x0080), (1e-300, 0x0000),
    ]
    for value, bits in cases:
        assert wfw.float64_to_bfloat16_bits(value) == bits, value
    assert math.isnan(wfw.bfloat16_bits_to_float64(wfw.float64_to_bfloat16_bits(math.nan)))


def test_bfloat16_rounds_to_nearest_even():
    """TestBFloat16RoundsToNearestEven (precision_test.go:126-142) on a sample."""
    for value in make_random_values(20000, 3):
        bits = wfw.float64_to_bfloat16_bits(float(value))
        r = wfw.bfloat16_bits_to_float64(bits)
        lo, hi = wfw.bfloat16_bits_to_float64(bits - 1), wfw.bfloat16_bits_to_float64(bits + 1)
        dist = abs(value - r)
        assert abs(value - lo) >= dist and abs(value - hi) >= dist
        if abs(value - lo) == dist or abs(value - hi) == dist:
            assert bits % 2 == 0


def test_version_one_file_loads(tmp_path):
    """TestVersionOneFixtureStillLoads (precision_test.go:16-38): every value
    bit for bit, the empty parameter included."""
    path = write(tmp_path, make_parameters())
    with open(path, "rb") as f:
        assert f.read(24) == b"GOTRANSFORMERS-WEIGHTS-1"
    with gt.WeightsFile(path) as wf:
        assert wf.names() == ["layer1.weights", "layer1.biases", "empty"]
        for name, values in make_parameters():
            e = wf.entry(wf.find(name))
            assert e.stored_as == gt.STORED_FLOAT64 and e.count == values.size and e.precision == -1
            got = wf.values(name)
            assert got.tobytes() == values.tobytes(), name
        assert wf.find("missing") == -1


@pytest.mark.parametrize("storage", [wfw.STORE_FLOAT64, wfw.STORE_FLOAT32, wfw.STORE_BFLOAT16])
def test_storage_precision_round_trips(tmp_path, storage):
    """TestStoragePrecisionRoundTrips (precision_test.go:49-82): loaded values
    equal StoragePrecision.Round bit for bit; bytes per value as stored."""
    big = make_random_values(20000, 1)
    small = np.array([0.1, -2.5, 1e-300, math.pi, 0, -math.inf, 1e300])
    params = [("big", big), ("small", small)]
    path = write(tmp_path, params, storage)
    with gt.WeightsFile(path) as wf:
        stored = {wfw.STORE_FLOAT64: gt.STORED_FLOAT64, wfw.STORE_FLOAT32: gt.STORED_FLOAT32,
                  wfw.STORE_BFLOAT16: gt.STORED_BFLOAT16}[storage]
        for name, values in params:
            assert wf.entry(wf.find(name)).stored_as == stored
            got = wf.values(name)
            if storage == wfw.STORE_FLOAT64:
                want = values
            elif storage == wfw.STORE_FLOAT32:
                with np.errstate(over="ignore"):
                    want = values.astype(np.float32).astype(np.float64)
            else:
                want = np.array([wfw.bfloat16_bits_to_float64(wfw.float64_to_bfloat16_bits(float(v)))
                                 for v in values])
            assert got.view(np.uint64).tolist() == want.view(np.uint64).tolist(), name
    per_value = os.path.getsize(path) / (big.size + small.size)
    want = {wfw.STORE_FLOAT64: 8, wfw.STORE_FLOAT32: 4, wfw.STORE_BFLOAT16: 2}[storage]
    assert want <= per_value <= want + 0.05


@pytest.mark.parametrize("precision", [FLOAT64, FLOAT32, INT8, FP4])
@pytest.mark.parametrize("storage", [wfw.STORE_FLOAT64, wfw.STORE_BFLOAT16])
def test_compressed_rows_round_trip(tmp_path, precision, storage):
    """TestCompressedParametersRoundTrip (precision_test.go:150-190): the rows
    come back as they were saved, whatever the plain storage precision."""
    rows = compressed(precision, 9, 37, 11)
    biases = make_random_values(9, 12)
    path = write(tmp_path, [("layer.weights", rows), ("layer.biases", biases)], storage)
    with gt.WeightsFile(path) as wf:
        e = wf.entry(0)
        assert (e.stored_as, e.precision, e.rows, e.width, e.count) == (gt.STORED_ROWS, precision, 9, 37, 9 * 37)
        got = wf.rows("layer.weights")
        assert got.values.tobytes() == np.ascontiguousarray(rows.values).tobytes()
        if precision in (INT8, FP4):
            assert got.scales.tobytes() == np.ascontiguousarray(rows.scales, np.float32).tobytes()
        else:
            assert got.scales is None
        with pytest.raises(gt.InvalidArgument, match="compressed rows, not plain values"):
            wf.values("layer.weights")
        with pytest.raises(gt.InvalidArgument, match="plain values, not compressed rows"):
            wf.rows("layer.biases")


@pytest.mark.parametrize("precision,wanted", [(FLOAT32, 4.0), (INT8, 1 + 4 / 16), (FP4, 0.5 + 4 / 16)])
def test_compressed_file_sizes(tmp_path, precision, wanted):
    """TestCompressedFileSizes (precision_test.go:192-211): 64 x 256 rows."""
    path = write(tmp_path, [("weights", compressed(precision, 64, 256, 5))])
    per_value = os.path.getsize(path) / (64 * 256)
    assert wanted <= per_value <= wanted + 0.01
    with gt.WeightsFile(path) as wf:
        r = wf.rows("weights")
        assert r.values.nbytes == {FLOAT32: 4, INT8: 1, FP4: 0.5}[precision] * 64 * 256


def test_compressed_load_errors(tmp_path):
    """TestCompressedLoadErrors (precision_test.go:213-262): every cut of a
    file fails, an unknown precision byte fails, an unknown storage byte
    fails."""
    path = write(tmp_path, [("weights", compressed(FP4, 3, 5, 1))])
    data = open(path, "rb").read()
    cut = str(tmp_path / "cut")
    for length in range(len(data)):
        with open(cut, "wb") as f:
            f.write(data[:length])
        with pytest.raises(gt.InvalidArgument):
            gt.WeightsFile(cut)
    with gt.WeightsFile(path) as wf:
        assert wf.entry(0).precision == FP4

    pos = len(b"GOTRANSFORMERS-WEIGHTS-2") + 4 + 4 + len("weights") + 1
    assert data[pos] == FP4 and data[pos - 1] == 4
    broken = bytearray(data)
    broken[pos] = 77
    bp = str(tmp_path / "broken")
    open(bp, "wb").write(bytes(broken))
    with pytest.raises(gt.InvalidArgument, match="unknown precision"):
        gt.WeightsFile(bp)
    broken[pos - 1] = 42
    open(bp, "wb").write(bytes(broken))
    with pytest.raises(gt.InvalidArgument, match=r"stored in an unknown way \(42\)"):
        gt.WeightsFile(bp)


def test_reader_errors(tmp_path):
    """The remaining refusals of ReadBinaryKeepingCompressed
    (binaryfile.go:157-372): not a weights file, a name twice, a count past
    what the file can hold, a name longer than the file, rows that do not fit
    the file, and rows whose value and scale bytes do not match their shape."""
    text = tmp_path / "weights.txt"
    text.write_text("layer1.biases 2\n7 -0.000123\n")
    with pytest.raises(gt.InvalidArgument, match="not a binary weights file"):
        gt.WeightsFile(str(text))
    with pytest.raises(gt.InvalidArgument, match="could not open"):
        gt.WeightsFile(str(tmp_path / "nothing here"))

    twice = write(tmp_path, [("a", np.ones(2)), ("a", np.ones(3))], name="twice")
    with pytest.raises(gt.InvalidArgument, match='"a" is in the file twice'):
        gt.WeightsFile(twice)

    hdr = b"GOTRANSFORMERS-WEIGHTS-1" + struct.pack("<I", 1)
    p = tmp_path / "count"
    p.write_bytes(hdr + struct.pack("<I", 1) + b"x" + struct.pack("<Q", 1 << 40))
    with pytest.raises(gt.InvalidArgument, match="more than the file can hold"):
        gt.WeightsFile(str(p))
    p.write_bytes(hdr + struct.pack("<I", 1 << 30))
    with pytest.raises(gt.InvalidArgument, match="bigger than the file"):
        gt.WeightsFile(str(p))

    hdr2 = b"GOTRANSFORMERS-WEIGHTS-2" + struct.pack("<I", 1) + struct.pack("<I", 1) + b"w"
    p.write_bytes(hdr2 + struct.pack("<BBQQ", 4, INT8, 1 << 40, 16))
    with pytest.raises(gt.InvalidArgument, match="does not fit in the file"):
        gt.WeightsFile(str(p))
    p.write_bytes(hdr2 + struct.pack("<BBQQ", 4, INT8, 1, 0))
    with pytest.raises(gt.InvalidArgument, match="does not fit in the file"):
        gt.WeightsFile(str(p))
    # one row of 16 int8 needs 16 value bytes and one scale: give 15 and one
    body = struct.pack("<BBQQ", 4, INT8, 1, 16) + struct.pack("<Q", 0) + struct.pack("<Q", 0)
    body += struct.pack("<Q", 15) + bytes(15) + struct.pack("<Q", 0) + struct.pack("<Q", 1) + struct.pack("<f", 1.0)
    p.write_bytes(hdr2 + body)
    with pytest.raises(gt.InvalidArgument, match="wrong amount of data"):
        gt.WeightsFile(str(p))


def test_layer_load_needs_open_handles():
    lib = gt.library()
    assert lib.gtmoe_layer_load_weights(None, None, b"moe") == gt.ERR_INVALID_ARGUMENT
    assert lib.gtmoe_weights_file_close(None) == gt.OK
    assert lib.gtmoe_weights_file_count(None, None) == gt.ERR_INVALID_ARGUMENT
