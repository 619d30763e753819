"""The host-side C and C++ of this repository under AddressSanitizer and
UndefinedBehaviorSanitizer (CPU only; the GPU kernels are not built here):
libgtmoe's encoder and weights-file reader (gotransformers_amd/csrc/
encode.cpp, weightfile.cpp) and the oracle (oracle/gtmoe_oracle.c), built
with g++/gcc by tests/sanitize/Makefile.  The reader is fed version-1 and
version-2 weights files of every storage kind (written by
tests/weightfile_writer.py), every cut of each file and corrupted copies;
a sanitizer report aborts the program and fails the test.  The precedent is
the reference's race-detector run (README.md:229-233, go test -race)."""
import os
import shutil
import subprocess

import numpy as np
import pytest

import gotransformers_amd as gt
from tests import weightfile_writer as wfw
from tests.moe_fixtures import FLOAT32, FLOAT64, FP4, INT8

HERE = os.path.dirname(os.path.abspath(__file__))

pytestmark = pytest.mark.skipif(shutil.which("g++") is None or shutil.which("make") is None,
                                reason="needs g++ and make")


@pytest.fixture(scope="module")
def built(tmp_path_factory):
    out = tmp_path_factory.mktemp("sanitize")
    r = subprocess.run(["make", "-s", "-C", os.path.join(HERE, "sanitize"), f"OUT={out}"], capture_output=True,
                       text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    return out


def run(binary, *args, tmp):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1",
               TMPDIR=str(tmp))
    r = subprocess.run([str(binary), *map(str, args)], capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
    return r.stdout


def test_oracle_under_sanitizers(built, tmp_path):
    assert "oracle_check: clean" in run(built / "oracle_check", tmp=tmp_path)


def test_encoder_and_weights_reader_under_sanitizers(built, tmp_path):
    rng = np.random.default_rng(0)
    files = []
    # version 1: plain float64 values
    p = tmp_path / "v1.weights"
    wfw.write(str(p), [("a.weights", rng.normal(size=12)), ("a.biases", rng.normal(size=3))])
    files.append(p)
    # version 2: compressed rows at every precision, widths off the blocks,
    # and plain values at every storage precision
    rows = [(f"r{prec}.weights", gt.encode_rows(prec, rng.normal(0, 0.02, (3, 21))))
            for prec in (FLOAT64, FLOAT32, INT8, FP4)]
    for storage in (wfw.STORE_FLOAT64, wfw.STORE_FLOAT32, wfw.STORE_BFLOAT16):
        p = tmp_path / f"v2_{storage}.weights"
        wfw.write(str(p), rows + [("b.biases", rng.normal(size=5)), ("c", np.array([1e300, -0.0, 3.5]))], storage)
        files.append(p)
    out = run(built / "host_check", *files, tmp=tmp_path)
    assert f"encoder and {len(files)} weights file(s) clean" in out
