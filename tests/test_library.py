"""CPU checks of libgtmoe: it loads, exports every entry point include/gtmoe.h
declares, and its host encoder (Rows.Append) is bit-exact against the oracle.
No GPU compute is called here."""
import ctypes
import os
import re

import numpy as np
import pytest

import gotransformers_amd as gt
import oracle
from tests.moe_fixtures import FLOAT32, FLOAT64, FP4, INT8

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "gtmoe.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gtmoe_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    lib = gt.library()
    names = declared_functions()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(gt.EXPORTED) == names


def test_abi_version():
    assert gt.library().gtmoe_abi_version() == 1


@pytest.mark.parametrize("p", [FLOAT64, FLOAT32, INT8, FP4])
@pytest.mark.parametrize("width", [1, 15, 16, 17, 37, 64, 1000])
def test_product_encoder_matches_oracle(p, width):
    rng = np.random.default_rng(width)
    w = rng.normal(0, 0.02, size=(9, width))
    w[0, :min(width, 16)] = 0.0  # an all-zero block
    if width >= 8:
        w[1, :8] = [6.0, 0.25, 0.75, 1.25, -1.75, 2.5, -3.5, 5.0]  # FP4 halfway points (scale 1)
    a = gt.encode_rows(p, w)
    b = oracle.encode_rows(p, w)
    assert np.array_equal(a.values, b.values)
    if b.scales is None:
        assert a.scales is None
    else:
        assert np.array_equal(a.scales, b.scales)


def test_encoder_rejects_bad_arguments():
    lib = gt.library()
    assert lib.gtmoe_encode_rows(7, 1, 4, None, None, None) == gt.ERR_INVALID_ARGUMENT
    assert lib.gtmoe_encode_rows(INT8, 1, 0, None, None, None) == gt.ERR_INVALID_ARGUMENT


def test_null_handles_are_rejected():
    lib = gt.library()
    assert lib.gtmoe_close(None) == gt.ERR_INVALID_ARGUMENT
    assert lib.gtmoe_layer_destroy(None) == gt.ERR_INVALID_ARGUMENT
    assert lib.gtmoe_forward(None, 1, None, None, None, 0) == gt.ERR_INVALID_ARGUMENT
    assert lib.gtmoe_open(0, None) == gt.ERR_INVALID_ARGUMENT
