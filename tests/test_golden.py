"""The committed regression fixtures in tests/golden/ (written by
tests/golden/make_golden.py from the pinned oracle): the oracle and the
product encoder reproduce them on the CPU, the device reproduces them on the
GPU (routing bit-exact, outputs within the fp32-path bar)."""
import os

import numpy as np
import pytest

import gotransformers_amd as gt
import oracle
from tests.golden.make_golden import spec_from_arrays
from tests.moe_fixtures import FLOAT32, FP4, INT8

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(HERE, name), allow_pickle=False)


@pytest.mark.parametrize("encode", [oracle.encode_rows, gt.encode_rows], ids=["oracle", "product"])
def test_encoders_reproduce_fixture(encode):
    f = load("encode_rows.npz")
    for name, prec in (("int8", INT8), ("fp4", FP4), ("float32", FLOAT32)):
        r = encode(prec, f[f"{name}_values_in"])
        assert np.array_equal(r.values, f[f"{name}_codes"])
        if r.scales is not None:
            assert np.array_equal(r.scales, f[f"{name}_scales"])


def test_oracle_reproduces_routing_fixture():
    f = load("routing.npz")
    for E, k in ((8, 2), (16, 2), (64, 6), (128, 8)):
        p = f"e{E}_k{k}_"
        r = oracle.route_from_logits(f[p + "logits"], k, f[p + "balance"])
        assert np.array_equal(r.chosen, f[p + "chosen"])
        assert np.array_equal(r.gates, f[p + "gates"])
        d = oracle.dispatch(r.chosen, E)
        assert np.array_equal(d.rows, f[p + "rows"])


def test_oracle_reproduces_layer_fixture():
    f = load("layer_int8.npz")
    spec = spec_from_arrays(f, oracle.encode_rows)
    r = oracle.moe_forward(spec, f["x"])
    assert np.array_equal(r.outputs, f["outputs"])
    assert np.array_equal(r.chosen, f["chosen"])


@pytest.mark.gpu
def test_device_reproduces_routing_fixture():
    f = load("routing.npz")
    from tests.moe_fixtures import make_moe
    with gt.Context(0) as ctx:
        for E, k in ((8, 2), (16, 2), (64, 6), (128, 8)):
            p = f"e{E}_k{k}_"
            m = gt.MixtureOfExperts.from_spec(ctx, make_moe(gt.encode_rows, d=4, h=4, E=E, k=k, seed=1))
            try:
                m.balance_biases = f[p + "balance"]
                r = m.route_from_logits(f[p + "logits"])
            finally:
                m.destroy()
            assert np.array_equal(r.chosen, f[p + "chosen"])
            assert np.array_equal(r.gates.view(np.int64), f[p + "gates"].view(np.int64))
            assert np.array_equal(r.load, f[p + "load"])
            assert np.array_equal(r.offsets, f[p + "offsets"])
            assert np.array_equal(r.rows, f[p + "rows"])


@pytest.mark.gpu
@pytest.mark.parametrize("path,tol", [(gt.PATH_FP32, 1e-4), (gt.PATH_BF16, 2e-2)])
def test_device_reproduces_layer_fixture(path, tol):
    f = load("layer_int8.npz")
    spec = spec_from_arrays(f, gt.encode_rows)
    with gt.Context(0) as ctx:
        m = gt.MixtureOfExperts.from_spec(ctx, spec)
        try:
            y = m.forward(f["x"], path=path)
            r = m.last_routing()
        finally:
            m.destroy()
    assert np.array_equal(r.chosen, f["chosen"])
    assert np.array_equal(r.load, f["load"])
    err = np.max(np.abs(y - f["outputs"])) / np.max(np.abs(f["outputs"]))
    assert err <= tol, err
