"""Pins the oracle's adapter forward and backward (oracle/lora.py) the way the
reference pins its own: gradientcheck.Compare's central differences
(mixtureofexperts_test.go:11-30 over the same six mixtures, with adapters on
every layer as perceptron_test.go:210-226 trains them), plus the invariants
a fresh adapter must keep (perceptron_test.go:228-247).  A dropped term, a
wrong sign or a transposed operand in the backward fails the finite
differences; the forward is also checked against the C oracle."""
import copy

import numpy as np
import pytest

import oracle
from oracle import lora
from tests.moe_fixtures import FLOAT32, FP4, INT8, make_moe

TOKEN_IDS = np.array([3, 7, 1, 12, 5])

# the six mixtures of TestGradients: (S, E, k, hash, clamp)
VERSIONS = {
    "routed, no shared": (0, 4, 2, False, 0.0),
    "routed with shared": (1, 4, 2, False, 0.0),
    "hashed, no shared": (0, 4, 2, True, 0.0),
    "hashed with shared": (1, 4, 2, True, 0.0),
    "routed, one per row": (1, 5, 1, False, 0.0),
    "clamped": (1, 4, 2, False, 0.5),
}


def encode(precision, values):
    return oracle.encode_rows(precision, values)


def mixture(name, precision, seed):
    S, E, k, hashed, clamp = VERSIONS[name]
    return make_moe(encode, d=4, h=6, E=E, k=k, S=S, precision=precision, seed=seed, std=0.5, router_std=0.5,
                    bias_std=0.1, clamp=clamp, use_hash=hashed)


@pytest.mark.parametrize("name", list(VERSIONS))
@pytest.mark.parametrize("precision", [INT8, FP4, FLOAT32])
def test_backward_matches_finite_differences(name, precision):
    moe = mixture(name, precision, seed=11)
    rng = np.random.default_rng(5)
    adapters = lora.make_adapters(moe, rank=2, alpha=4.0, rng=rng)
    x = rng.uniform(-1, 1, (len(TOKEN_IDS), 4))
    problems = lora.gradient_check(moe, adapters, x, TOKEN_IDS, seed=3)
    assert not problems, problems[:5]


def test_gradient_check_catches_a_planted_mistake():
    """The check is sharp enough: a backward with the adapter scale dropped
    from the Up gradient (a plausible slip) fails it."""
    moe = mixture("routed with shared", INT8, seed=11)
    rng = np.random.default_rng(5)
    adapters = lora.make_adapters(moe, rank=2, alpha=4.0, rng=rng)
    x = rng.uniform(-1, 1, (len(TOKEN_IDS), 4))
    original = lora._layer_backward

    def slipped(W, ad, xx, u, pre_grad, grads, key):
        if ad is not None:
            grads[key][1] -= (ad.alpha / ad.down.shape[0] - 1) * (pre_grad.T @ u)
        return original(W, ad, xx, u, pre_grad, grads, key)

    lora._layer_backward = slipped
    try:
        problems = lora.gradient_check(moe, adapters, x, TOKEN_IDS, seed=3)
    finally:
        lora._layer_backward = original
    assert any(".lora.up" in p for p in problems)


@pytest.mark.parametrize("name", ["routed with shared", "hashed with shared", "clamped"])
def test_fresh_adapters_leave_the_forward_alone(name):
    """Up starts at zero, so a new adapter does not change the output; the
    adapter forward then equals the C oracle's forward."""
    moe = mixture(name, INT8, seed=12)
    rng = np.random.default_rng(6)
    adapters = lora.make_adapters(moe, rank=2, alpha=4.0, rng=rng, up_scale=0.0)
    x = rng.uniform(-1, 1, (len(TOKEN_IDS), 4))
    got, st = lora.forward(moe, adapters, x, TOKEN_IDS)
    ref = oracle.moe_forward(moe, x, TOKEN_IDS if moe.use_hash_routing else None)
    assert np.array_equal(st.chosen, ref.chosen)
    assert np.max(np.abs(got - ref.outputs)) <= 1e-12 * max(1.0, np.max(np.abs(ref.outputs)))


def test_merged_adapter_keeps_the_output():
    """MergeLowRankAdapter's identity (perceptron_test.go:249-264): W + s Up
    Down in place of the adapter gives the same outputs (float64 weights)."""
    moe = mixture("routed with shared", oracle.FLOAT64, seed=13)
    rng = np.random.default_rng(7)
    adapters = lora.make_adapters(moe, rank=2, alpha=4.0, rng=rng)
    x = rng.uniform(-1, 1, (5, 4))
    with_adapters, _ = lora.forward(moe, adapters, x)
    merged = copy.deepcopy(moe)
    for (kind, i, which), ad in adapters.items():
        layer = merged.router if kind == "router" else getattr((merged.shared if kind == "shared" else merged.routed)[i],
                                                                which)
        W = oracle.decode_rows(layer.weights) + (ad.alpha / ad.down.shape[0]) * (ad.up @ ad.down)
        layer.weights = oracle.encode_rows(oracle.FLOAT64, W)
    plain, _ = lora.forward(merged, {}, x)
    assert np.max(np.abs(with_adapters - plain)) <= 1e-12
