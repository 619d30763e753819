"""Writes the small regression fixtures in tests/golden/ from the CPU oracle.

The reference holds no MoE golden vectors (its only fixed answer on this
path, the FP4 round trip of lowprecision_test.go:39-47, is asserted in
tests/test_oracle.py).  These fixtures are the oracle's outputs on seeded
inputs; test_oracle.py pins the oracle itself, and the fixtures then freeze
its answers so the oracle and the device are both checked against the same
stored vectors.  Run from the repository root:  python tests/golden/make_golden.py"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from tests.moe_fixtures import FLOAT32, FP4, INT8  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def encoders():
    rng = np.random.default_rng(1000)
    out = {}
    for name, prec in (("int8", INT8), ("fp4", FP4), ("float32", FLOAT32)):
        w = rng.normal(0, 0.02, size=(6, 45))
        w[0, :16] = 0.0
        w[1, :8] = [6.0, 0.25, 0.75, 1.25, -1.75, 2.5, -3.5, 5.0]
        r = oracle.encode_rows(prec, w)
        out[f"{name}_values_in"] = w
        out[f"{name}_codes"] = r.values
        if r.scales is not None:
            out[f"{name}_scales"] = r.scales
    np.savez(os.path.join(HERE, "encode_rows.npz"), **out)


def routing():
    rng = np.random.default_rng(1001)
    out = {}
    for E, k in ((8, 2), (16, 2), (64, 6), (128, 8)):
        logits = rng.normal(0, 1, size=(64, E))
        logits[:4] = rng.uniform(-30, 30, size=(4, E))
        logits[4:8, 1] = logits[4:8, 0]
        bal = rng.normal(0, 0.05, size=E)
        r = oracle.route_from_logits(logits, k, bal)
        d = oracle.dispatch(r.chosen, E)
        p = f"e{E}_k{k}_"
        out.update({p + "logits": logits, p + "balance": bal, p + "chosen": r.chosen, p + "gates": r.gates,
                    p + "load": d.load, p + "offsets": d.offsets, p + "rows": d.rows})
    np.savez(os.path.join(HERE, "routing.npz"), **out)


def layer():
    """A d=64, h=96, E=6, k=2, S=1 Int8 layer: its float64 weights, inputs and
    the oracle's outputs and routing."""
    rng = np.random.default_rng(1002)
    d, h, E, k, S = 64, 96, 6, 2, 1
    out = {"shape": np.array([d, h, E, k, S])}
    for kind, n in (("shared", S), ("routed", E)):
        for i in range(n):
            out[f"{kind}{i}_gate"] = rng.normal(0, 0.1, size=(h, d))
            out[f"{kind}{i}_up"] = rng.normal(0, 0.1, size=(h, d))
            out[f"{kind}{i}_down"] = rng.normal(0, 0.1, size=(d, h))
    out["router"] = rng.normal(0, 0.1, size=(E, d))
    out["x"] = rng.normal(size=(20, d))
    spec = spec_from_arrays(out, oracle.encode_rows)
    r = oracle.moe_forward(spec, out["x"])
    out.update({"outputs": r.outputs, "chosen": r.chosen, "gates": r.gates, "load": r.load})
    np.savez(os.path.join(HERE, "layer_int8.npz"), **out)


def spec_from_arrays(a, encode):
    from types import SimpleNamespace

    from tests.moe_fixtures import LINEAR, SILU
    d, h, E, k, S = (int(v) for v in a["shape"])

    def lay(w, act):
        return SimpleNamespace(weights=encode(INT8, w), biases=np.zeros(w.shape[0]), activation=act, clamp_limit=0.0)

    def exp(kind, i):
        return SimpleNamespace(gate=lay(a[f"{kind}{i}_gate"], SILU), up=lay(a[f"{kind}{i}_up"], LINEAR),
                               down=lay(a[f"{kind}{i}_down"], LINEAR))
    router = SimpleNamespace(weights=encode(FLOAT32, a["router"]), biases=np.zeros(E), activation=LINEAR,
                             clamp_limit=0.0)
    return SimpleNamespace(vector_size=d, hidden_size=h, experts_per_token=k, use_hash_routing=False,
                           shared=[exp("shared", i) for i in range(S)], routed=[exp("routed", i) for i in range(E)],
                           router=router, balance_biases=np.zeros(E), precision=INT8, clamp_limit=0.0)


if __name__ == "__main__":
    encoders()
    routing()
    layer()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
