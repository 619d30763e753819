"""Seeded synthetic MoE layers for the tests (weights N(0, std), biases 0 unless
asked), built as plain namespaces that both the oracle and the product accept."""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np

FLOAT64, FLOAT32, INT8, FP4 = 0, 1, 2, 3
LINEAR, SILU, CLAMPED_SILU, CLAMPED_LINEAR = 0, 1, 2, 3


def make_layer(encode, precision, rows, width, rng, std=0.02, bias_std=0.0, activation=LINEAR, clamp=0.0):
    w = rng.normal(0.0, std, size=(rows, width))
    b = rng.normal(0.0, bias_std, size=rows) if bias_std else np.zeros(rows)
    return SimpleNamespace(weights=encode(precision, w), biases=b, activation=activation, clamp_limit=clamp)


def make_expert(encode, precision, d, h, rng, std=0.02, bias_std=0.0, clamp=0.0):
    gate_act, up_act = (CLAMPED_SILU, CLAMPED_LINEAR) if clamp > 0 else (SILU, LINEAR)
    return SimpleNamespace(
        gate=make_layer(encode, precision, h, d, rng, std, bias_std, gate_act, clamp),
        up=make_layer(encode, precision, h, d, rng, std, bias_std, up_act, clamp),
        down=make_layer(encode, precision, d, h, rng, std, bias_std, LINEAR, 0.0),
    )


def make_moe(encode, *, d, h, E, k, S=0, precision=INT8, router_precision=FLOAT32, seed=0, std=0.02,
             router_std=0.02, bias_std=0.0, router_bias=None, clamp=0.0, use_hash=False, balance=None):
    rng = np.random.default_rng(seed)
    shared = [make_expert(encode, precision, d, h, rng, std, bias_std, clamp) for _ in range(S)]
    routed = [make_expert(encode, precision, d, h, rng, std, bias_std, clamp) for _ in range(E)]
    router = make_layer(encode, router_precision, E, d, rng, router_std, 0.0, LINEAR)
    if router_bias is not None:
        router.biases = np.asarray(router_bias, np.float64)
    bb = np.zeros(E) if balance is None else np.asarray(balance, np.float64)
    return SimpleNamespace(vector_size=d, hidden_size=h, experts_per_token=k, use_hash_routing=use_hash,
                           shared=shared, routed=routed, router=router, balance_biases=bb,
                           precision=precision, clamp_limit=clamp)


def zipf_router_bias(E, s, seed, scale=1.0):
    """Router biases whose ordering follows Zipf(s) over a seeded permutation
    of the experts: bias_e = scale * log(p_e / p_max) (<= 0)."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)
    p = 1.0 / np.arange(1, E + 1) ** s
    p /= p.sum()
    bias = np.empty(E)
    bias[perm] = scale * np.log(p / p[0])
    return bias


def make_moe_parallel(encode, *, d, h, E, k, S=0, precision=INT8, router_precision=FLOAT32, seed=0, std=0.02,
                      router_std=0.02, router_bias=None, threads=16):
    """A layer like make_moe's (weights N(0, std), biases 0), with every
    expert drawn from its own generator (SeedSequence(seed).spawn) so that
    the experts are drawn and encoded on a thread pool: for the
    configuration-sized layers (hundreds of millions of weights)."""
    from concurrent.futures import ThreadPoolExecutor
    seqs = np.random.SeedSequence(seed).spawn(S + E + 1)
    with ThreadPoolExecutor(max_workers=max(1, threads)) as pool:
        experts = list(pool.map(lambda q: make_expert(encode, precision, d, h, np.random.default_rng(q), std),
                                seqs[:S + E]))
    router = make_layer(encode, router_precision, E, d, np.random.default_rng(seqs[S + E]), router_std, 0.0, LINEAR)
    if router_bias is not None:
        router.biases = np.asarray(router_bias, np.float64)
    return SimpleNamespace(vector_size=d, hidden_size=h, experts_per_token=k, use_hash_routing=False,
                           shared=experts[:S], routed=experts[S:], router=router, balance_biases=np.zeros(E),
                           precision=precision, clamp_limit=0.0)
