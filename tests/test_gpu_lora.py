"""Adapters and the backward on the GPU against the oracle (oracle/lora.py,
itself pinned by finite differences in test_lora_oracle.py).

A layer gets adapters on every layer (Model.AddLowRankAdapters), their Down
and Up values are set to the oracle's, and the device's forward, input
gradients and every adapter's gradients must match the oracle under the
device's routing (the device computes router logits in fp32, so flips at
near-ties are allowed as in the other parity tests).  Bars: forward
max|y - r| / max|r| <= 1e-4; gradients the same measure <= 2e-4 (fp32
accumulation over the hidden and vector widths)."""
import numpy as np
import pytest

import gotransformers_amd as gt
from oracle import lora
from tests.moe_fixtures import FLOAT32, FP4, INT8, make_moe
from tests.test_gpu_parity import check_routing, rel_err, say

pytestmark = pytest.mark.gpu

FWD_TOL = 1e-4
GRAD_TOL = 2e-4


@pytest.fixture(scope="module")
def ctx():
    c = gt.Context(0)
    yield c
    c.close()


def keys_of(spec):
    for kind, experts in (("shared", spec.shared), ("routed", spec.routed)):
        for i in range(len(experts)):
            for which in ("gate", "up", "down"):
                yield (kind, i, which)
    yield ("router", 0, None)


def with_adapters(ctx, spec, adapters, rank, alpha):
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    m.add_adapters(rank, alpha, seed=1)
    for (kind, i, which), ad in adapters.items():
        assert m.adapter_rank(kind, i, which) == ad.down.shape[0]
        m.set_adapter(kind, i, which, ad.down, ad.up)
    return m


CASES = {
    # name: (d, h, E, k, S, precision, clamp, hash, T)
    "small int8 shared": (37, 53, 5, 2, 1, INT8, 0.0, False, 29),
    "small fp4 two shared": (64, 96, 6, 3, 2, FP4, 0.0, False, 17),
    "float32 experts": (40, 24, 4, 2, 0, FLOAT32, 0.0, False, 9),
    "clamped": (48, 40, 4, 2, 1, INT8, 0.3, False, 13),
    "hash routing": (32, 48, 6, 2, 1, FP4, 0.0, True, 11),
    "C2 int8 decode": (1024, 2048, 16, 2, 0, INT8, 0.0, False, 8),
    "C3 fp4 layer": (1024, 512, 64, 6, 1, FP4, 0.0, False, 64),
    # many positions per group: the transposed product on the matrix cores
    # (32-position tiles, the down layer's rows in sixteen chunks) and dx's
    # eight positions per thread
    "many positions per expert": (1024, 128, 4, 1, 1, INT8, 0.0, False, 1024),
    # the matrix-core product over FP4 rows with a partial last panel (d = 200
    # rows of the down layer, its gradient rows 200 floats apart) and half a
    # workgroup of column blocks (h = 40: four blocks)
    "many positions fp4 ragged": (200, 40, 3, 2, 1, FP4, 0.0, False, 256),
    "many positions float32": (48, 40, 2, 1, 0, FLOAT32, 0.0, False, 160),
    # fourteen positions per group on average: eight-position tiles
    "eight-position tiles": (96, 64, 8, 2, 0, INT8, 0.0, False, 56),
}
# adapter rank per case (4 unless listed): sixteen ranks take the float4 runs
# of t = s g Up, five the scalar paths
RANKS = {"many positions per expert": 16, "small fp4 two shared": 5, "clamped": 16}


@pytest.mark.parametrize("name", list(CASES))
def test_adapter_forward_and_backward(ctx, name):
    d, h, E, k, S, prec, clamp, hashed, T = CASES[name]
    rank = RANKS.get(name, 4)
    alpha = 2.0 * rank
    say(f"adapters {name}: d={d} h={h} E={E} k={k} S={S} precision={prec} T={T}")
    spec = make_moe(gt.encode_rows, d=d, h=h, E=E, k=k, S=S, precision=prec, seed=21, std=0.05, router_std=0.05,
                    bias_std=0.02, clamp=clamp, use_hash=hashed)
    rng = np.random.default_rng(22)
    adapters = lora.make_adapters(spec, rank, alpha, rng, up_scale=0.05)
    x = rng.uniform(-1, 1, (T, d))
    ids = rng.integers(0, 10000, T) if hashed else None
    G = rng.uniform(-1, 1, (T, d))
    m = with_adapters(ctx, spec, adapters, rank, alpha)
    try:
        y = m.forward(x, ids)
        r = m.last_routing()
        dx = m.backward(G)
        grads = {key: m.adapter_gradients(*key) for key in keys_of(spec)}
        dx2 = m.backward(G)  # gradients add up over calls
        grads2 = {key: m.adapter_gradients(*key) for key in keys_of(spec)}
        m.zero_adapter_gradients()
        zeroed = m.adapter_gradients("routed", 0, "gate")
    finally:
        m.destroy()
    if not hashed:
        # the oracle's routing, with its own float64 logits including the router adapter
        ref_y, st = lora.forward(spec, adapters, x, ids)
        flips = np.nonzero(np.any(st.chosen != r.chosen, axis=1))[0]
        say(f"[{name}] routing flips: {len(flips)} of {T}")
    ref_y, st = lora.forward(spec, adapters, x, ids, chosen=r.chosen)
    e = rel_err(y, ref_y)
    say(f"[{name}] forward max rel err {e:.2e}")
    assert e <= FWD_TOL
    ref_grads = lora.zero_grads(spec, adapters)
    ref_dx = lora.backward(spec, adapters, st, G, ref_grads)
    e = rel_err(dx, ref_dx)
    say(f"[{name}] input gradient max rel err {e:.2e}")
    assert e <= GRAD_TOL
    assert np.array_equal(dx, dx2)
    worst = 0.0
    for key in keys_of(spec):
        gd, gu = grads[key]
        rd, ru = ref_grads[key]
        if not np.any(rd) and not np.any(ru):  # e.g. the router under hash routing, an unused expert
            assert not np.any(gd) and not np.any(gu), key
            continue
        worst = max(worst, rel_err(gd, rd) if np.any(rd) else 0.0, rel_err(gu, ru) if np.any(ru) else 0.0)
        assert np.allclose(grads2[key][0], 2 * gd, rtol=1e-12, atol=0)
        assert np.allclose(grads2[key][1], 2 * gu, rtol=1e-12, atol=0)
    say(f"[{name}] adapter gradient max rel err {worst:.2e}")
    assert worst <= GRAD_TOL
    assert not np.any(zeroed[0]) and not np.any(zeroed[1])


def test_fresh_adapters_keep_the_output(ctx):
    """Up starts at zero (adapter.go:37-40): the adapter path's forward equals
    the adapter-free layer's to fp32 tolerance, and Down holds values in
    +-1/sqrt(inputs) while Up is zero."""
    say("fresh adapters")
    spec = make_moe(gt.encode_rows, d=64, h=96, E=8, k=2, S=1, precision=INT8, seed=23, std=0.05, bias_std=0.02)
    x = np.random.default_rng(24).uniform(-1, 1, (12, 64))
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        plain = m.forward(x, path=gt.PATH_FP32)
        m.add_adapters(8, 16.0, seed=5)
        down, up = m.adapter("routed", 3, "down")
        assert down.shape == (8, 96) and up.shape == (64, 8)
        assert not np.any(up) and np.all(np.abs(down) <= 1 / np.sqrt(96)) and np.any(down)
        assert m.adapter_rank("router", 0) == 8
        adapted = m.forward(x)
        m.remove_adapters()
        again = m.forward(x, path=gt.PATH_FP32)
    finally:
        m.destroy()
    assert rel_err(adapted, plain) <= FWD_TOL
    assert np.array_equal(again, plain)


def test_adapter_errors_mirror_the_reference(ctx):
    say("adapter errors")
    spec = make_moe(gt.encode_rows, d=32, h=32, E=4, k=2, S=0, precision=INT8, seed=25)
    x = np.random.default_rng(26).uniform(-1, 1, (3, 32))
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        m.forward(x)
        with pytest.raises(gt.GtmoeError, match="add a low-rank adapter to train around them") as info:
            m.backward(np.zeros((3, 32)))
        assert info.value.code == gt.ERR_UNSUPPORTED
        with pytest.raises(gt.InvalidArgument, match="rank must be at least 1, got 0"):
            m.add_adapters(0, 1.0)
        m.add_adapters(2, 4.0)
        with pytest.raises(gt.InvalidArgument, match="already has adapters"):
            m.add_adapters(2, 4.0)
        with pytest.raises(gt.GtmoeError, match="call Forward before Backward") as info:
            m.backward(np.zeros((3, 32)))
        assert info.value.code == gt.ERR_NOT_READY
        m.forward(x)
        with pytest.raises(gt.InvalidArgument, match="output gradients are 2x32 but the last Forward produced 3x32"):
            m.backward(np.zeros((2, 32)))
        with pytest.raises(gt.InvalidArgument, match="routed expert 4 of 4"):
            m.adapter("routed", 4, "gate")
        import torch
        xd = torch.zeros((3, 32), device="cuda")
        with pytest.raises(gt.GtmoeError, match="runs through gtmoe_forward") as info:
            m.forward_device(3, xd.data_ptr(), xd.data_ptr())
        assert info.value.code == gt.ERR_UNSUPPORTED
    finally:
        m.destroy()
