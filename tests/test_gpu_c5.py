"""The 24-block stack at its workload size: per block d=2048, 64 routed
experts plus 1 shared expert, top-4, hidden 1024, FP4 experts, RMSNorm
(weights 1, epsilon 1e-6) and the residual x <- x + MoE(RMSNorm(x))
(transformer/block.go:71-78, normalization/rmsnorm.go:33-53).

The device runs every token through all 24 blocks; the oracle runs a seeded
sample of 16 tokens through all 24 blocks under the device's routing of
each block (a token's result depends only on its own row and routing).
Every block's dispatch (load, rowsForExpert, offsets) is checked bit for bit
against the oracle's dispatch of the device's choices, and every block's
routing of the sampled tokens against the oracle's routing (float64 router)
of the device's own input to that block: flips are allowed only at
near-ties and are reported.  Bars: 1e-4 on the fp32 path (decode chunk, T=64), 2e-2 on the
bf16 MFMA path (prefill chunk, T=8192), max |y - r| / max |r| over the
sampled rows after block 24; the error after blocks 1, 6, 12 and 18 is
reported too."""
import numpy as np
import pytest

import gotransformers_amd as gt
import oracle
from tests.moe_fixtures import FP4, make_moe_parallel
from tests.test_gpu_parity import rel_err, say

pytestmark = pytest.mark.gpu

BLOCKS = 24
SETS = 4  # distinct seeded weight sets, cycled over the blocks (each block its own resident copy)
D = 2048


@pytest.fixture(scope="module")
def stack():
    say("C5 stack: drawing and encoding 4 weight sets")
    specs = [make_moe_parallel(gt.encode_rows, d=D, h=1024, E=64, k=4, S=1, precision=FP4, seed=500 + 101 * i)
             for i in range(SETS)]
    ctx = gt.Context(0)
    layers = []
    try:
        for b in range(BLOCKS):
            m = gt.MixtureOfExperts.from_spec(ctx, specs[b % SETS])
            m.set_norm_weights(np.ones(D))
            layers.append(m)
        say(f"C5 stack: {BLOCKS} blocks resident")
        yield specs, layers
    finally:
        for m in layers:
            m.destroy()
        ctx.close()


def oracle_blocks(specs, x, chosen, gates):
    """The oracle's stack over x (sampled rows) block by block, each MoE
    under the given routing; returns the rows after every block."""
    norm = np.ones(D)
    after = []
    for b in range(BLOCKS):
        spec = specs[b % SETS]
        y = oracle.rmsnorm(x, norm)
        x = x + oracle.moe_forward_routed(spec, y, chosen[b], gates[b], threads=16).outputs
        after.append(x)
    return after


@pytest.mark.timeout(600)
@pytest.mark.parametrize("T,path,tol", [(64, gt.PATH_AUTO, 1e-4), (8192, gt.PATH_AUTO, 2e-2)])
def test_c5_stack_at_workload_size(stack, T, path, tol):
    specs, layers = stack
    say(f"C5 stack, {BLOCKS} blocks, T={T}")
    x0 = np.random.default_rng(5).normal(size=(T, D))
    x, chosen, gates = gt.stack_forward(layers, x0, path=path, with_routing=True)
    expect = gt.PATH_FP32 if T == 64 else gt.PATH_BF16
    assert all(m.last_path == expect for m in layers)
    # every block's dispatch bit for bit
    for b, m in enumerate(layers):
        r = m.last_routing()
        assert np.array_equal(r.chosen, chosen[b])
        d = oracle.dispatch(r.chosen, 64)
        assert np.array_equal(r.load, d.load), b
        assert np.array_equal(r.offsets, d.offsets), b
        assert np.array_equal(r.rows, d.rows), b
    sample = np.sort(np.random.default_rng(55).choice(T, 16, replace=False))
    ref = oracle_blocks(specs, x0[sample], chosen[:, sample], gates[:, sample])
    # Each block's routing against the oracle's routing (float64 logits) of
    # the device's own input to that block, taken from the device stack over
    # the blocks before it (all rows, so every block routes as in the full
    # run): flips only at near-ties.  The error against the oracle after
    # each block is reported.
    flips = 0
    x_in = x0[sample]
    for b in range(BLOCKS):
        spec = specs[b % SETS]
        if b > 0:
            x_in = gt.stack_forward(layers[:b], x0, path=path)[sample]
            if b in (1, 6, 12, 18):
                say(f"[C5 T={T}] after {b:2d} blocks: max rel err {rel_err(x_in, ref[b - 1]):.3e}")
        logits = oracle.layer_forward(spec.router, oracle.rmsnorm(x_in, np.ones(D)), threads=16)
        mine = oracle.route_from_logits(logits, spec.experts_per_token, spec.balance_biases)
        dev = chosen[b][sample]
        for t in np.nonzero(np.any(dev != mine.chosen, axis=1))[0]:
            srt = np.sort(mine.affinities[t] + spec.balance_biases)[::-1]
            assert srt[3] - srt[4] <= 1e-5 * max(1.0, abs(srt[3])), (b, t, srt[3] - srt[4])
            flips += 1
    say(f"[C5 T={T}] routing flips at near-ties over {BLOCKS} blocks x {len(sample)} sampled tokens: {flips}")
    e = rel_err(x[sample], ref[-1])
    say(f"[C5 T={T}] path {expect}, after {BLOCKS} blocks: max rel err on {len(sample)} sampled tokens {e:.3e}")
    assert e <= tol
