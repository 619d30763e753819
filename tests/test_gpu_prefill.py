"""GPU parity of the bf16 MFMA path (prefill) against the CPU oracle.

Bars: routing equal to the oracle's except at near-ties (reported); the
dispatch permutation and load bit-exact for the device's routing; outputs
under the device's routing within max |y - r| / max |r| <= 2e-2.  At the
full configuration sizes the oracle evaluates a seeded sample of tokens:
a token's output depends only on its own row and routing."""
import sys

import numpy as np
import pytest

import gotransformers_amd as gt
import oracle
from tests.moe_fixtures import FLOAT32, FP4, INT8, make_moe, zipf_router_bias
from tests.test_gpu_parity import SMALL, rel_err, say

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2
FP32_TOL = 1e-4


@pytest.fixture(scope="module")
def ctx():
    c = gt.Context(0)
    yield c
    c.close()


def oracle_routing(spec, x):
    logits = oracle.layer_forward(spec.router, x, threads=16)
    return oracle.route_from_logits(logits, spec.experts_per_token, spec.balance_biases)


def check_flips(gpu_chosen, ref, spec, label):
    k = spec.experts_per_token
    diff = np.nonzero(np.any(gpu_chosen != ref.chosen, axis=1))[0]
    for t in diff:
        s = np.sort(ref.affinities[t] + spec.balance_biases)[::-1]
        assert s[k - 1] - s[k] <= 1e-5 * max(1.0, abs(s[k - 1])), (label, t)
    say(f"[{label}] routing flips at near-ties: {len(diff)} of {len(gpu_chosen)} tokens")


def check_dispatch(r, E):
    d = oracle.dispatch(r.chosen, E)
    assert np.array_equal(r.load, d.load)
    assert np.array_equal(r.offsets, d.offsets)
    assert np.array_equal(r.rows, d.rows)


@pytest.mark.parametrize("name", list(SMALL))
@pytest.mark.parametrize("prec", [FLOAT32, INT8, FP4])
def test_small_layers_bf16_path(ctx, name, prec):
    say(f"bf16 small layer {name} precision {prec}")
    cfg = SMALL[name]
    spec = make_moe(gt.encode_rows, precision=prec, seed=7, std=0.3, bias_std=0.05, **cfg)
    rng = np.random.default_rng(8)
    T = 300
    x = rng.uniform(-1, 1, size=(T, cfg["d"]))
    ids = rng.integers(0, 1000, size=T) if cfg.get("use_hash") else None
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        y = m.forward(x, ids, path=gt.PATH_BF16)
        r = m.last_routing()
        assert m.last_path == gt.PATH_BF16
    finally:
        m.destroy()
    check_dispatch(r, cfg["E"])
    ref = oracle.moe_forward_routed(spec, x, r.chosen, r.gates)
    e = rel_err(y, ref.outputs)
    assert e <= BF16_TOL, e


def run_prefill(ctx, spec, x, ids=None):
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        y = m.forward(x, ids, path=gt.PATH_BF16)
        r = m.last_routing()
        assert m.last_path == gt.PATH_BF16
    finally:
        m.destroy()
    check_dispatch(r, len(spec.routed))
    ref = oracle.moe_forward_routed(spec, x, r.chosen, r.gates, threads=16)
    return y, ref.outputs


def row_rel_err(y, r):
    """Worst row of max |y - r| / max |r| (rows of any magnitude)."""
    return float(np.max(np.max(np.abs(y - r), axis=1) / np.max(np.abs(r), axis=1)))


@pytest.mark.parametrize("name", list(SMALL))
@pytest.mark.parametrize("prec", [FLOAT32, INT8, FP4])
def test_small_layers_past_the_fused_routing(ctx, name, prec):
    """T*k above the fused routing's 2048: the rows are prepared by the
    conversion kernel and routed by the separate router and top-k."""
    cfg = SMALL[name]
    T = 2048 // cfg["k"] + 37
    say(f"prefill past the fused routing {name} precision {prec} T={T}")
    spec = make_moe(gt.encode_rows, precision=prec, seed=17, std=0.3, bias_std=0.05, **cfg)
    rng = np.random.default_rng(18)
    x = rng.uniform(-1, 1, size=(T, cfg["d"]))
    ids = rng.integers(0, 1000, size=T) if cfg.get("use_hash") else None
    y, ref = run_prefill(ctx, spec, x, ids)
    e = rel_err(y, ref)
    say(f"[{name} / {prec}] max rel err {e:.3e}")
    assert e <= BF16_TOL, e


@pytest.mark.parametrize("prec", [INT8, FP4])
def test_rows_of_any_magnitude(ctx, prec):
    """Rows from 1e-8 to 1e8 in magnitude: every row to the bar on its own.
    Hash routing: learned routing of a 1e8 row can drive every affinity to
    zero and its gates to 0/0, in the reference as well."""
    say(f"prefill rows of any magnitude, precision {prec}")
    spec = make_moe(gt.encode_rows, d=96, h=64, E=8, k=2, S=1, precision=prec, seed=19, std=0.3, bias_std=0.05,
                    use_hash=True)
    rng = np.random.default_rng(20)
    T = 1100
    x = rng.uniform(-1, 1, size=(T, 96)) * (10.0 ** rng.integers(-8, 9, size=(T, 1)))
    ids = rng.integers(0, 1000, size=T)
    y, ref = run_prefill(ctx, spec, x, ids)
    e = row_rel_err(y, ref)
    say(f"[{prec}] worst row rel err {e:.3e}")
    assert e <= BF16_TOL, e


@pytest.mark.parametrize("prec", [INT8, FP4])
@pytest.mark.parametrize("std", [1e-6, 1e5])
def test_weights_of_extreme_scale(ctx, prec, std):
    """Block scales far from 1 in either direction (weights of std 1e-6 and
    1e5), to the same bar."""
    say(f"weights std {std} precision {prec}")
    spec = make_moe(gt.encode_rows, d=64, h=48, E=6, k=2, S=1, precision=prec, seed=21, std=std, router_std=0.3,
                    bias_std=0.0)
    x = np.random.default_rng(22).uniform(-1, 1, size=(1100, 64))
    y, ref = run_prefill(ctx, spec, x)
    e = rel_err(y, ref)
    say(f"[std {std} / {prec}] max rel err {e:.3e}")
    assert e <= BF16_TOL, e


def test_bf16_one_row_matches_many_rows(ctx):
    say("bf16 one row vs many rows")
    spec = make_moe(gt.encode_rows, d=128, h=192, E=4, k=2, S=1, seed=9, precision=INT8)
    x = np.random.default_rng(10).uniform(-1, 1, (200, 128))
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        allrows = m.forward(x, path=gt.PATH_BF16)
        for t in (0, 77, 199):
            one = m.forward(x[t:t + 1], path=gt.PATH_BF16)
            assert np.array_equal(one[0], allrows[t])
    finally:
        m.destroy()


def run_full(ctx, spec, x, sample, label, path=gt.PATH_AUTO, tol=BF16_TOL):
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        y = m.forward(x, path=path)
        r = m.last_routing()
        used = m.last_path
    finally:
        m.destroy()
    E = len(spec.routed)
    check_dispatch(r, E)
    check_flips(r.chosen, oracle_routing(spec, x), spec, label)
    ref = oracle.moe_forward_routed(spec, x[sample], r.chosen[sample], r.gates[sample], threads=16)
    e = rel_err(y[sample], ref.outputs)
    say(f"[{label}] path {used}, max rel err on {len(sample)} sampled tokens {e:.3e}")
    assert e <= tol
    return r, used


def test_c3_fp4_prefill(ctx):
    # d=1024, 64 routed + 1 shared expert, top-6, hidden 512, FP4, 4096 tokens
    say("C3 fp4 prefill T=4096")
    spec = make_moe(gt.encode_rows, d=1024, h=512, E=64, S=1, k=6, precision=FP4, seed=3)
    x = np.random.default_rng(3).normal(size=(4096, 1024))
    sample = np.sort(np.random.default_rng(33).choice(4096, 48, replace=False))
    _, used = run_full(ctx, spec, x, sample, "C3")
    assert used == gt.PATH_BF16


def test_c4_int8_skewed_prefill(ctx):
    # d=2048, 128 experts, top-8, hidden 768, Int8, 16384 tokens, Zipf(1.2) router-bias skew
    say("C4 int8 skewed prefill T=16384")
    bias = zipf_router_bias(128, 1.2, seed=4, scale=0.6)
    spec = make_moe(gt.encode_rows, d=2048, h=768, E=128, S=0, k=8, precision=INT8, seed=4, router_bias=bias)
    x = np.random.default_rng(4).normal(size=(16384, 2048))
    sample = np.sort(np.random.default_rng(44).choice(16384, 24, replace=False))
    r, used = run_full(ctx, spec, x, sample, "C4")
    assert used == gt.PATH_BF16
    load = np.sort(r.load)[::-1]
    say(f"[C4] realized loads (desc), first 8: {load[:8].tolist()}, median {int(np.median(load))}, "
        f"min {int(load[-1])}")


@pytest.mark.parametrize("T,path,tol", [(64, gt.PATH_AUTO, FP32_TOL), (1024, gt.PATH_AUTO, BF16_TOL)])
def test_c5_shaped_stack(ctx, T, path, tol):
    # per layer d=2048, 64 experts + 1 shared, top-4, hidden 1024, FP4; 3 layers
    say(f"C5-shaped stack, 3 layers, T={T}")
    layers = [make_moe(gt.encode_rows, d=2048, h=1024, E=64, S=1, k=4, precision=FP4, seed=50 + i)
              for i in range(3)]
    norms = [np.ones(2048)] * 3
    x0 = np.random.default_rng(5).normal(size=(T, 2048))
    ms = [gt.MixtureOfExperts.from_spec(ctx, s) for s in layers]
    try:
        for m, w in zip(ms, norms):
            m.set_norm_weights(w)
        x, chosen, gates = gt.stack_forward(ms, x0, path=path, with_routing=True)
        used = ms[0].last_path
    finally:
        for m in ms:
            m.destroy()
    sample = np.sort(np.random.default_rng(55).choice(T, min(T, 24), replace=False))
    ref = oracle.stack_forward_routed(layers, norms, x0[sample], chosen[:, sample], gates[:, sample], threads=16)
    e = rel_err(x[sample], ref)
    say(f"[C5 stack T={T}] path {used}, max rel err {e:.3e}")
    assert e <= tol


@pytest.mark.parametrize("path,T", [(gt.PATH_BF16, 1100), (gt.PATH_FP32, 300)])
def test_device_buffers_off_16_byte_alignment(ctx, path, T):
    """forward_device on caller buffers that start 4 bytes past a 16-byte
    boundary (the combine then takes its scalar stores) gives the same bits
    as on aligned buffers."""
    import torch
    say(f"device buffers off alignment, path {path}, T={T}")
    d = 64
    spec = make_moe(gt.encode_rows, d=d, h=96, E=8, k=3, S=1, precision=INT8, seed=31, std=0.1, bias_std=0.02)
    x = np.random.default_rng(32).uniform(-1, 1, (T, d)).astype(np.float32)
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        xa = torch.from_numpy(x).cuda()
        ya = torch.full((T, d), float("nan"), device="cuda")
        xbuf = torch.zeros(T * d + 4, device="cuda")
        ybuf = torch.full((T * d + 4,), float("nan"), device="cuda")
        xo, yo = xbuf[1:1 + T * d], ybuf[1:1 + T * d]  # 4 bytes past the allocation's alignment
        xo.copy_(xa.reshape(-1))
        assert xo.data_ptr() % 16 == 4 and yo.data_ptr() % 16 == 4
        m.forward_device(T, xa.data_ptr(), ya.data_ptr(), path=path)
        m.forward_device(T, xo.data_ptr(), yo.data_ptr(), path=path)
        torch.cuda.synchronize()
        assert m.last_path == path
        a, b = ya.cpu().numpy(), yo.cpu().numpy().reshape(T, d)
    finally:
        m.destroy()
    assert np.all(np.isfinite(a))
    assert np.array_equal(a, b)


@pytest.mark.parametrize("T,E", [(4100, 64), (8200, 128), (1100, 8)])
def test_fp32_rows_converted_by_the_router(ctx, T, E):
    """fp32 device rows on the bf16 path, read in place by the router: at
    4100 tokens x 64 experts and 8200 x 128 the staged router writes the
    bf16 rows itself (one and two expert tiles per workgroup, a last token
    tile part-filled); at 1100 x 8 the rows are converted first.  Two calls
    with different rows (a row left unwritten would keep the first call's
    values), each against the float64-input forward of the same values,
    whose rows go through the separate conversion, and the oracle on a
    sample."""
    import torch
    say(f"fp32 rows converted by the router, T={T} E={E}")
    d = 256
    spec = make_moe(gt.encode_rows, d=d, h=64, E=E, k=2, S=1, precision=FP4, seed=41, std=0.2, bias_std=0.05)
    rng = np.random.default_rng(42)
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        for call in range(2):
            x = rng.uniform(-1, 1, (T, d)).astype(np.float32)
            xa = torch.from_numpy(x).cuda()
            ya = torch.full((T, d), float("nan"), device="cuda")
            torch.cuda.synchronize()
            m.forward_device(T, xa.data_ptr(), ya.data_ptr(), path=gt.PATH_BF16)
            torch.cuda.synchronize()
            assert m.last_path == gt.PATH_BF16
            y = ya.cpu().numpy().astype(np.float64)
            r = m.last_routing()
            y64 = m.forward(x.astype(np.float64), path=gt.PATH_BF16)
            r64 = m.last_routing()
            assert np.array_equal(r.chosen, r64.chosen), call
            e = float(np.max(np.abs(y - y64)) / np.max(np.abs(y64)))
            say(f"[T={T} E={E} call {call}] max rel diff to the float64-input forward {e:.3e}")
            assert e <= 1e-6, (call, e)
            sample = np.sort(rng.choice(T, 16, replace=False))
            sample[-1] = T - 1
            ref = oracle.moe_forward_routed(spec, x[sample].astype(np.float64), r.chosen[sample], r.gates[sample],
                                            threads=16)
            assert rel_err(y[sample], ref.outputs) <= BF16_TOL
    finally:
        m.destroy()


@pytest.mark.parametrize("d,hash_mid", [(128, False), (128, True), (96, False)])
def test_bf16_stack_norm_done_by_the_combine(ctx, d, hash_mid):
    """A bf16 stack past the fused routing (T*k > 2048).  With d a multiple of
    64 each layer's combine also writes the next layer's normalised bf16 rows
    and inverse RMS, and the next router reads the raw rows against its rows
    times the norm weights; d = 96 keeps the separate RMSNorm pass.  A
    hash-routed middle layer takes the normalised rows without a router."""
    say(f"bf16 stack, norm in the combine, d={d} hash_mid={hash_mid}")
    T = 600
    rng = np.random.default_rng(70 + d)
    specs = [make_moe(gt.encode_rows, d=d, h=64, E=8, k=4, S=1, precision=FP4, seed=71 + i, std=0.1,
                      bias_std=0.01, use_hash=hash_mid and i == 1) for i in range(3)]
    norms = [1.0 + 0.2 * rng.standard_normal(d) for _ in range(3)]
    x0 = rng.standard_normal((T, d))
    ids = rng.integers(0, 10000, T) if hash_mid else None
    ms = [gt.MixtureOfExperts.from_spec(ctx, s) for s in specs]
    try:
        for m, w in zip(ms, norms):
            m.set_norm_weights(w)
        x, chosen, gates = gt.stack_forward(ms, x0, ids, path=gt.PATH_BF16, with_routing=True)
        assert all(m.last_path == gt.PATH_BF16 for m in ms)
    finally:
        for m in ms:
            m.destroy()
    ref = oracle.stack_forward_routed(specs, norms, x0, chosen, gates, threads=16)
    e = rel_err(x, ref)
    say(f"[d={d} hash_mid={hash_mid}] max rel err {e:.3e}")
    assert e <= BF16_TOL
