"""GPU parity of libgtmoe against the CPU oracle (restating the reference's
float64 path), through the C ABI.

Bars (stated per test):
* routing from given logits: chosen experts, gates, load and the dispatch
  permutation bit-exact;
* end-to-end routing: equal to the oracle's except at near-ties of the k-th
  and (k+1)-th score (the device computes router logits in fp32); every flip
  is checked to be such a near tie and reported;
* layer outputs under the device's routing: max |y - r| / max |r| <= 1e-4 on
  the fp32 path, <= 2e-2 on the bf16 MFMA path."""
import sys

import numpy as np
import pytest

import gotransformers_amd as gt
import oracle

torch = pytest.importorskip("torch")
from tests.moe_fixtures import FLOAT32, FP4, INT8, make_moe, zipf_router_bias

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
BF16_TOL = 2e-2


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = gt.Context(0)
    yield c
    c.close()


def rel_err(y, r):
    return float(np.max(np.abs(y - r)) / max(float(np.max(np.abs(r))), 1e-30))


def check_routing(gpu_chosen, spec, x, k, label):
    """Compare the device routing with the oracle's own; flips are allowed only
    at near-ties of the k-th and (k+1)-th score.  Returns the flip count."""
    ref = oracle.moe_forward(spec, x)
    diff = np.nonzero(np.any(gpu_chosen != ref.chosen, axis=1))[0]
    for t in diff:
        s = np.sort(ref.affinities[t] + spec.balance_biases)[::-1]
        gap = s[k - 1] - s[k]
        assert gap <= 1e-5 * max(1.0, abs(s[k - 1])), (label, t, gap)
    say(f"[{label}] routing flips at near-ties: {len(diff)} of {len(x)} tokens")
    return len(diff), ref


def run_layer(ctx, spec, x, path, token_ids=None):
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        y = m.forward(x, token_ids, path=path)
        r = m.last_routing()
        used = m.last_path
    finally:
        m.destroy()
    return y, r, used


# --------------------------------------------------------------------------- routing

@pytest.mark.parametrize("E,k", [(8, 2), (16, 2), (64, 6), (128, 8), (256, 8), (5, 5), (3, 1), (64, 4)])
def test_route_from_logits_bit_exact(ctx, E, k):
    say(f"route_from_logits E={E} k={k}")
    rng = np.random.default_rng(100 + E + k)
    T = 3000
    logits = rng.normal(0, 1.0, size=(T, E))
    logits[:200] = rng.uniform(-30, 30, size=(200, E))  # all softplus branches
    logits[200:300, 1] = logits[200:300, 0]  # exact ties
    logits[300:320] = 0.5  # everything tied
    bal = rng.normal(0, 0.05, size=E)
    bal[E // 2] = bal[0]
    spec = make_moe(gt.encode_rows, d=4, h=4, E=E, k=k, seed=1)
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        m.balance_biases = bal
        got = m.route_from_logits(logits)
    finally:
        m.destroy()
    want = oracle.route_from_logits(logits, k, bal)
    assert np.array_equal(got.chosen, want.chosen)
    assert np.array_equal(got.gates.view(np.int64), want.gates.view(np.int64))
    d = oracle.dispatch(want.chosen, E)
    assert np.array_equal(got.load, d.load)
    assert np.array_equal(got.offsets, d.offsets)
    assert np.array_equal(got.rows, d.rows)


def same_gates(got, want):
    """Bit-equal gates, NaN where the oracle's are NaN (a chosen expert with a
    NaN affinity makes every gate of its token NaN)."""
    nan = np.isnan(want)
    return bool(np.array_equal(np.isnan(got), nan) and np.array_equal(got[~nan].view(np.int64),
                                                                      want[~nan].view(np.int64)))


@pytest.mark.parametrize("E,k", [(8, 2), (21, 3), (32, 4), (64, 6), (128, 8), (256, 8)])
def test_route_from_logits_with_some_nan_scores(ctx, E, k):
    """Rows with one to five NaN logits, and a NaN balance bias: no NaN
    compares greater or less than anything, so the reference's choice is
    whatever sort.SliceStable's block insertion sort and SymMerge leave
    (mixtureofexperts.go:106).  The many-token top-k repeats that sort for
    such rows: chosen experts, load and permutation bit-exact, gates bit-exact
    or NaN where the oracle's are."""
    say(f"route_from_logits with NaN scores E={E} k={k}")
    rng = np.random.default_rng(500 + E + k)
    T = 400
    logits = rng.normal(0, 1.0, size=(T, E))
    for t in range(T):
        logits[t, rng.choice(E, size=1 + t % 5, replace=False)] = np.nan
    logits[::7] = rng.normal(0, 1.0, size=logits[::7].shape)  # rows without NaN in between
    bal = rng.normal(0, 0.05, size=E)
    if E >= 32:
        bal[E // 3] = np.nan
    spec = make_moe(gt.encode_rows, d=4, h=4, E=E, k=k, seed=1)
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        m.balance_biases = bal
        got = m.route_from_logits(logits)
    finally:
        m.destroy()
    with np.errstate(invalid="ignore"):
        want = oracle.route_from_logits(logits, k, bal)
    assert np.array_equal(got.chosen, want.chosen)
    assert same_gates(got.gates, want.gates)
    d = oracle.dispatch(want.chosen, E)
    assert np.array_equal(got.load, d.load)
    assert np.array_equal(got.rows, d.rows)


@pytest.mark.parametrize("E,k", [(32, 4), (64, 4), (96, 2), (256, 8)])
def test_decode_routing_with_some_nan_scores(ctx, E, k):
    """The decode routing kernel (one to eight workgroups per token) on rows
    with NaN scores: a router of zero weights makes every logit its bias, three
    biases are NaN and one balance bias is; chosen experts and gates against
    the oracle's routing of the same float64 logits."""
    say(f"decode routing with NaN scores E={E} k={k}")
    d, T = 64, 6
    rng = np.random.default_rng(600 + E)
    spec = make_moe(gt.encode_rows, d=d, h=64, E=E, k=k, S=0, precision=INT8, seed=15)
    spec.router.weights = gt.encode_rows(FLOAT32, np.zeros((E, d)))
    bias = rng.normal(0, 1.0, size=E)
    bias[rng.choice(E, size=3, replace=False)] = np.nan
    spec.router.biases = bias
    balance = rng.normal(0, 0.05, size=E)
    balance[(E // 2 + 1) % E] = np.nan
    x = rng.uniform(-1, 1, (T, d))
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        m.balance_biases = balance
        m.forward(x, path=gt.PATH_FP32)
        r = m.last_routing()
    finally:
        m.destroy()
    with np.errstate(invalid="ignore"):
        want = oracle.route_from_logits(np.tile(bias, (T, 1)), k, balance)
    assert np.array_equal(r.chosen, want.chosen)
    assert same_gates(r.gates, want.gates)


def test_hash_routing_matches_closed_form(ctx):
    say("hash routing forward")
    spec = make_moe(gt.encode_rows, d=32, h=48, E=8, k=3, S=1, seed=3, use_hash=True, precision=INT8)
    ids = np.array([0, 1, 2, 42, 9, 42, 2**40 + 7, 123456789, 5, 5])
    x = np.random.default_rng(4).normal(size=(len(ids), 32))
    y, r, _ = run_layer(ctx, spec, x, gt.PATH_FP32, ids)
    want = oracle.hash_route(ids, 8, 3)
    assert np.array_equal(r.chosen, want.chosen)
    assert np.all(r.gates == 1.0 / 3)
    ref = oracle.moe_forward(spec, x, ids)
    assert rel_err(y, ref.outputs) <= FP32_TOL


# --------------------------------------------------------------------------- forward, fp32 path

SMALL = {
    # the reference's own test shapes (mixtureofexperts_test.go:13-20)
    "routed, no shared": dict(d=4, h=6, E=4, k=2, S=0),
    "routed with shared": dict(d=4, h=6, E=4, k=2, S=1),
    "hashed with shared": dict(d=4, h=6, E=4, k=2, S=1, use_hash=True),
    "routed, one per row": dict(d=4, h=6, E=5, k=1, S=1),
    "clamped": dict(d=4, h=6, E=4, k=2, S=1, clamp=0.5),
    "ragged widths": dict(d=37, h=53, E=7, k=3, S=2),
    "wide": dict(d=130, h=70, E=9, k=4, S=1),
}


@pytest.mark.parametrize("name", list(SMALL))
@pytest.mark.parametrize("prec", [FLOAT32, INT8, FP4])
def test_small_layers_fp32_path(ctx, name, prec):
    say(f"small layer {name} precision {prec}")
    cfg = SMALL[name]
    spec = make_moe(gt.encode_rows, precision=prec, seed=7, std=0.3, bias_std=0.05, **cfg)
    T = 29
    rng = np.random.default_rng(8)
    x = rng.uniform(-1, 1, size=(T, cfg["d"]))
    ids = rng.integers(0, 1000, size=T) if cfg.get("use_hash") else None
    y, r, used = run_layer(ctx, spec, x, gt.PATH_FP32, ids)
    assert used == gt.PATH_FP32
    if not cfg.get("use_hash"):
        check_routing(r.chosen, spec, x, cfg["k"], name)
    ref = oracle.moe_forward_routed(spec, x, r.chosen, r.gates)
    assert np.array_equal(r.load, ref.load)
    assert rel_err(y, ref.outputs) <= FP32_TOL, rel_err(y, ref.outputs)


def test_c1_float32_layer(ctx):
    # d=256, 8 routed experts, top-2, hidden 512, 128 tokens, float32 weights
    say("C1 float32 d256 E8 k2 h512 T128")
    spec = make_moe(gt.encode_rows, d=256, h=512, E=8, k=2, S=0, precision=FLOAT32, seed=0)
    x = np.random.default_rng(0).normal(size=(128, 256))
    y, r, used = run_layer(ctx, spec, x, gt.PATH_FP32)
    assert used == gt.PATH_FP32
    check_routing(r.chosen, spec, x, 2, "C1")
    ref = oracle.moe_forward_routed(spec, x, r.chosen, r.gates, threads=8)
    e = rel_err(y, ref.outputs)
    say(f"C1 max rel err {e:.3e}")
    assert e <= FP32_TOL


@pytest.mark.parametrize("T", [1, 8, 32])
def test_c2_int8_decode(ctx, T):
    # d=1024, 16 experts, top-2, hidden 2048, Int8 experts (per-16 absmax/127)
    say(f"C2 int8 decode T={T}")
    spec = make_moe(gt.encode_rows, d=1024, h=2048, E=16, k=2, S=0, precision=INT8, seed=0)
    x = np.random.default_rng(T).normal(size=(T, 1024))
    y, r, used = run_layer(ctx, spec, x, gt.PATH_AUTO)
    assert used == gt.PATH_FP32
    check_routing(r.chosen, spec, x, 2, f"C2 T={T}")
    ref = oracle.moe_forward_routed(spec, x, r.chosen, r.gates, threads=8)
    e = rel_err(y, ref.outputs)
    say(f"C2 T={T} max rel err {e:.3e}")
    assert e <= FP32_TOL


FEW = {
    "C5 block, 16 experts": (dict(d=2048, h=1024, E=16, k=4, S=1), FP4),
    "C2 shape": (dict(d=1024, h=2048, E=16, k=2, S=0), FP4),
    "clamped, one shared": (dict(d=512, h=512, E=4, k=2, S=1, clamp=0.3, std=0.05), INT8),
    "hashed, two shared": (dict(d=512, h=1024, E=8, k=3, S=2, use_hash=True), FP4),
}


@pytest.mark.parametrize("name", list(FEW))
def test_few_token_decode(ctx, name):
    """Up to six tokens through a layer at least 512 values wide run the
    few-token expert kernels (each (token, slot) pair's and each (shared
    expert, token) pair's rows spread over the whole GPU, 8 or 16 rows per
    workgroup); the results must match the oracle under the device's
    routing, as the many-token kernels' do, at one token and at six (one
    layer object, so both calls also share its workspace)."""
    cfg, prec = FEW[name]
    spec = make_moe(gt.encode_rows, precision=prec, seed=21, **cfg)
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        for T in (1, 6):
            say(f"few tokens {name} T={T}")
            rng = np.random.default_rng(22 + T)
            x = rng.normal(size=(T, cfg["d"]))
            ids = rng.integers(0, 5000, T) if cfg.get("use_hash") else None
            y = m.forward(x, ids, path=gt.PATH_AUTO)
            r = m.last_routing()
            assert m.last_path == gt.PATH_FP32
            if ids is None:
                check_routing(r.chosen, spec, x, cfg["k"], f"few tokens {name} T={T}")
            else:
                assert np.array_equal(r.chosen, oracle.hash_route(ids, cfg["E"], cfg["k"]).chosen)
            # the dispatch tables, built on request, agree with the oracle's
            assert np.array_equal(m.last_expert_load(), oracle.dispatch(r.chosen, cfg["E"]).load)
            ref = oracle.moe_forward_routed(spec, x, r.chosen, r.gates, threads=8)
            e = rel_err(y, ref.outputs)
            say(f"few tokens {name} T={T} max rel err {e:.3e}")
            assert e <= FP32_TOL
    finally:
        m.destroy()


@pytest.mark.parametrize("name,cfg,prec,T", [
    ("C2 top-2", dict(d=1024, h=2048, E=16, k=2, S=0), INT8, 1),
    ("C2 top-2", dict(d=1024, h=2048, E=16, k=2, S=0), INT8, 32),
    ("top-2, two slices per expert", dict(d=4, h=6, E=4, k=2, S=0), FP4, 29),
    ("top-1 with one shared", dict(d=37, h=53, E=5, k=1, S=1), INT8, 29),
])
def test_device_forward_folds_two_term_combine(ctx, name, cfg, prec, T):
    """With at most two contributions per output row (shared + routed <= 2)
    the fp32 device forward adds them straight into the zeroed outputs from
    the down kernel; fp32 addition of two terms onto zero does not depend on
    their order, so repeated forwards are bit-identical, and the result
    matches the oracle and the host-path forward (which runs the combine
    kernel)."""
    say(f"folded combine {name} T={T}")
    spec = make_moe(gt.encode_rows, precision=prec, seed=9, std=0.1, bias_std=0.02, **cfg)
    x = np.random.default_rng(10 + T).normal(size=(T, cfg["d"]))
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        xd = torch.from_numpy(x.astype(np.float32)).cuda()
        y1 = torch.full((T, cfg["d"]), float("nan"), device="cuda")
        y2 = torch.full((T, cfg["d"]), float("nan"), device="cuda")
        m.forward_device(T, xd.data_ptr(), y1.data_ptr(), path=gt.PATH_FP32)
        m.forward_device(T, xd.data_ptr(), y2.data_ptr(), path=gt.PATH_FP32)
        torch.cuda.synchronize()
        r = m.last_routing()
        a, b = y1.cpu().numpy(), y2.cpu().numpy()
        host = m.forward(x.astype(np.float32).astype(np.float64), path=gt.PATH_FP32)
    finally:
        m.destroy()
    assert np.array_equal(a, b)
    assert np.all(np.isfinite(a))
    ref = oracle.moe_forward_routed(spec, x.astype(np.float32).astype(np.float64), r.chosen, r.gates)
    assert rel_err(a, ref.outputs) <= FP32_TOL
    assert rel_err(a, host) <= 1e-6


@pytest.mark.parametrize("d,h,T", [(4096, 192, 16), (192, 4096, 64)])
def test_widest_decode_gemv(ctx, d, h, T):
    """The fp32 path at its widest K (4096): the gate/up (d) or down (h)
    kernel stages 8 tokens x 4096 values as bf16 hi/lo (128 KiB of LDS) plus
    the self-dispatch entry list."""
    say(f"widest GEMV d={d} h={h} T={T}")
    spec = make_moe(gt.encode_rows, d=d, h=h, E=6, k=3, S=1, precision=FP4, seed=15, std=0.02, bias_std=0.01)
    x = np.random.default_rng(16).uniform(-1, 1, (T, d))
    y, r, used = run_layer(ctx, spec, x, gt.PATH_FP32)
    assert used == gt.PATH_FP32
    ref = oracle.moe_forward_routed(spec, x, r.chosen, r.gates, threads=8)
    e = rel_err(y, ref.outputs)
    say(f"widest GEMV max rel err {e:.2e}")
    assert e <= FP32_TOL


@pytest.mark.parametrize("E,k", [(16, 3), (64, 4), (96, 2)])
def test_decode_routing_ties_and_nan_match_the_oracle(ctx, E, k):
    """The decode routing kernel (ranked choice for E <= 64, rounds of
    arg-max above) on logits with exact ties and NaN: a router of zero
    weights makes every logit of a token equal to its bias, and a NaN input
    makes a token's logits NaN.  Chosen experts and gates are bit-exact
    against the oracle's routing of the same float64 logits."""
    say(f"decode routing ties/NaN E={E} k={k}")
    d, T = 64, 6
    spec = make_moe(gt.encode_rows, d=d, h=64, E=E, k=k, S=0, precision=INT8, seed=13)
    spec.router.weights = gt.encode_rows(FLOAT32, np.zeros((E, d)))
    bias = np.zeros(E)
    bias[E // 3] = bias[E // 2] = 0.25  # a tie above the rest
    spec.router.biases = bias
    balance = np.zeros(E)
    balance[1] = balance[E - 1] = 0.125  # ties among the balance-lifted experts
    x = np.random.default_rng(14).uniform(-1, 1, (T, d))
    x[2, 5] = np.nan
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        m.balance_biases = balance
        with np.errstate(invalid="ignore"):
            m.forward(x, path=gt.PATH_FP32)
        r = m.last_routing()
    finally:
        m.destroy()
    logits = np.tile(bias, (T, 1))
    logits[2] = np.nan
    want = oracle.route_from_logits(logits, k, balance)
    assert np.array_equal(r.chosen, want.chosen)
    finite = np.arange(T) != 2
    assert np.array_equal(r.gates[finite].view(np.int64), want.gates[finite].view(np.int64))
    assert np.all(np.isnan(r.gates[2])) and np.all(np.isnan(want.gates[2]))


@pytest.mark.parametrize("T", [1, 17, 64, 65])
@pytest.mark.parametrize("use_hash", [False, True])
def test_decode_kernels_find_their_own_tokens(ctx, T, use_hash):
    """Up to 64 tokens the fp32 path launches no dispatch: the expert kernels
    read the routing choices directly (a hot expert takes many passes of 8
    tokens), and the dispatch tables a caller reads afterwards (load,
    rowsForExpert, offsets) are built on request and equal the oracle's
    dispatch of the same choices.  65 tokens takes the dispatch path; both
    agree with the oracle."""
    say(f"decode without dispatch T={T} hash={use_hash}")
    cfg = dict(d=96, h=80, E=6, k=3, S=2)
    spec = make_moe(gt.encode_rows, precision=FP4, seed=12, std=0.2, bias_std=0.02, use_hash=use_hash, **cfg)
    if not use_hash:
        spec.router.biases = zipf_router_bias(cfg["E"], 2.0, seed=3, scale=4.0)  # one expert takes most tokens
    rng = np.random.default_rng(20 + T)
    x = rng.uniform(-1, 1, (T, cfg["d"]))
    ids = rng.integers(0, 5000, T) if use_hash else None
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        y = m.forward(x, ids, path=gt.PATH_FP32)
        load = m.last_expert_load()
        r = m.last_routing()
        y2 = m.forward(x, ids, path=gt.PATH_FP32)
    finally:
        m.destroy()
    assert np.array_equal(y, y2)
    d = oracle.dispatch(r.chosen, cfg["E"])
    assert np.array_equal(load, d.load)
    assert np.array_equal(r.load, d.load)
    assert np.array_equal(r.offsets, d.offsets)
    assert np.array_equal(r.rows, d.rows)
    if not use_hash:
        assert d.load.max() >= min(T, 17), d.load  # the skew gives many passes to one expert
    ref = oracle.moe_forward_routed(spec, x, r.chosen, r.gates)
    assert rel_err(y, ref.outputs) <= FP32_TOL


# --------------------------------------------------------------------------- reference invariants on the device

@pytest.mark.parametrize("path", [gt.PATH_FP32])
@pytest.mark.parametrize("use_hash", [False, True])
def test_one_row_matches_many_rows(ctx, path, use_hash):
    # mixtureofexperts_test.go:83-100; on the device each row's result does
    # not depend on the other rows, so the match is exact.
    say(f"one row vs many rows hash={use_hash}")
    spec = make_moe(gt.encode_rows, d=64, h=96, E=4, k=2, S=1, seed=9, use_hash=use_hash, precision=FP4)
    ids = np.array([4, 8, 15, 16])
    x = np.random.default_rng(10).uniform(-1, 1, (4, 64))
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        allrows = m.forward(x, ids, path=path)
        for t in range(4):
            one = m.forward(x[t:t + 1], ids[t:t + 1], path=path)
            assert np.array_equal(one[0], allrows[t])
    finally:
        m.destroy()


def test_update_balance_evens_out_load(ctx):
    # mixtureofexperts_test.go:116-147
    say("update balance")
    spec = make_moe(gt.encode_rows, d=4, h=6, E=4, k=1, S=0, seed=11, std=0.5, router_std=0.5,
                    router_bias=[3.0, 0, 0, 0])
    x = np.random.default_rng(12).uniform(-1, 1, (64, 4))
    m = gt.MixtureOfExperts.from_spec(ctx, spec)

    def imbalance(load):
        return int(load.max() - load.min())
    try:
        m.forward(x)
        start = m.last_expert_load()
        m.update_balance(0.05)
        bb = m.balance_biases
        assert bb[0] < 0
        for e in range(1, 4):
            if start[e] < 16:
                assert bb[e] > 0
        for _ in range(300):
            m.forward(x)
            m.update_balance(0.05)
        total = 0
        for _ in range(50):
            m.forward(x)
            total += imbalance(m.last_expert_load())
            m.update_balance(0.05)
        assert total / 50 <= imbalance(start) / 2
    finally:
        m.destroy()


def test_balance_biases_do_not_change_outputs_when_every_expert_is_chosen(ctx):
    # mixtureofexperts_test.go:149-160
    say("k = E balance biases")
    spec = make_moe(gt.encode_rows, d=16, h=24, E=3, k=3, seed=13, std=0.3)
    x = np.random.default_rng(14).uniform(-1, 1, (2, 16))
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        before = m.forward(x, path=gt.PATH_FP32)
        m.balance_biases = [0.0, 100.0, 0.0]
        after = m.forward(x, path=gt.PATH_FP32)
        assert np.array_equal(before, after)
    finally:
        m.destroy()


def test_errors_mirror_reference_panics(ctx):
    say("errors")
    with pytest.raises(gt.InvalidArgument):
        gt.MixtureOfExperts(ctx, 4, 6, 0, 2, 3)  # more experts per token than experts
    with pytest.raises(gt.InvalidArgument):
        gt.MixtureOfExperts(ctx, 4, 6, 1, 0, 1)  # no routed experts
    spec = make_moe(gt.encode_rows, d=8, h=8, E=4, k=2, seed=15, use_hash=True)
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        with pytest.raises(gt.InvalidArgument):
            m.forward(np.zeros((2, 8)), None)  # hash routing without token IDs
        with pytest.raises(gt.InvalidArgument):
            m.forward(np.zeros((2, 8)), [1, -2])  # negative token ID
        with pytest.raises(gt.InvalidArgument):
            m.forward(np.zeros((2, 5)), [1, 2])  # wrong vector size
    finally:
        m.destroy()
    fresh = gt.MixtureOfExperts(ctx, 8, 8, 0, 4, 2, INT8)
    try:
        with pytest.raises(gt.GtmoeError) as info:
            fresh.forward(np.zeros((1, 8)))
        assert info.value.code == gt.ERR_NOT_READY
        with pytest.raises(gt.GtmoeError):
            fresh.last_expert_load()  # before any Forward
        bad = gt.encode_rows(FP4, np.zeros((8, 8)))
        with pytest.raises(gt.InvalidArgument):
            fresh.upload("routed", 0, "gate", bad, np.zeros(8))  # precision differs from the layer
    finally:
        fresh.destroy()


def test_zero_tokens(ctx):
    say("zero tokens")
    spec = make_moe(gt.encode_rows, d=8, h=8, E=4, k=2, seed=16)
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        y = m.forward(np.zeros((0, 8)))
        assert y.shape == (0, 8)
        assert np.array_equal(m.last_expert_load(), np.zeros(4, np.int32))
    finally:
        m.destroy()


# --------------------------------------------------------------------------- stack

def test_small_stack_fp32(ctx):
    say("stack of 3 layers fp32 path")
    layers = [make_moe(gt.encode_rows, d=64, h=48, E=8, k=2, S=1, seed=20 + i, precision=FP4) for i in range(3)]
    norms = [np.ones(64), np.linspace(0.5, 1.5, 64), np.ones(64)]
    x0 = np.random.default_rng(21).normal(size=(12, 64))
    ms = [gt.MixtureOfExperts.from_spec(ctx, s) for s in layers]
    try:
        for m, w in zip(ms, norms):
            m.set_norm_weights(w)
        x, chosen, gates = gt.stack_forward(ms, x0, path=gt.PATH_FP32, with_routing=True)
    finally:
        for m in ms:
            m.destroy()
    ref = oracle.stack_forward_routed(layers, norms, x0, chosen, gates)
    assert rel_err(x, ref) <= FP32_TOL


def test_device_forward_refuses_overlapping_buffers(ctx):
    """A forward does not run in place: overlapping inputs and outputs are
    refused before anything is enqueued (the routing may clear the outputs
    while input rows are still being read)."""
    say("device forward in place refused")
    spec = make_moe(gt.encode_rows, d=32, h=48, E=4, k=2, S=0, precision=INT8, seed=17)
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        buf = torch.zeros(8 * 32 + 16, device="cuda")
        with pytest.raises(gt.InvalidArgument, match="overlap"):
            m.forward_device(8, buf.data_ptr(), buf.data_ptr())
        with pytest.raises(gt.InvalidArgument, match="overlap"):
            m.forward_device(8, buf.data_ptr(), buf[16:].data_ptr())
        # adjacent, not overlapping: accepted
        x = torch.from_numpy(np.random.default_rng(18).standard_normal(8 * 32).astype(np.float32)).cuda()
        buf[:8 * 32].copy_(x)
        out = torch.empty(8 * 32, device="cuda")
        m.forward_device(8, buf.data_ptr(), out.data_ptr(), path=gt.PATH_FP32)
        torch.cuda.synchronize()
        r = m.last_routing()
    finally:
        m.destroy()
    xs = x.cpu().numpy().astype(np.float64).reshape(8, 32)
    ref = oracle.moe_forward_routed(spec, xs, r.chosen, r.gates)
    assert rel_err(out.cpu().numpy().reshape(8, 32), ref.outputs) <= FP32_TOL


def test_stack_routing_outputs_need_one_k(ctx):
    """gtmoe_stack_forward's routing outputs are [n_layers][T][k]: layers
    with different k are refused when they are asked for, and run when not."""
    say("stack with different k")
    specs = [make_moe(gt.encode_rows, d=32, h=48, E=6, k=k, S=1, seed=19 + k, precision=INT8) for k in (2, 3)]
    ms = [gt.MixtureOfExperts.from_spec(ctx, s) for s in specs]
    try:
        for m in ms:
            m.set_norm_weights(np.ones(32))
        x0 = np.random.default_rng(20).standard_normal((5, 32))
        with pytest.raises(gt.InvalidArgument, match="one k"):
            gt.stack_forward(ms, x0, with_routing=True)
        x = gt.stack_forward(ms, x0)
    finally:
        for m in ms:
            m.destroy()
    assert np.all(np.isfinite(x))
