"""Pins the CPU oracle against the reference's own known answers and
invariants, closed forms, and independent numpy brute force.

Reference tests followed: lowprecision/lowprecision_test.go:9-103,
mixtureofexperts/mixtureofexperts_test.go:37-160,
normalization/normalization_test.go (RMS of the output is 1)."""
import math

import numpy as np
import pytest

import oracle
from tests.moe_fixtures import FLOAT32, FLOAT64, FP4, INT8, make_moe

PRECISIONS = [FLOAT64, FLOAT32, INT8, FP4]


def ulp_diff(a, b):
    """Distance in units in the last place between two float64 arrays."""
    ia = np.asarray(a, np.float64).view(np.int64)
    ib = np.asarray(b, np.float64).view(np.int64)
    ia = np.where(ia < 0, np.int64(-(2**63)) - ia, ia)
    ib = np.where(ib < 0, np.int64(-(2**63)) - ib, ib)
    return np.abs(ia - ib)


# ---------------------------------------------------------------- encoders

def test_fp4_keeps_exact_values():
    # lowprecision_test.go:39-47
    values = np.array([0, 0.5, -1, 1.5, 2, -3, 4, 6, -6, 3], np.float64)
    r = oracle.encode_rows(FP4, values)
    assert np.array_equal(oracle.decode_rows(r)[0], values)


def test_bytes_used():
    # lowprecision_test.go:49-64: Float64 10*64*8, FP4 10*(32+4*4)
    zeros = np.zeros((10, 64))
    sizes = {}
    for p in PRECISIONS:
        r = oracle.encode_rows(p, zeros)
        sizes[p] = r.values.nbytes + (0 if r.scales is None else r.scales.nbytes)
    assert sizes[FLOAT64] == 10 * 64 * 8
    assert sizes[FP4] == 10 * (32 + 4 * 4)
    assert sizes[INT8] == 10 * (64 + 4 * 4)
    assert sizes[FLOAT64] > sizes[FLOAT32] > sizes[INT8] > sizes[FP4]


def test_rows_keep_values_close_enough():
    # lowprecision_test.go:9-37: U(-3,3), width 37, error <= 3 * allowed
    rng = np.random.default_rng(1)
    allowed = {FLOAT64: 0, FLOAT32: 1e-6, INT8: 0.01, FP4: 0.25}
    for p, a in allowed.items():
        values = rng.uniform(-3, 3, size=(5, 37))
        back = oracle.decode_rows(oracle.encode_rows(p, values))
        assert np.max(np.abs(back - values)) <= 3 * a, p


def test_int8_closed_form():
    # scale = float32(absmax/127); q = round half away from zero of v/scale
    v = np.array([127.0, -63.5, 0.5, -0.5, 2.5, -2.5, 1.49, 0.0] + [0.0] * 8 + [3.0, -1.5])
    r = oracle.encode_rows(INT8, v)
    assert r.scales[0, 0] == np.float32(1.0)
    assert list(r.values[0, :8]) == [127, -64, 1, -1, 3, -3, 1, 0]
    # second (short) block: absmax 3 -> scale float32(3/127)
    s = np.float32(3.0 / 127)
    assert r.scales[0, 1] == s
    assert list(r.values[0, 16:]) == [int(math.copysign(math.floor(abs(x / float(s)) + 0.5), x)) for x in (3.0, -1.5)]
    # an all-zero block has scale 0 and codes 0
    z = oracle.encode_rows(INT8, np.zeros(16))
    assert z.scales[0, 0] == 0 and not z.values.any()


def test_int8_codes_match_independent_numpy():
    rng = np.random.default_rng(2)
    w = rng.normal(0, 0.02, size=(33, 75))
    r = oracle.encode_rows(INT8, w)
    blocks = (75 + 15) // 16
    pad = np.zeros((33, blocks * 16))
    pad[:, :75] = np.abs(w)
    scale32 = (pad.reshape(33, blocks, 16).max(axis=2) / 127).astype(np.float32)
    assert np.array_equal(scale32, r.scales)
    s = np.repeat(scale32.astype(np.float64), 16, axis=1)[:, :75]
    q = w / s
    rounded = np.sign(q) * np.floor(np.abs(q) + 0.5)
    assert np.array_equal(np.clip(rounded, -127, 127).astype(np.int8), r.values)


def test_fp4_halfway_points_round_to_smaller_magnitude():
    # lowprecision.go:88-96: code = number of halfway points strictly below |v|/s
    v = np.zeros(16)
    v[0] = 6.0  # scale = 1 exactly
    v[1:8] = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]
    v[8:15] = np.nextafter(v[1:8], 10)
    v[15] = -0.0
    r = oracle.encode_rows(FP4, v)
    assert r.scales[0, 0] == np.float32(1.0)
    codes = [(r.values[0, i // 2] >> (4 * (i % 2))) & 15 for i in range(16)]
    assert codes[0] == 7
    assert codes[1:8] == [0, 1, 2, 3, 4, 5, 6]
    assert codes[8:15] == [1, 2, 3, 4, 5, 6, 7]
    assert codes[15] == 0  # -0 encodes as +0
    n = oracle.encode_rows(FP4, -v)
    ncodes = [(n.values[0, i // 2] >> (4 * (i % 2))) & 15 for i in range(16)]
    assert ncodes[0] == 15 and ncodes[8] == 9 and ncodes[1] == 8  # sign bit even on magnitude 0


def test_fp4_codes_match_independent_numpy():
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.02, size=(21, 53))
    r = oracle.encode_rows(FP4, w)
    blocks = (53 + 15) // 16
    pad = np.zeros((21, blocks * 16))
    pad[:, :53] = np.abs(w)
    scale32 = (pad.reshape(21, blocks, 16).max(axis=2) / 6).astype(np.float32)
    assert np.array_equal(scale32, r.scales)
    s = np.repeat(scale32.astype(np.float64), 16, axis=1)[:, :53]
    m = np.abs(w) / s
    halfway = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])
    mag = (m[..., None] > halfway).sum(axis=-1)
    codes = mag | np.where(w < 0, 8, 0)
    packed = np.zeros((21, 27), np.uint8)
    for i in range(53):
        packed[:, i // 2] |= (codes[:, i] << (4 * (i % 2))).astype(np.uint8)
    assert np.array_equal(packed, r.values)


def test_float32_rows_round_to_nearest():
    rng = np.random.default_rng(4)
    w = rng.normal(size=(3, 17))
    assert np.array_equal(oracle.encode_rows(FLOAT32, w).values, w.astype(np.float32))


# ---------------------------------------------------------------- decode / DotRow

def numpy_decode(r):
    if r.precision == FLOAT64:
        return r.values.astype(np.float64)
    if r.precision == FLOAT32:
        return r.values.astype(np.float64)
    s = np.repeat(r.scales.astype(np.float64), 16, axis=1)[:, :r.width]
    if r.precision == INT8:
        return r.values.astype(np.float64) * s
    lo = r.values & 15
    hi = r.values >> 4
    codes = np.stack([lo, hi], axis=-1).reshape(r.rows, -1)[:, :r.width]
    table = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6])
    mag = table[codes & 7] * s
    return np.where(codes & 8, -mag, mag)


@pytest.mark.parametrize("p", PRECISIONS)
def test_decode_matches_numpy(p):
    rng = np.random.default_rng(5)
    w = rng.uniform(-3, 3, size=(7, 41))
    r = oracle.encode_rows(p, w)
    assert np.array_equal(oracle.decode_rows(r), numpy_decode(r))


@pytest.mark.parametrize("p", PRECISIONS)
def test_dot_row_matches_reading_the_row(p):
    # lowprecision_test.go:82-103
    rng = np.random.default_rng(6)
    r = oracle.encode_rows(p, rng.uniform(-3, 3, size=(4, 37)))
    v = rng.uniform(-1, 1, size=37)
    dec = oracle.decode_rows(r)
    for row in range(4):
        want = float(np.dot(dec[row], v))
        assert abs(oracle.dot_row(r, row, v) - want) <= 1e-9


def test_dot_row_blocks_are_scaled_once():
    # Int8 DotRow = sum_b (sum_{i in b} x_i q_i) * s_b, sequential; with
    # integer-valued x every partial sum is exact, so the result is exact.
    rng = np.random.default_rng(7)
    r = oracle.encode_rows(INT8, rng.normal(size=(1, 40)))
    x = rng.integers(-5, 6, size=40).astype(np.float64)
    q = r.values[0].astype(np.int64)
    expected = 0.0
    for b in range(3):
        bs = int(np.dot(q[16 * b:16 * b + 16], x[16 * b:16 * b + 16].astype(np.int64)))
        expected += bs * float(r.scales[0, b])
    assert oracle.dot_row(r, 0, x) == expected


# ---------------------------------------------------------------- scalar math

def test_exp_and_log1p_within_one_ulp_of_libm():
    rng = np.random.default_rng(8)
    x = np.concatenate([rng.uniform(-30, 30, 200000), rng.uniform(-1e-6, 1e-6, 20000),
                        rng.uniform(-700, 700, 20000), [0.0, 1.0, -1.0, 0.5 * math.log(2), math.log(2)]])
    ours = oracle.map_fn("exp", x)
    libm = np.array([math.exp(v) for v in x])
    d = ulp_diff(ours, libm)
    # the fdlibm exp method is faithful (< 1 ulp), not correctly rounded:
    # about 9-10% of results sit one ulp from glibc's correctly rounded exp
    assert d.max() <= 1
    assert (d == 0).mean() > 0.85
    y = np.concatenate([np.exp(rng.uniform(-25, 25, 200000)), rng.uniform(-0.29, 0.41, 50000),
                        rng.uniform(-0.999, 1e9, 20000), [1e-30, 2.0**-30, 1.0, 3.0]])
    ours = oracle.map_fn("log1p", y)
    libm = np.array([math.log1p(v) for v in y])
    d = ulp_diff(ours, libm)
    assert d.max() <= 1
    assert (d == 0).mean() > 0.99


def test_softplus_branches_and_affinity():
    assert oracle.map_fn("softplus", np.array([25.0]))[0] == 25.0
    assert oracle.map_fn("softplus", np.array([-25.0]))[0] == oracle.map_fn("exp", np.array([-25.0]))[0]
    x = np.linspace(-19.5, 19.5, 1001)
    sp = oracle.map_fn("softplus", x)
    assert np.allclose(sp, np.log1p(np.exp(x)), rtol=2e-16 * 4, atol=0)
    a = oracle.map_fn("affinity", x)
    assert np.array_equal(a, np.sqrt(sp))
    assert np.all(np.diff(a) > 0)  # strictly increasing on a fine grid


def test_silu_closed_form():
    x = np.linspace(-30, 30, 2001)
    assert np.allclose(oracle.map_fn("silu", x), x / (1 + np.exp(-x)), rtol=1e-15, atol=1e-300)


# ---------------------------------------------------------------- routing

def numpy_route(logits, k, balance):
    a = np.sqrt(np.where(logits > 20, logits, np.where(logits < -20, np.exp(logits), np.log1p(np.exp(logits)))))
    score = a + balance
    chosen = np.sort(np.argsort(-score, axis=1, kind="stable")[:, :k], axis=1)
    ca = np.take_along_axis(a, chosen, axis=1)
    total = np.zeros(len(a))
    for i in range(k):
        total = total + ca[:, i]
    return chosen, ca / total[:, None], a


def test_route_matches_numpy_stable_sort():
    rng = np.random.default_rng(9)
    for E, k in [(8, 2), (16, 2), (64, 6), (128, 8), (5, 5)]:
        logits = rng.normal(0, 1.0, size=(300, E))
        bal = rng.normal(0, 0.1, size=E)
        r = oracle.route_from_logits(logits, k, bal)
        c, g, a = numpy_route(logits, k, bal)
        assert np.array_equal(r.chosen, c)
        assert np.allclose(r.gates, g, rtol=1e-15, atol=0)
        assert np.max(np.abs(r.affinities - a) / a) < 3e-16


def test_route_ties_keep_lower_index():
    logits = np.array([[1.0, 2.0, 2.0, 0.0, 2.0],
                       [0.5, 0.5, 0.5, 0.5, 0.5],
                       [3.0, -1.0, 3.0, 3.0, -1.0]])
    r = oracle.route_from_logits(logits, 2)
    assert r.chosen.tolist() == [[1, 2], [0, 1], [0, 2]]
    r1 = oracle.route_from_logits(logits, 1)
    assert r1.chosen.tolist() == [[1], [0], [0]]
    assert np.all(r1.gates == 1.0)  # k = 1: every gate is exactly 1


def test_route_balance_bias_changes_choice_not_gates():
    logits = np.array([[0.0, 1.0, 2.0, 3.0]])
    r = oracle.route_from_logits(logits, 2, np.array([100.0, 0, 0, 0]))
    assert r.chosen.tolist() == [[0, 3]]
    a = r.affinities[0]
    assert r.gates[0].tolist() == [a[0] / (a[0] + a[3]), a[3] / (a[0] + a[3])]


def insertion_order(s):
    """One insertion sort over the whole row with the reference's less
    function (score[i] > score[j]): what the restatement used before it
    followed sort.SliceStable's blocks and merges."""
    c = list(range(len(s)))
    for i in range(1, len(c)):
        j = i
        while j > 0 and s[c[j]] > s[c[j - 1]]:
            c[j], c[j - 1] = c[j - 1], c[j]
            j -= 1
    return c


def test_go_stable_order_is_a_stable_sort_for_ordered_scores():
    """sort.SliceStable (mixtureofexperts.go:106) on totally ordered scores,
    many ties, across one block of 20, several, and ragged last blocks: the
    order is numpy's stable argsort of -score."""
    rng = np.random.default_rng(31)
    for n in list(range(1, 45)) + [63, 64, 65, 100, 127, 128, 160, 255, 256]:
        for _ in range(8):
            s = rng.integers(0, 6, n).astype(np.float64) * rng.choice([1.0, -0.5])
            s[rng.random(n) < 0.1] = -np.inf
            assert oracle.go_stable_order(s).tolist() == np.argsort(-s, kind="stable").tolist(), (n, s)


def test_go_stable_order_with_nan_inside_one_block():
    """Up to 20 scores the sort is one insertion sort: a NaN compares neither
    greater nor less than anything, so nothing moves past it; each run
    between NaNs is stably sorted on its own and the NaNs stay in place."""
    rng = np.random.default_rng(32)
    for n in range(1, 21):
        for _ in range(30):
            s = rng.integers(0, 5, n).astype(np.float64)
            s[rng.random(n) < 0.25] = np.nan
            want, start = [], 0
            for i in list(np.nonzero(np.isnan(s))[0]) + [n]:
                seg = np.arange(start, i)
                want += seg[np.argsort(-s[seg], kind="stable")].tolist()
                if i < n:
                    want.append(int(i))
                start = i + 1
            assert oracle.go_stable_order(s).tolist() == want
    assert oracle.go_stable_order(np.full(77, np.nan)).tolist() == list(range(77))


def test_go_stable_order_merge_traced_by_hand():
    """22 scores: a sorted block 20, 19, ..., 1 and a block [NaN, 100].  The
    insertion sort leaves the second block as it is (100 does not pass the
    NaN); SymMerge(0, 20, 22) splits at mid 11, finds start 11 (NaN is never
    less), recurses to (11, 20, 22), (16, 20, 22) and (19, 20, 22), whose
    one-element case binary-searches [20, 22) for the first score not above
    1 -- 100 is above it, so i = 22 -- and moves element 19 to the end:
    0..18, then the NaN (20), then 100 (21), then element 19.  One insertion
    sort over all 22 stops at the NaN too but moves nothing else."""
    s = np.concatenate([np.arange(20, 0, -1).astype(np.float64), [np.nan, 100.0]])
    assert oracle.go_stable_order(s).tolist() == list(range(19)) + [20, 21, 19]
    assert insertion_order(s) == list(range(22))
    # through the routing: k = 1 takes expert 0 (score 20), not expert 21
    # (score 100)
    logits = np.where(np.isnan(s), np.nan, 0.0)[None, :]
    r = oracle.route_from_logits(logits, 1, np.where(np.isnan(s), 0.0, s))
    assert r.chosen.tolist() == [[0]]


def test_route_with_some_nan_scores_follows_the_reference_sort():
    """Rows with a few NaN scores: the chosen experts are the first k of
    sort.SliceStable's order, sorted ascending (mixtureofexperts.go:98-112),
    and for rows past one block of 20 that order differs from one insertion
    sort's in some rows (so the block and merge steps are what decide)."""
    rng = np.random.default_rng(33)
    differs = 0
    for E, k in [(8, 2), (21, 3), (32, 4), (64, 6), (128, 8), (256, 8)]:
        logits = rng.normal(0, 1.0, size=(40, E))
        for t in range(40):
            logits[t, rng.choice(E, size=1 + t % 5, replace=False)] = np.nan
        bal = rng.normal(0, 0.1, size=E)
        r = oracle.route_from_logits(logits, k, bal)
        score = r.affinities + bal
        for t in range(40):
            order = oracle.go_stable_order(score[t]).tolist()
            assert r.chosen[t].tolist() == sorted(order[:k])
            differs += sorted(insertion_order(score[t])[:k]) != sorted(order[:k])
    assert differs > 0


def test_hash_route_closed_form():
    ids = np.array([0, 1, 2, 42, 9, 42, 2**40 + 7, 123456789], np.int64)
    for E, k in [(8, 2), (6, 3), (128, 8)]:
        r = oracle.hash_route(ids, E, k)
        for t, i in enumerate(ids):
            first = ((int(i) * 2654435761 + 12345) % 2**64) % E
            assert r.chosen[t].tolist() == [(first + j) % E for j in range(k)]
        assert np.all(r.gates == 1.0 / k)
    with pytest.raises(ValueError):
        oracle.hash_route(np.array([3, -1]), 8, 2)


def test_dispatch_is_stable_by_expert():
    rng = np.random.default_rng(10)
    E, k, T = 16, 3, 200
    chosen = np.stack([np.sort(rng.choice(E, k, replace=False)) for _ in range(T)]).astype(np.int32)
    d = oracle.dispatch(chosen, E)
    flat_e = chosen.reshape(-1)
    flat_t = np.repeat(np.arange(T), k)
    order = np.argsort(flat_e, kind="stable")
    assert np.array_equal(d.rows, flat_t[order])
    assert np.array_equal(d.load, np.bincount(flat_e, minlength=E))
    assert d.offsets[0] == 0 and np.array_equal(np.diff(d.offsets), d.load)


# ---------------------------------------------------------------- layers / MoE

def silu(x):
    return x / (1 + np.exp(-x))


def numpy_expert(e, x):
    def lay(l, v):
        pre = v @ numpy_decode(l.weights).T + l.biases
        if l.activation == 1:
            return silu(pre)
        if l.activation == 2:
            return silu(np.minimum(pre, l.clamp_limit))
        if l.activation == 3:
            return np.clip(pre, -l.clamp_limit, l.clamp_limit)
        return pre
    return lay(e.down, lay(e.gate, x) * lay(e.up, x))


def numpy_moe(m, x, token_ids=None):
    T = x.shape[0]
    if m.use_hash_routing:
        r = oracle.hash_route(token_ids, len(m.routed), m.experts_per_token)
        chosen, gates = r.chosen, r.gates
    else:
        logits = x @ numpy_decode(m.router.weights).T + m.router.biases
        chosen, gates, _ = numpy_route(logits, m.experts_per_token, m.balance_biases)
    out = np.zeros((T, m.vector_size))
    for s in m.shared:
        out = out + numpy_expert(s, x)
    for t in range(T):
        for i, e in enumerate(chosen[t]):
            out[t] += gates[t, i] * numpy_expert(m.routed[e], x[t:t + 1])[0]
    return out, chosen, gates


@pytest.mark.parametrize("p", PRECISIONS)
@pytest.mark.parametrize("clamp", [0.0, 0.5])
def test_layer_and_expert_match_numpy(p, clamp):
    m = make_moe(oracle.encode_rows, d=20, h=36, E=3, k=1, precision=p, seed=11, std=0.3, bias_std=0.1, clamp=clamp)
    x = np.random.default_rng(12).normal(size=(6, 20))
    e = m.routed[0]
    got = oracle.layer_forward(e.gate, x)
    want = x @ numpy_decode(e.gate.weights).T + e.gate.biases
    want = silu(np.minimum(want, clamp)) if clamp else silu(want)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-14)
    for threads in (1, 4):
        y = oracle.moe_forward_routed(m, x, np.zeros((6, 1), np.int32), np.ones((6, 1)), threads).outputs
        assert np.allclose(y, numpy_expert(e, x), rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("case", [
    dict(d=4, h=6, E=4, k=2, S=0), dict(d=4, h=6, E=4, k=2, S=1), dict(d=4, h=6, E=5, k=1, S=1),
    dict(d=4, h=6, E=4, k=2, S=1, clamp=0.5), dict(d=4, h=6, E=4, k=2, S=1, use_hash=True),
    dict(d=37, h=50, E=8, k=3, S=1, precision=FP4), dict(d=32, h=48, E=6, k=2, S=2, precision=FLOAT32),
    dict(d=48, h=40, E=7, k=4, S=0, precision=INT8, router_precision=INT8),
])
def test_moe_matches_numpy_brute_force(case):
    case = dict(case)
    p = case.pop("precision", INT8)
    m = make_moe(oracle.encode_rows, precision=p, seed=13, std=0.3, bias_std=0.05, **case)
    x = np.random.default_rng(14).uniform(-1, 1, size=(9, m.vector_size))
    ids = np.array([3, 7, 1, 12, 5, 0, 2, 99, 7])
    r = oracle.moe_forward(m, x, ids if m.use_hash_routing else None)
    want, chosen, gates = numpy_moe(m, x, ids)
    assert np.array_equal(r.chosen, chosen)
    assert np.allclose(r.gates, gates, rtol=1e-14, atol=0)
    assert np.allclose(r.outputs, want, rtol=1e-11, atol=1e-13)
    assert np.array_equal(r.load, np.bincount(chosen.reshape(-1), minlength=len(m.routed)))


def test_each_token_uses_experts_per_token():
    # mixtureofexperts_test.go:37-68
    for use_hash in (False, True):
        m = make_moe(oracle.encode_rows, d=4, h=6, E=6, k=3, S=1, seed=15, std=0.5, use_hash=use_hash)
        ids = np.arange(8)
        r = oracle.moe_forward(m, np.random.default_rng(16).uniform(-1, 1, (8, 4)), ids)
        for t in range(8):
            assert len(set(r.chosen[t].tolist())) == 3
            assert abs(r.gates[t].sum() - 1) <= 1e-12
        assert r.load.sum() == 24


def test_hash_routing_depends_only_on_token_id():
    # mixtureofexperts_test.go:70-81
    m = make_moe(oracle.encode_rows, d=4, h=6, E=8, k=2, seed=17, use_hash=True)
    rng = np.random.default_rng(18)
    a = oracle.moe_forward(m, rng.uniform(-1, 1, (3, 4)), [42, 9, 42])
    b = oracle.moe_forward(m, rng.uniform(-1, 1, (1, 4)), [42])
    assert a.chosen[0].tolist() == a.chosen[2].tolist() == b.chosen[0].tolist()
    with pytest.raises(ValueError):
        oracle.moe_forward(m, rng.uniform(-1, 1, (2, 4)), [1, -3])


@pytest.mark.parametrize("use_hash", [False, True])
def test_one_row_matches_many_rows(use_hash):
    # mixtureofexperts_test.go:83-100 (1e-12)
    m = make_moe(oracle.encode_rows, d=4, h=6, E=4, k=2, S=1, seed=19, std=0.5, use_hash=use_hash)
    ids = np.array([4, 8, 15, 16])
    x = np.random.default_rng(20).uniform(-1, 1, (4, 4))
    allrows = oracle.moe_forward(m, x, ids).outputs
    for t in range(4):
        one = oracle.moe_forward(m, x[t:t + 1], ids[t:t + 1]).outputs
        assert np.max(np.abs(one[0] - allrows[t])) <= 1e-12


def test_balance_biases_do_not_change_outputs_when_every_expert_is_chosen():
    # mixtureofexperts_test.go:149-160
    m = make_moe(oracle.encode_rows, d=4, h=6, E=3, k=3, seed=21, std=0.5)
    x = np.random.default_rng(22).uniform(-1, 1, (2, 4))
    before = oracle.moe_forward(m, x).outputs
    m.balance_biases = np.array([0.0, 100.0, 0.0])
    after = oracle.moe_forward(m, x).outputs
    assert np.max(np.abs(before - after)) <= 1e-12


def test_threads_never_change_results():
    m = make_moe(oracle.encode_rows, d=96, h=160, E=8, k=2, S=1, seed=23, precision=FP4)
    x = np.random.default_rng(24).normal(size=(70, 96))
    a = oracle.moe_forward(m, x, threads=1).outputs
    b = oracle.moe_forward(m, x, threads=7).outputs
    assert np.array_equal(a, b)


# ---------------------------------------------------------------- RMSNorm and stacks

def test_rmsnorm_closed_form_and_unit_rms():
    rng = np.random.default_rng(25)
    x = rng.normal(size=(5, 64)) * 3
    y = oracle.rmsnorm(x, np.ones(64))
    want = x / np.sqrt((x * x).mean(axis=1, keepdims=True) + 1e-6)
    assert np.allclose(y, want, rtol=1e-14)
    assert np.allclose(np.sqrt((y * y).mean(axis=1)), 1.0, atol=1e-6)


def test_stack_matches_layer_by_layer():
    layers = [make_moe(oracle.encode_rows, d=32, h=24, E=6, k=2, S=1, seed=30 + i, precision=FP4) for i in range(3)]
    norms = [np.ones(32), np.linspace(0.5, 1.5, 32), np.ones(32)]
    x0 = np.random.default_rng(26).normal(size=(7, 32))
    x, chosen = oracle.stack_forward(layers, norms, x0)
    ref = x0.copy()
    gates_all = []
    for l, m in enumerate(layers):
        r = oracle.moe_forward(m, oracle.rmsnorm(ref, norms[l]))
        assert np.array_equal(r.chosen, chosen[l])
        gates_all.append(r.gates)
        ref = ref + r.outputs
    assert np.array_equal(x, ref)
    y = oracle.stack_forward_routed(layers, norms, x0, chosen, np.stack(gates_all))
    assert np.array_equal(y, ref)
