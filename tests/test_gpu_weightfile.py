"""LoadBinary into a layer on the GPU: a mixture-of-experts layer whose
parameters come from a GoTransformers binary weights file must hold exactly
the buffers of the same layer uploaded from memory, so both forwards agree bit
for bit; the forward is then checked against the oracle as in the other GPU
tests.  Refusals follow checkSavedParameterFits (weightfile/weightfile.go:69-87)
and leave a fresh layer without weights."""
import copy
from types import SimpleNamespace

import numpy as np
import pytest

import gotransformers_amd as gt
import oracle
from tests import weightfile_writer as wfw
from tests.moe_fixtures import FLOAT32, FP4, INT8, make_moe
from tests.test_gpu_parity import rel_err, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = gt.Context(0)
    yield c
    c.close()


def new_layer(ctx, spec):
    return gt.MixtureOfExperts(ctx, spec.vector_size, spec.hidden_size, len(spec.shared), len(spec.routed),
                               spec.experts_per_token, spec.precision, spec.clamp_limit, spec.use_hash_routing)


def bf16_round(values):
    return np.array([wfw.bfloat16_bits_to_float64(wfw.float64_to_bfloat16_bits(float(v))) for v in values])


@pytest.mark.parametrize("precision,storage,plain_router,S,hash_routing", [
    (INT8, wfw.STORE_FLOAT64, False, 1, False),
    (FP4, wfw.STORE_FLOAT32, True, 2, False),
    (INT8, wfw.STORE_BFLOAT16, True, 0, False),
    (FP4, wfw.STORE_FLOAT64, False, 1, True),
])
def test_layer_from_file_equals_upload(ctx, tmp_path, precision, storage, plain_router, S, hash_routing):
    say(f"weights file precision={precision} storage={storage} plain_router={plain_router} S={S} hash={hash_routing}")
    d, h, E, k, T = 128, 192, 8, 2, 24
    spec = make_moe(gt.encode_rows, d=d, h=h, E=E, k=k, S=S, precision=precision, seed=50 + precision,
                    bias_std=0.01, use_hash=hash_routing)
    file_spec = copy.deepcopy(spec)
    if plain_router:
        file_spec.router.weights = oracle.decode_rows(spec.router.weights)  # plain float64 values
    params = wfw.moe_parameters(file_spec, "block3.moe")
    params.append(("unrelated.weights", np.ones(5)))  # other parameters of the file are ignored
    path = str(tmp_path / "model.weights")
    wfw.write(path, params, storage)

    # the layer uploaded from memory gets the biases as the file stores them
    mem_spec = copy.deepcopy(spec)
    if storage != wfw.STORE_FLOAT64:
        rnd = (lambda b: np.asarray(b, np.float32).astype(np.float64)) if storage == wfw.STORE_FLOAT32 else bf16_round
        for e in mem_spec.shared + mem_spec.routed:
            for which in ("gate", "up", "down"):
                getattr(e, which).biases = rnd(getattr(e, which).biases)
        mem_spec.router.biases = rnd(mem_spec.router.biases)
        if plain_router:  # plain weights are stored at the storage precision too
            w = oracle.decode_rows(spec.router.weights)
            mem_spec.router.weights = gt.encode_rows(gt.FLOAT64, rnd(w.reshape(-1)).reshape(w.shape))

    rng = np.random.default_rng(7)
    x = rng.standard_normal((T, d))
    ids = rng.integers(0, 50000, T) if hash_routing else None
    a = gt.MixtureOfExperts.from_spec(ctx, mem_spec)
    b = new_layer(ctx, spec)
    try:
        with gt.WeightsFile(path) as wf:
            b.load_weights(wf, "block3.moe")
        for path_flag in (gt.PATH_FP32, gt.PATH_BF16):
            ya = a.forward(x, ids, path=path_flag)
            yb = b.forward(x, ids, path=path_flag)
            assert np.array_equal(ya, yb), path_flag
        ra, rb = a.last_routing(), b.last_routing()
        assert np.array_equal(ra.chosen, rb.chosen)
        yb = b.forward(x, ids, path=gt.PATH_FP32)
        r = b.last_routing()
    finally:
        a.destroy()
        b.destroy()
    ref = oracle.moe_forward_routed(mem_spec, x, r.chosen, r.gates)
    assert rel_err(yb, ref.outputs) <= 1e-4


def test_layer_load_refusals(ctx, tmp_path):
    say("weights file refusals")
    spec = make_moe(gt.encode_rows, d=64, h=64, E=4, k=2, S=1, precision=INT8, seed=60)
    good = wfw.moe_parameters(spec, "moe")

    def expect(params, exc, match, name="moe", layer_spec=spec):
        p = str(tmp_path / "w")
        wfw.write(p, params)
        m = new_layer(ctx, layer_spec)
        try:
            with gt.WeightsFile(p) as wf:
                with pytest.raises(exc, match=match):
                    m.load_weights(wf, name)
            # checked before anything is uploaded: the layer still has no weights
            with pytest.raises(gt.GtmoeError) as info:
                m.forward(np.zeros((1, 64)))
            assert info.value.code == gt.ERR_NOT_READY
        finally:
            m.destroy()

    missing = [(n, v) for n, v in good if not n.startswith("moe.expert4.")]
    expect(missing, gt.InvalidArgument, 'no saved parameter named "moe.expert4.gate.weights"')
    expect(good, gt.InvalidArgument, 'no saved parameter named "other.shared1.gate.weights"', name="other")

    plain = [(n, oracle.decode_rows(v) if n == "moe.expert2.up.weights" else v) for n, v in good]
    expect(plain, gt.InvalidArgument, "is compressed but the file holds it as plain numbers")

    short_bias = [(n, v[:-1] if n == "moe.router.biases" else v) for n, v in good]
    expect(short_bias, gt.InvalidArgument, 'saved parameter "moe.router.biases" has 3 values')

    wrong_shape = [(n, gt.encode_rows(INT8, np.ones((32, 64))) if n == "moe.shared1.down.weights" else v)
                   for n, v in good]
    expect(wrong_shape, gt.InvalidArgument, "is 32x64 compressed values but the parameter it's loading into is 64x64")

    other_precision = [(n, gt.encode_rows(FP4, oracle.decode_rows(v)) if n == "moe.expert1.gate.weights" else v)
                       for n, v in good]
    expect(other_precision, gt.GtmoeError, "precision 3")

    router_count = [(n, np.ones(4 * 63) if n == "moe.router.weights" else v) for n, v in good]
    expect(router_count, gt.InvalidArgument, 'saved parameter "moe.router.weights" has 252 values')

    # a router stored as Int8 rows of another shape (8 x 32, as many values)
    # whose codes and scales sum to the right byte count but do not fit that
    # shape each (252 codes and 17 scales instead of 256 and 16):
    # RowsFromSnapshot's byte sum takes it, decoding it at 8 x 32 would read
    # past the codes, so the load refuses it first
    r = gt.encode_rows(INT8, oracle.decode_rows(spec.router.weights).reshape(8, 32))
    unbalanced = SimpleNamespace(precision=INT8, rows=8, width=32, values=r.values.reshape(-1)[:252].copy(),
                                 scales=np.concatenate([r.scales.reshape(-1), [1.0]]).astype(np.float32))
    router_split = [(n, unbalanced if n == "moe.router.weights" else v) for n, v in good]
    expect(router_split, gt.InvalidArgument, "holds 252 value bytes and 17 scales, 8x32 rows need 256 and 16")


def test_router_rows_of_another_shape(ctx, tmp_path):
    """An uncompressed target takes compressed rows of any shape with as many
    values, expanded by Rows.AllValues (weightfile.go:84-85,102-103)."""
    say("weights file router reshaped")
    spec = make_moe(gt.encode_rows, d=64, h=64, E=4, k=2, S=0, precision=FP4, seed=61, router_precision=FLOAT32)
    router_values = oracle.decode_rows(spec.router.weights)  # 4 x 64
    params = [(n, gt.encode_rows(FLOAT32, router_values.reshape(8, 32)) if n == "moe.router.weights" else v)
              for n, v in wfw.moe_parameters(spec, "moe")]
    p = str(tmp_path / "w")
    wfw.write(p, params)
    x = np.random.default_rng(3).standard_normal((5, 64))
    a = gt.MixtureOfExperts.from_spec(ctx, spec)
    b = new_layer(ctx, spec)
    try:
        with gt.WeightsFile(p) as wf:
            b.load_weights(wf, "moe")
        assert np.array_equal(a.forward(x), b.forward(x))
    finally:
        a.destroy()
        b.destroy()
