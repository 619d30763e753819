"""gtmoe_forward_device_noalloc, the forward that allocates nothing, through
the C ABI: its outputs equal gtmoe_forward_device's on the same layer and
inputs bit for bit (same kernels; only where the intermediates live
differs), call after call, with a smaller input second and layers of other
shapes in between sharing the one scratch area; sizes beyond the area are
refused.  That it allocates nothing is checked two ways: the library's own
count of device allocations does not move over the calls, and the call
records into a HIP graph under global capture mode (where an allocation in
any thread would break the capture) whose replays equal the eager forward.  The layers' outputs are checked
against the oracle as in the other GPU tests."""
import numpy as np
import pytest

import gotransformers_amd as gt
import oracle
from tests.moe_fixtures import FP4, INT8, make_moe
from tests.test_gpu_parity import rel_err, say

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ctx():
    c = gt.Context(0)
    yield c
    c.close()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def both(m, x, path, ids=None):
    """(forward_device, forward_device_noalloc) outputs of the same rows; the
    second call is checked to allocate and free nothing on the device."""
    T, d = x.shape
    xd = dev(x)
    idp = None
    if ids is not None:
        idd = torch.from_numpy(np.ascontiguousarray(ids, np.int64)).cuda()
        idp = idd.data_ptr()
    ya = torch.full((T, d), float("nan"), device="cuda")
    yb = torch.full((T, d), float("nan"), device="cuda")
    m.forward_device(T, xd.data_ptr(), ya.data_ptr(), token_ids_ptr=idp, path=path)
    torch.cuda.synchronize()
    r = m.last_routing()
    before = gt.device_allocations()
    m.forward_device_noalloc(T, xd.data_ptr(), yb.data_ptr(), token_ids_ptr=idp, path=path)
    torch.cuda.synchronize()
    assert gt.device_allocations() == before
    return ya.cpu().numpy(), yb.cpu().numpy(), r


@pytest.mark.parametrize("path", [gt.PATH_FP32, gt.PATH_BF16])
def test_noalloc_matches_forward_device(ctx, path):
    say(f"forward without allocation, path {path}")
    # C2-shaped (d = 1024, k = 2, folded combine on the fp32 path) and a
    # layer whose d and h are not multiples of 64 (padding columns that the
    # scratch area must hold as zeros)
    a_spec = make_moe(gt.encode_rows, d=1024, h=2048, E=16, k=2, S=0, precision=INT8, seed=70)
    b_spec = make_moe(gt.encode_rows, d=100, h=90, E=6, k=3, S=1, precision=FP4, seed=71, std=0.1, bias_std=0.02)
    # hash routing: the token ids are read where the caller keeps them
    h_spec = make_moe(gt.encode_rows, d=128, h=96, E=8, k=2, S=1, precision=INT8, seed=75, use_hash=True)
    # many tokens over 64 experts: routed by the staged router (which, on the
    # bf16 path, writes the bf16 rows into the area) and dispatched per chunk
    c_spec = make_moe(gt.encode_rows, d=256, h=64, E=64, k=2, S=1, precision=FP4, seed=74, std=0.2, bias_std=0.05)
    rng = np.random.default_rng(72)
    a = gt.MixtureOfExperts.from_spec(ctx, a_spec)
    b = gt.MixtureOfExperts.from_spec(ctx, b_spec)
    c = gt.MixtureOfExperts.from_spec(ctx, c_spec)
    hl = gt.MixtureOfExperts.from_spec(ctx, h_spec)
    tol = 1e-4 if path == gt.PATH_FP32 else 2e-2
    try:
        # two calls in a row on one layer, the second smaller, then the other
        # layer, then the first again
        for m, spec, T in ((a, a_spec, 48), (a, a_spec, 5), (b, b_spec, 40), (a, a_spec, 17), (b, b_spec, 3)):
            x = rng.standard_normal((T, spec.vector_size))
            ya, yb, r = both(m, x, path)
            assert np.all(np.isfinite(ya))
            assert np.array_equal(ya, yb), (spec.vector_size, T)
            ref = oracle.moe_forward_routed(spec, x.astype(np.float32).astype(np.float64), r.chosen, r.gates)
            e = rel_err(yb, ref.outputs)
            say(f"[d={spec.vector_size} T={T}] equal to forward_device; max rel err vs oracle {e:.2e}")
            assert e <= tol
        for T in (33, 6):
            x = rng.standard_normal((T, 128))
            ids = rng.integers(0, 2**40, T)
            ya, yb, r = both(hl, x, path, ids)
            assert np.array_equal(ya, yb), ("hash", T)
            ref = oracle.moe_forward(h_spec, x.astype(np.float32).astype(np.float64), ids)
            assert np.array_equal(r.chosen, ref.chosen)
            e = rel_err(yb, ref.outputs)
            say(f"[hash routing T={T}] equal to forward_device; max rel err vs oracle {e:.2e}")
            assert e <= tol
        for T in (4100, 1500):
            x = rng.standard_normal((T, 256))
            ya, yb, r = both(c, x, path)
            assert np.all(np.isfinite(ya))
            assert np.array_equal(ya, yb), (256, T)
            sample = np.sort(rng.choice(T, 24, replace=False))
            ref = oracle.moe_forward_routed(c_spec, x[sample].astype(np.float32).astype(np.float64),
                                            r.chosen[sample], r.gates[sample])
            e = rel_err(yb[sample], ref.outputs)
            say(f"[d=256 E=64 T={T}] equal to forward_device; max rel err vs oracle on a sample {e:.2e}")
            assert e <= tol
        # the call keeps no routing state on the layer
        with pytest.raises(gt.GtmoeError) as info:
            b.last_routing()
        assert info.value.code == gt.ERR_NOT_READY
    finally:
        a.destroy()
        b.destroy()
        c.destroy()
        hl.destroy()


@pytest.mark.parametrize("path", [gt.PATH_FP32, gt.PATH_BF16])
@pytest.mark.parametrize("use_hash", [False, True])
def test_noalloc_records_into_a_graph_under_global_capture(ctx, path, use_hash):
    """The forward without allocation recorded on a side stream into a HIP
    graph with global capture mode, the mode in which a device allocation or
    free made anywhere during the capture invalidates it; the replays, with
    new rows filled in and eager forwards between them, equal
    gtmoe_forward_device on the same rows bit for bit, and the library's
    allocation count does not move."""
    say(f"forward without allocation under graph capture, path {path}, hash routing {use_hash}")
    spec = make_moe(gt.encode_rows, d=256, h=192, E=12, k=3, S=1, precision=FP4, seed=76, std=0.1, bias_std=0.02,
                    use_hash=use_hash)
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    rng = np.random.default_rng(77)
    T = 40
    x = torch.zeros(T, 256, device="cuda")
    y = torch.zeros(T, 256, device="cuda")
    ids = torch.zeros(T, dtype=torch.int64, device="cuda")
    idp = ids.data_ptr() if use_hash else None
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # one eager call first, as torch asks
            m.forward_device_noalloc(T, x.data_ptr(), y.data_ptr(), token_ids_ptr=idp, path=path,
                                     stream=side.cuda_stream)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        before = gt.device_allocations()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side, capture_error_mode="global"):
            m.forward_device_noalloc(T, x.data_ptr(), y.data_ptr(), token_ids_ptr=idp, path=path,
                                     stream=side.cuda_stream)
        torch.cuda.synchronize()
        assert gt.device_allocations() == before
        want = torch.empty_like(y)
        for rep in range(4):
            xs = rng.standard_normal((T, 256))
            x.copy_(torch.from_numpy(xs.astype(np.float32)))
            ids.copy_(torch.from_numpy(rng.integers(0, 2**40, T)))
            g.replay()
            torch.cuda.synchronize()
            got = y.clone()
            m.forward_device(T, x.data_ptr(), want.data_ptr(), token_ids_ptr=idp, path=path)  # eager, between
            torch.cuda.synchronize()
            assert torch.equal(got, want), rep
        del g
    finally:
        m.destroy()


def test_noalloc_refuses_sizes_beyond_the_scratch_area(ctx):
    say("forward without allocation: size limit")
    spec = make_moe(gt.encode_rows, d=1024, h=2048, E=16, k=2, S=0, precision=INT8, seed=73)
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        T = 1716  # one token past what the area holds for this shape
        x = torch.zeros(T, 1024, device="cuda")
        y = torch.zeros(T, 1024, device="cuda")
        with pytest.raises(gt.InvalidArgument, match="without allocation has"):
            m.forward_device_noalloc(T, x.data_ptr(), y.data_ptr(), path=gt.PATH_BF16)
        m.forward_device_noalloc(1715, x.data_ptr(), y.data_ptr(), path=gt.PATH_BF16)
        torch.cuda.synchronize()
        assert np.all(y[:1715].cpu().numpy() == 0.0)  # zero rows, zero biases
    finally:
        m.destroy()
