"""gtmoe_forward_device_noalloc, the forward that allocates nothing, through
the C ABI: its outputs equal gtmoe_forward_device's on the same layer and
inputs bit for bit (same kernels; only where the intermediates live
differs), call after call, with a smaller input second and layers of other
shapes in between sharing the one scratch area; sizes beyond the area are
refused.  The layers' outputs are checked against the oracle as in the other
GPU tests."""
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


def both(m, x, path):
    """(forward_device, forward_device_noalloc) outputs of the same rows."""
    T, d = x.shape
    xd = dev(x)
    ya = torch.full((T, d), float("nan"), device="cuda")
    yb = torch.full((T, d), float("nan"), device="cuda")
    m.forward_device(T, xd.data_ptr(), ya.data_ptr(), path=path)
    torch.cuda.synchronize()
    r = m.last_routing()
    m.forward_device_noalloc(T, xd.data_ptr(), yb.data_ptr(), path=path)
    torch.cuda.synchronize()
    return ya.cpu().numpy(), yb.cpu().numpy(), r


@pytest.mark.parametrize("path", [gt.PATH_FP32, gt.PATH_BF16])
def test_noalloc_matches_forward_device(ctx, path):
    say(f"forward without allocation, path {path}")
    # C2-shaped (d = 1024, k = 2, folded combine on the fp32 path) and a
    # layer whose d and h are not multiples of 64 (padding columns that the
    # scratch area must hold as zeros)
    a_spec = make_moe(gt.encode_rows, d=1024, h=2048, E=16, k=2, S=0, precision=INT8, seed=70)
    b_spec = make_moe(gt.encode_rows, d=100, h=90, E=6, k=3, S=1, precision=FP4, seed=71, std=0.1, bias_std=0.02)
    # many tokens over 64 experts: routed by the staged router (which, on the
    # bf16 path, writes the bf16 rows into the area) and dispatched per chunk
    c_spec = make_moe(gt.encode_rows, d=256, h=64, E=64, k=2, S=1, precision=FP4, seed=74, std=0.2, bias_std=0.05)
    rng = np.random.default_rng(72)
    a = gt.MixtureOfExperts.from_spec(ctx, a_spec)
    b = gt.MixtureOfExperts.from_spec(ctx, b_spec)
    c = gt.MixtureOfExperts.from_spec(ctx, c_spec)
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
