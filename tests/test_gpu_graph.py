"""A whole forward recorded as a HIP graph and replayed: every replay must
equal the eager forward bit for bit (the same kernels on the same buffers),
with the program's own eager work and synchronisations between replays, and
after the inputs are refilled in place.  The eager results are checked
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


@pytest.mark.parametrize("T,path,S,E", [(16, gt.PATH_FP32, 1, 8), (1, gt.PATH_FP32, 1, 8), (64, gt.PATH_BF16, 1, 8),
                                        (16, gt.PATH_FP32, 0, 8), (3, gt.PATH_FP32, 0, 8),
                                        (4100, gt.PATH_BF16, 1, 64)])
def test_graph_forward_replays_equal_eager(ctx, T, path, S, E):
    # S = 0 with top-2: the combine is folded into the down kernel; 4100
    # tokens x 64 experts: the staged router writes the bf16 rows, the
    # dispatch runs per chunk of tokens
    say(f"graph forward T={T} path={path} S={S} E={E}")
    spec = make_moe(gt.encode_rows, d=256, h=512, E=E, k=2, S=S, precision=INT8, seed=21)
    rng = np.random.default_rng(22)
    x0 = rng.standard_normal((T, 256))
    x1 = rng.standard_normal((T, 256))
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        xa, ya = dev(x0), torch.empty(T, 256, device="cuda")
        m.forward_device(T, xa.data_ptr(), ya.data_ptr(), path=path)
        torch.cuda.synchronize()
        eager0 = ya.cpu().numpy().copy()
        r0 = m.last_routing()
        xb, yb = dev(x1), torch.empty(T, 256, device="cuda")
        m.forward_device(T, xb.data_ptr(), yb.data_ptr(), path=path)
        torch.cuda.synchronize()
        eager1 = yb.cpu().numpy().copy()

        xg, yg = dev(x0), torch.empty(T, 256, device="cuda")
        with gt.Graph.capture_forward(m, T, xg.data_ptr(), yg.data_ptr(), path=path) as g:
            for rep in range(3):
                yg.fill_(float("nan"))
                torch.cuda.synchronize()
                g.launch()
                torch.cuda.synchronize()
                assert np.array_equal(yg.cpu().numpy(), eager0), rep
                # eager work of the program between replays
                m.forward_device(T, xb.data_ptr(), yb.data_ptr(), path=path)
                torch.cuda.synchronize()
            g.launch()
            torch.cuda.synchronize()
            r = m.last_routing()
            assert np.array_equal(r.chosen, r0.chosen)
            assert np.array_equal(r.load, r0.load)
            xg.copy_(xb)  # refill the recorded input in place
            torch.cuda.synchronize()
            g.launch()
            torch.cuda.synchronize()
            assert np.array_equal(yg.cpu().numpy(), eager1)
    finally:
        m.destroy()
    sample = np.arange(T) if T <= 256 else np.sort(rng.choice(T, 32, replace=False))
    ref = oracle.moe_forward_routed(spec, x0[sample], r0.chosen[sample], r0.gates[sample])
    tol = 1e-4 if path == gt.PATH_FP32 else 2e-2
    assert rel_err(eager0[sample], ref.outputs) <= tol


# E = 64 at T = 8: the routing splits each token's experts over several
# workgroups (arrival counts that reset themselves, replay after replay) and
# the residual alternates between x and a second buffer; four layers end
# with the last combine reading the second buffer.
@pytest.mark.parametrize("T,path,E,nl", [(8, gt.PATH_FP32, 6, 3), (96, gt.PATH_BF16, 6, 3), (8, gt.PATH_FP32, 64, 4)])
def test_graph_stack_replays_equal_eager(ctx, T, path, E, nl):
    say(f"graph stack T={T} path={path} E={E} layers={nl}")
    d = 128
    specs = [make_moe(gt.encode_rows, d=d, h=192, E=E, k=2, S=1, precision=FP4, seed=30 + i) for i in range(nl)]
    rng = np.random.default_rng(31)
    x0 = rng.standard_normal((T, d))
    layers = [gt.MixtureOfExperts.from_spec(ctx, s) for s in specs]
    try:
        for i, m in enumerate(layers):
            m.set_norm_weights(1.0 + 0.1 * rng.standard_normal(d))
        xe = dev(x0)
        gt.stack_forward_device(layers, T, xe.data_ptr(), path=path)
        torch.cuda.synchronize()
        eager = xe.cpu().numpy().copy()

        xg = dev(x0)
        with gt.Graph.capture_stack(layers, T, xg.data_ptr(), path=path) as g:
            for rep in range(3):
                xg.copy_(dev(x0))  # the stack updates x in place: reset it
                torch.cuda.synchronize()
                g.launch()
                torch.cuda.synchronize()
                assert np.array_equal(xg.cpu().numpy(), eager), rep
                xe.copy_(dev(x0))
                gt.stack_forward_device(layers, T, xe.data_ptr(), path=path)
                torch.cuda.synchronize()
    finally:
        for m in layers:
            m.destroy()
    assert np.all(np.isfinite(eager))


def test_graph_capture_rejects_bad_arguments(ctx):
    spec = make_moe(gt.encode_rows, d=64, h=64, E=4, k=2, S=0, precision=INT8, seed=40)
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        with pytest.raises(gt.InvalidArgument):
            gt.Graph.capture_forward(m, -1, 0, 0)
        with pytest.raises(gt.InvalidArgument):
            gt.Graph.capture_forward(m, 4, 0, 0)  # null buffers
    finally:
        m.destroy()


def test_graph_keeps_its_layers_workspace(ctx):
    """A recorded graph holds pointers into its layer's workspace: while it
    exists a forward that would need a larger workspace, and destroying the
    layer, are refused; after the graph is destroyed both work again."""
    say("graph keeps the workspace it was recorded with")
    d = 64
    spec = make_moe(gt.encode_rows, d=d, h=96, E=4, k=2, S=1, precision=INT8, seed=41)
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    try:
        T = 4
        xg, yg = dev(np.random.default_rng(42).standard_normal((T, d))), torch.empty(T, d, device="cuda")
        g = gt.Graph.capture_forward(m, T, xg.data_ptr(), yg.data_ptr(), path=gt.PATH_FP32)
        big = np.random.default_rng(43).standard_normal((300, d))
        with pytest.raises(gt.InvalidArgument, match="destroy the graphs first"):
            m.forward(big)
        with pytest.raises(gt.InvalidArgument, match="recorded graph"):
            m.destroy()
        assert m.handle
        m.forward(big[:T])  # within the recorded workspace: allowed
        g.launch()
        torch.cuda.synchronize()
        assert np.all(np.isfinite(yg.cpu().numpy()))
        g.destroy()
        y = m.forward(big)
        r = m.last_routing()
    finally:
        m.destroy()
    ref = oracle.moe_forward_routed(spec, big, r.chosen, r.gates)
    assert rel_err(y, ref.outputs) <= 2e-2
