"""The host-API forward stages the rows as fp32 (the host rounds the float64
rows, as the kernels' first step would, and widens the fp32 outputs).  Every
call must equal the device-API forward of the same rows bit for bit, whatever
changed in between: new rows, another token count, new balance biases,
re-uploaded expert weights, per-kernel timing."""
import numpy as np
import pytest

import gotransformers_amd as gt
from tests.moe_fixtures import INT8, make_moe
from tests.test_gpu_parity import say

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ctx():
    c = gt.Context(0)
    yield c
    c.close()


def device_forward(m, x, path):
    """forward_device on the fp32-rounded rows: outputs as float64, routing."""
    T, d = x.shape
    xa = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    ya = torch.empty(T, d, device="cuda")
    m.forward_device(T, xa.data_ptr(), ya.data_ptr(), path=path)
    torch.cuda.synchronize()
    return ya.cpu().numpy().astype(np.float64), m.last_routing()


@pytest.mark.parametrize("path", [gt.PATH_FP32, gt.PATH_BF16])
def test_host_forward_replays_equal_device_forward(ctx, path):
    d = 256
    spec = make_moe(gt.encode_rows, d=d, h=512, E=8, k=2, S=1, precision=INT8, seed=31)
    other = make_moe(gt.encode_rows, d=d, h=512, E=8, k=2, S=1, precision=INT8, seed=32)
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    rng = np.random.default_rng(33)
    try:
        plan = [(1, None), (5, None), (1, None), (64, "balance"), (5, None), (65, None), (1, "weights"), (64, None),
                (5, "timing"), (1, None)]
        for i, (T, change) in enumerate(plan):
            say(f"host forward call {i}: T={T} path={path} change={change}")
            if change == "balance":
                m.balance_biases = rng.standard_normal(8) * 0.5
            elif change == "weights":
                e = other.routed[3]
                for which, lay in (("gate", e.gate), ("up", e.up), ("down", e.down)):
                    m.upload("routed", 3, which, lay.weights, lay.biases)
            timing = change == "timing"
            if timing:
                ctx.timing(True)
            x = rng.standard_normal((T, d))
            try:
                y = m.forward(x, path=path)
                r = m.last_routing()
            finally:
                if timing:
                    ctx.timing(False)
            y_dev, r_dev = device_forward(m, x, path)
            assert np.array_equal(y, y_dev), f"call {i}: outputs differ"
            assert np.array_equal(r.chosen, r_dev.chosen), f"call {i}: choices differ"
            assert np.array_equal(r.gates.view(np.int64), r_dev.gates.view(np.int64)), f"call {i}: gates differ"
            assert np.array_equal(r.load, r_dev.load) and np.array_equal(r.offsets, r_dev.offsets)
    finally:
        m.destroy()
