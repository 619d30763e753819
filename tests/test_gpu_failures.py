"""Failure paths on a live device: a closed context answers with an error
instead of working (a closed gpu.Device answers on the CPU,
gpu/device.go:729-731, gpu/gpu_test.go:145-154: close twice, then use), and
a failure injected into a forward entry point comes back as its status with
gtmoe_last_error's text, once, leaving the layer usable."""
import ctypes as C

import numpy as np
import pytest

import gotransformers_amd as gt
import oracle
from tests.moe_fixtures import INT8, make_moe
from tests.test_gpu_parity import rel_err, say

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def test_close_twice_and_use_after_close():
    say("closed context")
    lib = gt.library()
    spec = make_moe(gt.encode_rows, d=64, h=96, E=4, k=2, S=1, precision=INT8, seed=80)
    x = np.random.default_rng(81).standard_normal((6, 64))
    ctx = gt.Context(0)
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    y = m.forward(x)
    handle = ctx.handle
    assert lib.gtmoe_close(handle) == gt.OK
    assert lib.gtmoe_close(handle) == gt.OK  # closing twice does nothing
    for call in (lambda: m.forward(x), lambda: m.last_expert_load(), lambda: m.update_balance(0.1),
                 lambda: m.set_norm_weights(np.ones(64))):
        with pytest.raises(gt.InvalidArgument, match="the context is closed"):
            call()
    assert lib.gtmoe_last_error(handle).decode() == "the context is closed"
    h = C.c_void_p()
    desc = gt.LayerDesc(64, 96, 1, 4, 2, INT8, 0, 0, 0.0)
    assert lib.gtmoe_layer_create(handle, C.byref(desc), C.byref(h)) == gt.ERR_INVALID_ARGUMENT
    assert lib.gtmoe_timing_enable(handle, 1) == gt.ERR_INVALID_ARGUMENT
    m.destroy()  # a layer of a closed context is still freed
    ctx.handle = None
    r = oracle.moe_forward(spec, x)
    assert rel_err(y, r.outputs) <= 2e-2  # the forward before the close was sound


def test_context_free_keeps_layers_answering_until_they_are_destroyed():
    """gtmoe_context_free gives up the caller's handle: a layer made on the
    context still answers "the context is closed" (the context lives on while
    a layer or graph refers to it) and is still freed by gtmoe_layer_destroy,
    which then frees the context too."""
    say("context free")
    lib = gt.library()
    spec = make_moe(gt.encode_rows, d=64, h=96, E=4, k=2, S=1, precision=INT8, seed=86)
    x = np.random.default_rng(87).standard_normal((4, 64))
    ctx = gt.Context(0)
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    m.forward(x)
    handle = ctx.handle
    assert lib.gtmoe_context_free(handle) == gt.OK
    with pytest.raises(gt.GtmoeError) as info:
        m.forward(x)
    assert info.value.code == gt.ERR_INVALID_ARGUMENT
    assert lib.gtmoe_last_error(handle).decode() == "the context is closed"
    m.destroy()  # the last reference: the context goes with it
    ctx.handle = None


@pytest.mark.parametrize("entry", ["gtmoe_forward", "gtmoe_forward_device", "gtmoe_stack_forward",
                                   "gtmoe_upload_rows", "gtmoe_last_routing"])
def test_injected_failure_is_reported_once(entry):
    say(f"injected failure in {entry}")
    spec = make_moe(gt.encode_rows, d=64, h=96, E=4, k=2, S=1, precision=INT8, seed=82)
    x = np.random.default_rng(83).standard_normal((5, 64))
    with gt.Context(0) as ctx:
        m = gt.MixtureOfExperts.from_spec(ctx, spec)
        try:
            m.set_norm_weights(np.ones(64))
            want = m.forward(x, path=gt.PATH_FP32)
            xd = torch.from_numpy(x.astype(np.float32)).cuda()
            yd = torch.empty(5, 64, device="cuda")
            calls = {
                "gtmoe_forward": lambda: m.forward(x, path=gt.PATH_FP32),
                "gtmoe_forward_device": lambda: m.forward_device(5, xd.data_ptr(), yd.data_ptr(),
                                                                 path=gt.PATH_FP32),
                "gtmoe_stack_forward": lambda: gt.stack_forward([m], x),
                "gtmoe_upload_rows": lambda: m.upload("routed", 0, "gate", spec.routed[0].gate.weights,
                                                      spec.routed[0].gate.biases),
                "gtmoe_last_routing": lambda: m.last_routing(),
            }
            gt.inject_failure(entry, gt.ERR_DEVICE)
            with pytest.raises(gt.GtmoeError) as info:
                calls[entry]()
            assert info.value.code == gt.ERR_DEVICE
            assert str(info.value).endswith(f"injected failure in {entry}")
            assert gt.library().gtmoe_last_error(ctx.handle).decode() == f"injected failure in {entry}"
            calls[entry]()  # the next call runs
            torch.cuda.synchronize()
            got = m.forward(x, path=gt.PATH_FP32)
        finally:
            m.destroy()
    assert np.array_equal(got, want)


def test_host_forward_waits_for_a_device_forward_on_another_stream():
    """gtmoe_forward right after gtmoe_forward_device on the null stream, with
    other inputs and no synchronisation between: both use the layer's
    workspace, and the host call's own stream does not synchronise with the
    null stream, so the host call first waits for the device call's kernels.
    Each result is checked against the oracle under its own routing."""
    say("host forward after a device forward on the null stream")
    d, T = 1024, 32
    spec = make_moe(gt.encode_rows, d=d, h=2048, E=16, k=2, S=1, precision=INT8, seed=84)
    rng = np.random.default_rng(85)
    xa = rng.standard_normal((T, d))
    xb = rng.standard_normal((T, d))
    xa_d = torch.from_numpy(xa.astype(np.float32)).cuda()
    ya_d = torch.empty(T, d, device="cuda")
    torch.cuda.synchronize()
    with gt.Context(0) as ctx:
        m = gt.MixtureOfExperts.from_spec(ctx, spec)
        try:
            m.forward_device(T, xa_d.data_ptr(), ya_d.data_ptr(), path=gt.PATH_FP32)
            yb = m.forward(xb, path=gt.PATH_FP32)
            rb = m.last_routing()
            torch.cuda.synchronize()
            ya = ya_d.cpu().numpy().astype(np.float64)
        finally:
            m.destroy()
    ref_b = oracle.moe_forward_routed(spec, xb, rb.chosen, rb.gates, threads=8)
    ref_a = oracle.moe_forward(spec, xa.astype(np.float32).astype(np.float64), threads=8)
    eb, ea = rel_err(yb, ref_b.outputs), rel_err(ya, ref_a.outputs)
    say(f"host forward {eb:.2e}, device forward {ea:.2e}")
    assert eb <= 1e-4 and ea <= 1e-4
