"""Failure paths a caller falls back on (the Go side answers on the CPU and
records lastError, gpu/device.go:723-739), checked without a GPU:

* the library cannot be loaded (missing file, a file that is no library):
  the binding raises ImportError naming the path, as the reference's loader
  reports a missing Vulkan library (gpu/library_unix.go:12-29);
* the library loads but no gfx950 device answers: gtmoe_open returns
  GTMOE_ERR_DEVICE with the reason in gtmoe_last_error(NULL);
* a status injected through the test hook gtmoe_test_inject_failure: the
  armed entry point answers that status and the text "injected failure in
  <entry point>" once, on the arming thread only, then runs normally;
* null handles are refused.
The GPU side (a closed context, injected failures on forwards) is in
tests/test_gpu_failures.py."""
import ctypes as C
import threading

import pytest

import gotransformers_amd as gt


@pytest.fixture
def fresh_binding(monkeypatch):
    """The binding with its loaded library forgotten (restored afterwards)."""
    monkeypatch.setattr(gt, "_lib", None)
    return monkeypatch


def test_missing_library_raises_naming_the_path(fresh_binding, tmp_path):
    missing = str(tmp_path / "libgtmoe.so")
    fresh_binding.setattr(gt, "LIB_PATH", missing)
    with pytest.raises(ImportError, match="libgtmoe.so is not built"):
        gt.library()
    with pytest.raises(ImportError):
        gt.Context(0)


def test_file_that_is_no_library_raises(fresh_binding, tmp_path):
    bogus = tmp_path / "libgtmoe.so"
    bogus.write_text("not an ELF shared object\n")
    fresh_binding.setattr(gt, "LIB_PATH", str(bogus))
    with pytest.raises(ImportError, match="cannot load .*libgtmoe.so"):
        gt.library()


def no_device():
    return gt.device_count() == 0


def test_open_without_a_device_reports_why():
    if not no_device():
        pytest.skip("a GPU is present: gtmoe_open succeeds here")
    lib = gt.library()
    h = C.c_void_p()
    code = lib.gtmoe_open(0, C.byref(h))
    assert code == gt.ERR_DEVICE
    assert h.value is None
    assert lib.gtmoe_last_error(None).decode().startswith("no HIP device")
    with pytest.raises(gt.GtmoeError, match="no HIP device") as info:
        gt.Context(0)
    assert info.value.code == gt.ERR_DEVICE


def test_injected_status_on_open_is_reported_once():
    lib = gt.library()
    h = C.c_void_p()
    gt.inject_failure("gtmoe_open", gt.ERR_OUT_OF_MEMORY)
    assert lib.gtmoe_open(0, C.byref(h)) == gt.ERR_OUT_OF_MEMORY
    assert h.value is None
    assert lib.gtmoe_last_error(None).decode() == "injected failure in gtmoe_open"
    # one-shot: the next call runs (here without a device it fails for real)
    code = lib.gtmoe_open(0, C.byref(h))
    if no_device():
        assert code == gt.ERR_DEVICE
        assert lib.gtmoe_last_error(None).decode().startswith("no HIP device")
    else:
        assert code == gt.OK
        assert lib.gtmoe_close(h) == gt.OK


def test_injection_is_per_thread_and_per_entry_point():
    lib = gt.library()
    gt.inject_failure("gtmoe_open", gt.ERR_UNSUPPORTED)
    seen = {}

    def other():
        h = C.c_void_p()
        seen["code"] = lib.gtmoe_open(0, C.byref(h))
        if h.value:
            lib.gtmoe_close(h)
        seen["text"] = lib.gtmoe_last_error(None).decode()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["code"] != gt.ERR_UNSUPPORTED and "injected" not in seen["text"]
    h = C.c_void_p()
    assert lib.gtmoe_open(0, C.byref(h)) == gt.ERR_UNSUPPORTED  # still armed on this thread
    # arming another entry point replaces the armed one
    gt.inject_failure("gtmoe_open", gt.ERR_DEVICE)
    gt.inject_failure("gtmoe_forward", gt.ERR_DEVICE)
    code = lib.gtmoe_open(0, C.byref(h))
    assert "injected" not in lib.gtmoe_last_error(None).decode() or code == gt.OK
    if h.value:
        lib.gtmoe_close(h)
    gt.inject_failure("gtmoe_forward", gt.OK)  # disarm


def test_injection_rejects_bad_arguments():
    lib = gt.library()
    assert lib.gtmoe_test_inject_failure(None, gt.ERR_DEVICE) == gt.ERR_INVALID_ARGUMENT
    assert lib.gtmoe_test_inject_failure(b"gtmoe_open", 99) == gt.ERR_INVALID_ARGUMENT
    assert lib.gtmoe_test_inject_failure(b"gtmoe_open", -1) == gt.ERR_INVALID_ARGUMENT


def test_null_handles_are_refused():
    lib = gt.library()
    for call in (lambda: lib.gtmoe_close(None), lambda: lib.gtmoe_layer_destroy(None),
                 lambda: lib.gtmoe_forward(None, 1, None, None, None, 0),
                 lambda: lib.gtmoe_forward_device(None, 1, None, None, None, 0, None),
                 lambda: lib.gtmoe_last_routing(None, None, None, None, None, None, None),
                 lambda: lib.gtmoe_update_balance(None, 0.1), lambda: lib.gtmoe_graph_launch(None, None),
                 lambda: lib.gtmoe_timing_enable(None, 1), lambda: lib.gtmoe_relaunch(None, 0, None),
                 lambda: lib.gtmoe_backward(None, 1, None, None)):
        assert call() == gt.ERR_INVALID_ARGUMENT
