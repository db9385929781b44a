"""CPU checks of slideformer_amd.cpu_adam_compat, the stand-in for the
reference's pybind module cpu_adam (cpu_adam.cpp:8-13, cpu_adam.h:199-221):
its signatures, its error behaviour, and that a call whose tensors are not
all on the host or all on one HIP device fails before it reaches the library,
so that no host address is ever handed to a device kernel."""
from __future__ import annotations

import inspect
import types

import pytest
import torch

from slideformer_amd import cpu_adam_compat as C
from slideformer_amd import _lib


def test_signatures_follow_the_reference_declarations():
    # cpu_adam.h:199-221
    create = inspect.signature(C.create_adam)
    assert list(create.parameters) == ["optimizer_id", "alpha", "betta1", "betta2", "eps", "weight_decay",
                                       "adamw_mode", "should_log"]
    assert [create.parameters[k].default for k in list(create.parameters)[1:]] == [
        1e-3, 0.9, 0.999, 1e-8, 0, True, False]
    assert list(inspect.signature(C.adam_update).parameters) == [
        "optimizer_id", "step", "lr", "beta1", "beta2", "epsilon", "weight_decay", "bias_correction",
        "params", "grads", "exp_avg", "exp_avg_sq"]
    assert list(inspect.signature(C.destroy_adam).parameters) == ["optimizer_id"]


class _NoLibrary:
    """A library handle that fails the test on any use."""

    def __getattr__(self, name):
        raise AssertionError(f"the library was reached ({name})")


@pytest.fixture
def no_library(monkeypatch):
    monkeypatch.setattr(C, "_library", lambda: _NoLibrary())


def _four(n=8, device="cpu"):
    return (torch.zeros(n, device=device), torch.zeros(n, dtype=torch.bfloat16, device=device),
            torch.zeros(n, device=device), torch.zeros(n, device=device))


def test_placement_rules():
    cpu, g0, g1 = torch.device("cpu"), torch.device("cuda", 0), torch.device("cuda", 1)
    fake = lambda *ds: [types.SimpleNamespace(device=d) for d in ds]  # noqa: E731
    assert C._where(fake(cpu, cpu, cpu, cpu)) == "host"
    assert C._where(fake(g0, g0, g0, g0)) == g0
    with pytest.raises(RuntimeError, match="all be in host memory or all on one"):
        C._where(fake(cpu, g0, cpu, cpu))            # a host master beside a device grad
    with pytest.raises(RuntimeError, match="all be in host memory or all on one"):
        C._where(fake(g0, g0, g1, g0))               # two devices
    with pytest.raises(RuntimeError, match="unsupported device type"):
        C._where(fake(torch.device("meta"), cpu, cpu, cpu))


def test_unsupported_devices_fail_before_the_library(no_library):
    p, g, m, v = _four()
    with pytest.raises(RuntimeError, match="unsupported device type meta"):
        C.adam_update(0, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, True, p, g.to("meta"), m, v)


def test_errors_before_the_library(no_library):
    p, g, m, v = _four()
    # the reference's contiguity checks and messages (cpu_adam_impl.cpp:234-237)
    strided = torch.zeros(16)[::2]
    for i, name in enumerate(("params", "grads", "exp_avg", "exp_avg_sq")):
        args = [p, g, m, v]
        args[i] = strided if i != 1 else torch.zeros(16, dtype=torch.bfloat16)[::2]
        with pytest.raises(RuntimeError, match=f"^{name} must be contiguous$"):
            C.adam_update(0, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, True, *args)
    with pytest.raises(RuntimeError, match="size mismatch"):
        C.adam_update(0, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, True, p, g[:4], m, v)
    with pytest.raises(TypeError):
        C.adam_update(0, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, True, p, None, m, v)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU behaviour")
def test_host_tensors_without_a_gpu_fail_loudly(no_library):
    with pytest.raises(RuntimeError, match="needs a HIP device"):
        C.adam_update(0, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, True, *_four())


def test_host_tensors_take_the_pipeline_never_the_device_kernel(monkeypatch):
    """With a GPU present (simulated), host tensors go to the pipeline path
    after the state machine advanced, and no direct kernel entry point is called."""
    calls = []

    class Recorder:
        def la_scalars(self, *args):
            calls.append("la_scalars")
            return 0

        def __getattr__(self, name):
            raise AssertionError(f"{name} must not be called for host tensors")

    monkeypatch.setattr(C, "_library", lambda: Recorder())
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(C, "_host_step", lambda L, sc, codes, tensors, n: calls.append(("pipeline", n, codes)))
    assert C.adam_update(0, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, True, *_four(10)) == 0
    assert calls == ["la_scalars", ("pipeline", 10, [_lib.LA_F32, _lib.LA_BF16, _lib.LA_F32])]
    # an unregistered triple: the state advances, then the reference's message
    calls.clear()
    p, g, m, v = _four(10)
    with pytest.raises(RuntimeError, match="param type Float, grads type Float and state type BFloat16 is not "
                                           "supported on current hardware"):
        C.adam_update(0, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, True, p, g.float(), m.bfloat16(), v.bfloat16())
    assert calls == ["la_scalars"]


def test_create_and_destroy_on_the_host_registry():
    # host-side only: the scalar state of an id, as the reference's registry holds it
    assert C.create_adam(7, 1e-3, 0.9, 0.999, 1e-8, 0.0, True, False) == 0
    assert C.destroy_adam(7) == 0
    with pytest.raises(RuntimeError):
        # an unknown id is an error, not a null dereference
        sc = _lib.LaScalars()
        import ctypes
        _lib.check(_lib.load().la_scalars(7, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, ctypes.byref(sc)), "la_scalars")


def test_layer_adam_holds_the_module_as_cpu_adam():
    from slideformer_amd import LayerAdam
    assert LayerAdam().cpu_adam is C


def test_creation_log_text_and_stream(capfd):
    """create_adam(..., should_log=True) prints the reference's two lines
    (cpu_adam_impl.cpp:116-125) with this build's capability name, on stderr
    rather than the reference's stdout, so that a caller's stdout (bench.py's
    one JSON line) stays its own; should_log=False prints nothing."""
    C.create_adam(77, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, True)
    C.destroy_adam(77)
    out, err = capfd.readouterr()
    assert out == ""
    assert err == ("Adam Optimizer #77 is created with MI355X (gfx950 HIP) arithmetic capability.\n"
                   "Config: alpha=0.001000, betas=(0.900000, 0.999000), weight_decay=0.010000, adam_w=1\n")
    C.create_adam(78, 1e-3, 0.9, 0.999, 1e-8, 0.0, False, False)
    C.destroy_adam(78)
    assert capfd.readouterr() == ("", "")
