"""A forward never stalls the host on the GPU (reference: its engine is sync-free by
design, ``conductance/kernels.py:181-182``): after a first call has built the cached
layouts, a forward through the network API under ``torch.cuda.set_sync_debug_mode
("error")`` makes no synchronising call — the fixed-point bound stays on the device and
the run's error word is read back without waiting. Checked on a compressed (fly-scale
form) network and on a dense one, and the deferred error check finds nothing."""

import pytest
import torch

from wiretorch_amd import engine, synthetic

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _workloads():
    fly = synthetic.fly_scale_network(N=5000, n_types=200, mean_degree=120, k_max=1500, B=2,
                                      T=100, device=DEV)
    dense = synthetic.config1(T=100, B=4)
    dense.model.to(DEV)
    return {"compressed": fly, "dense": dense}


@pytest.mark.parametrize("name", ["compressed", "dense"])
def test_forward_makes_no_synchronising_call(name):
    wl = _workloads()[name]
    model = wl.model
    x = torch.from_numpy(wl.x).float().to(DEV)
    with torch.no_grad():
        model.reset_state()
        first = model(x)  # builds and caches the layouts (host reads allowed here)
        torch.cuda.synchronize()
        torch.cuda.set_sync_debug_mode("error")
        try:
            model.reset_state()
            second = model(x)
        finally:
            torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    assert first.sum() > 0
    assert torch.equal(first, second)
    engine.check_errors(wait=True)
    assert not engine._PENDING


def test_new_learnt_physiology_makes_no_synchronising_call(monkeypatch):
    """A network with learnt per-type ``tau_mem`` and ``theta`` builds new tables after
    every parameter update. With the network's cell types as the classes of its
    per-neuron tables (``Physiology.type_of``) that forward makes no synchronising call
    either, and its raster equals the one from the distinct-row search (``type_of``
    cleared)."""
    import dataclasses

    from wiretorch_amd import network

    wl = synthetic.config3(T=60, B=4)
    model = wl.model.to(DEV)
    x = torch.from_numpy(wl.x).float().to(DEV)
    with torch.no_grad():
        model.reset_state()
        model(x)
        torch.cuda.synchronize()
        for prm in model.cell_parameters.parameters():
            prm.add_(0.01)
        torch.cuda.set_sync_debug_mode("error")
        try:
            model.reset_state()
            hinted = model(x)
        finally:
            torch.cuda.set_sync_debug_mode(0)
        engine.check_errors(wait=True)
        real = network.ConductanceNetwork._physiology
        monkeypatch.setattr(network.ConductanceNetwork, "_physiology",
                            lambda self: dataclasses.replace(real(self), type_of=None))
        model.reset_state()
        searched = model(x)
    assert hinted.sum() > 0
    assert torch.equal(hinted, searched)


def test_tables_that_differ_within_a_class_are_reported():
    """One neuron's threshold moved off its cell type's: the tables taken one row per
    type no longer describe it, which the device check reports at the next check."""
    wl = synthetic.config1(T=20, B=2)
    model = wl.model.to(DEV)
    x = torch.from_numpy(wl.x).float().to(DEV)
    engine.check_errors(wait=True)
    with torch.no_grad():
        model.theta[0] += 1.0
        model.reset_state()
        model(x)
    with pytest.raises(RuntimeError, match="type_of"):
        engine.check_errors(wait=True)
    assert not engine._PENDING
