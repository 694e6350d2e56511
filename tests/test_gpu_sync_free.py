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
