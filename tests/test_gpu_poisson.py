"""On-device Poisson input on the GPU (``PoissonInput``: drawn inside ``wt_cond_run``):

* ``wt_poisson_fill`` writes the host replay's spikes bit for bit (configuration 2's
  sensory channels, 8 trials, a window that continues the stream);
* a network run with the input drawn on the device equals the run on the replayed
  tensor (raster and voltages bit for bit) and the oracle on it with exactly rounded sums
  (raster, voltages within 1e-5 relative) — on a fly-scale-form network (one channel per sensory neuron) and on an
  Erdős–Rényi network whose 500 channels at up to 200 Hz put some (trial, step) rows past
  the 64-entry input lists (drawn again inside the run kernel);
* a chunked run (two windows of the stream) equals one call.
"""

import numpy as np
import pytest
import torch

import oracle.dynamics as oracle_engine
import scenarios as sc
from wiretorch_amd import engine, synthetic
from wiretorch_amd.inputs import PoissonInput

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_fill_equals_host_replay():
    x = PoissonInput(np.full(7000, 10.0), dt=0.1, batch_size=8, n_steps=300, seed=99)
    assert np.array_equal(x.materialize().cpu().numpy() != 0, x.replay())
    w = x.window(1000, 1100)
    assert np.array_equal(w.materialize().cpu().numpy() != 0, w.replay())
    dense = PoissonInput(np.linspace(1.0, 900.0, 333), dt=1.0, batch_size=3, n_steps=50,
                         seed=2**40 + 7)
    assert np.array_equal(dense.materialize().cpu().numpy() != 0, dense.replay())


def _run(model, x, eng, device, track=True):
    model = model.to(device)
    sc.use_engine(model, eng)
    model.reset_state()
    model.track_variables, model.track_batch_idx = track, None
    with torch.no_grad():
        out = model(x)
    model.track_variables = False
    return (out["spikes"].cpu().numpy(), out["voltages"].cpu().numpy()) if track else out


def _workloads():
    fly = synthetic.fly_scale_network(N=5000, n_types=200, mean_degree=120, k_max=1500, B=4,
                                      T=200)
    rates = np.random.default_rng(3).uniform(20.0, 200.0, 500)
    er = synthetic.er_network(N=2000, frac_e=0.8, p=0.05, n_in=500, p_in=0.04, in_scale=8.0,
                              rates_hz=rates, B=4, T=200, dt=1.0, seed=4)
    return {"fly": (fly, np.full(fly.model.n_inputs, 10.0), 0.1),
            "er-dense-rows": (er, rates, 1.0)}


@pytest.mark.parametrize("name", ["fly", "er-dense-rows"])
def test_network_with_drawn_input(name, monkeypatch):
    monkeypatch.setattr(oracle_engine, "SUMS", "exact")  # the sums the kernel computes
    wl, rates, dt = _workloads()[name]
    B, T = wl.x.shape[:2]
    pin = PoissonInput(rates, dt=dt, batch_size=B, n_steps=T, seed=7)
    replay = torch.from_numpy(pin.replay()).float()
    if name == "er-dense-rows":
        assert (replay.sum(dim=2) > 64).any(), "no row past the input lists"
    s_pin, v_pin = _run(wl.model, pin, engine, DEV)
    s_x, v_x = _run(wl.model, replay.to(DEV), engine, DEV)
    assert s_pin.sum() > 0
    assert np.array_equal(s_pin, s_x) and np.array_equal(v_pin, v_x)
    s_ref, v_ref = _run(wl.model, replay, oracle_engine, "cpu")
    differs = (s_pin != s_ref).any(axis=(0, 2))
    assert not differs.any(), f"rasters differ from step {int(np.argmax(differs))}"
    np.testing.assert_allclose(v_pin, v_ref, rtol=1e-5, atol=65e-5)


def test_chunked_stream_equals_one_call():
    wl, rates, dt = _workloads()["fly"]
    B, T = wl.x.shape[:2]
    pin = PoissonInput(rates, dt=dt, batch_size=B, n_steps=T, seed=11)
    model = wl.model.to(DEV)
    sc.use_engine(model, engine)
    with torch.no_grad():
        model.reset_state()
        whole = model(pin)
        model.reset_state()
        parts = torch.cat([model(pin.window(0, 120)), model(pin.window(120, T))], dim=1)
    assert whole.sum() > 0 and torch.equal(whole, parts)
