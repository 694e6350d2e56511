"""Configurations 1 and 3 on the GPU against the CPU oracle, at their full network size
(10,000 neurons, ~2M synapses) with fewer trials and steps than the benchmark.

* Configuration 1 (forward, dt 0.1 ms): spike raster identical to the oracle's over the
  first 200 steps, voltages within 1e-5 relative — the bar of configuration 0.
* Configuration 3 (training step: per-synapse learnt weights, learnt per-type tau_mem and
  theta, fast-sigmoid surrogate of slope 10, squared error of 20 ms-binned rates against
  gamma(2, 5 Hz) targets, dt 1 ms): over 100 steps, the same raster, the loss within 1e-5
  relative and every gradient within 1e-4 of its largest magnitude.
"""

import numpy as np
import pytest
import torch

import oracle.dynamics as oracle_engine
import scenarios as sc
from wiretorch_amd import engine, synthetic

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _forward(model, x, eng):
    sc.use_engine(model, eng)
    model.reset_state()
    model.track_variables, model.track_batch_idx = True, None
    with torch.no_grad():
        out = model(x)
    return out["spikes"].cpu().numpy(), out["voltages"].cpu().numpy()


def test_config1_matches_oracle():
    wl = synthetic.config1(T=200, B=4)
    x = torch.from_numpy(wl.x).float()
    s_ref, v_ref = _forward(wl.model, x, oracle_engine)
    wl.model.to(DEV)
    s_gpu, v_gpu = _forward(wl.model, x.to(DEV), engine)
    assert s_ref.sum() > 0, "no spikes: the check would be vacuous"
    differs = (s_gpu != s_ref).any(axis=(0, 2))
    assert not differs.any(), f"rasters differ from step {int(np.argmax(differs))}"
    np.testing.assert_allclose(v_gpu, v_ref, rtol=1e-5, atol=1e-5 * 65)


def _training_step(wl, x, target, eng, device):
    model = wl.model.to(device)
    sc.use_engine(model, eng)
    model.reset_state()
    model.zero_grad(set_to_none=True)
    spikes = model(x.to(device))
    loss = synthetic.binned_rate_loss(spikes, target.to(device), wl.model.dt.item())
    loss.backward()
    grads = {n: p.grad.detach().cpu().numpy() for n, p in model.named_parameters()
             if p.grad is not None}
    return spikes.detach().cpu().numpy(), float(loss.detach()), grads


def test_config3_training_step_matches_oracle():
    wl = synthetic.config3(B=2, T=100)
    x = torch.from_numpy(wl.x).float()
    target = torch.from_numpy(synthetic.gamma_targets(3, wl.N, 5))
    s_ref, l_ref, g_ref = _training_step(wl, x, target, oracle_engine, "cpu")
    s_gpu, l_gpu, g_gpu = _training_step(wl, x, target, engine, DEV)
    assert s_ref.sum() > 0
    differs = (s_gpu != s_ref).any(axis=(0, 2))
    assert not differs.any(), f"rasters differ from step {int(np.argmax(differs))}"
    np.testing.assert_allclose(l_gpu, l_ref, rtol=1e-5)
    assert g_ref.keys() == g_gpu.keys() and len(g_ref) == 6
    for key, value in g_ref.items():
        scale = np.abs(value).max()
        assert scale > 0, key
        np.testing.assert_allclose(g_gpu[key], value, rtol=0, atol=1e-4 * scale, err_msg=key)
