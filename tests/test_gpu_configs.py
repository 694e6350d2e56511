"""Configurations 1 and 3 on the GPU against the CPU oracle, at their full network size
(10,000 neurons, ~2M synapses) with fewer trials and steps than the benchmark.

* Configuration 1 (forward, dt 0.1 ms): spike raster identical to the oracle's over the
  first 200 steps, voltages within 1e-5 relative — the bar of configuration 0.
* Dense firing (a strongly driven configuration-3 network at 70 Hz, 16 trials in 8
  groups, two per workgroup): most steps list more than 1,024 fired sources per workgroup, some more than
  2,048. With the 2,048-entry event list most steps are pushed in one round, with the
  1,024-entry list (``engine.MAX_LIST``) in two or three. Forward and training step to the
  bars of configurations 1 and 3, both ways.
* Two training steps of configuration 3's network with the learnt weights changed in
  between: the second takes the new weights through the cached layout of the dense
  pathways (no new compression), to the same bar; and the network's synapse-by-synapse
  form of those weights (what the engine is given by default) following a changed mask.
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
from wiretorch_amd.connectome import Connectome

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


def _dense_workload():
    rates = np.random.default_rng([5, 99]).uniform(20.0, 40.0, 500)
    return synthetic.er_network(N=10_000, frac_e=0.8, p=0.02, n_in=500, p_in=0.04,
                                in_scale=20.0, rates_hz=rates, B=16, T=40, dt=1.0, seed=5,
                                learnt=True, learn={"tau_mem": True, "theta": True},
                                surrgrad_scale=10.0)


def _fired_per_workgroup_step(spikes):
    """Sources fired per (group, step): every workgroup of a group lists the fired sources
    of all the group's trials (trial b in group b % groups)."""
    B, T, N = spikes.shape
    groups, _, _ = engine.geometry(B, N, 2, 256, 160 * 1024)
    return spikes.reshape(-1, groups, T, N).sum(axis=(0, 3))


@pytest.fixture(params=[2048, 1024], ids=["list-2048", "list-1024"])
def max_list(request):
    """The event list's size, with 8 groups (two trials per group, so that a workgroup
    lists more than 1,024 fired sources in most steps)."""
    saved = engine.MAX_LIST, engine.MAX_GROUPS
    engine.MAX_LIST, engine.MAX_GROUPS = request.param, 8
    yield request.param
    engine.MAX_LIST, engine.MAX_GROUPS = saved


def test_dense_firing_forward_matches_oracle(max_list):
    wl = _dense_workload()
    x = torch.from_numpy(wl.x).float()
    s_ref, v_ref = _forward(wl.model, x, oracle_engine)
    per = _fired_per_workgroup_step(s_ref)
    assert per.max() > 2 * 1024 and (per > 1024).mean() > 0.5, per.max()
    wl.model.to(DEV)
    s_gpu, v_gpu = _forward(wl.model, x.to(DEV), engine)
    differs = (s_gpu != s_ref).any(axis=(0, 2))
    assert not differs.any(), f"rasters differ from step {int(np.argmax(differs))}"
    np.testing.assert_allclose(v_gpu, v_ref, rtol=1e-5, atol=1e-5 * 65)


def test_dense_firing_training_step_matches_oracle(max_list):
    wl = _dense_workload()
    x = torch.from_numpy(wl.x).float()
    target = torch.from_numpy(synthetic.gamma_targets(5, wl.N, 2))
    s_ref, l_ref, g_ref = _training_step(wl, x, target, oracle_engine, "cpu")
    assert _fired_per_workgroup_step(s_ref).max() > 2 * 1024
    s_gpu, l_gpu, g_gpu = _training_step(wl, x, target, engine, DEV)
    differs = (s_gpu != s_ref).any(axis=(0, 2))
    assert not differs.any(), f"rasters differ from step {int(np.argmax(differs))}"
    np.testing.assert_allclose(l_gpu, l_ref, rtol=1e-5)
    assert g_ref.keys() == g_gpu.keys() and len(g_ref) == 6
    for key, value in g_ref.items():
        scale = np.abs(value).max()
        assert scale > 0, key
        np.testing.assert_allclose(g_gpu[key], value, rtol=0, atol=1e-4 * scale, err_msg=key)


def test_learnt_weights_update_reuses_layout(monkeypatch):
    """The engine's dense path (rows of learnt weights, compressed once and gathered
    again while the nonzero pattern holds), taken here by turning off the network's
    synapse-by-synapse form (``_edge_sides``)."""
    wl = synthetic.config3(B=2, T=60)
    monkeypatch.setattr(type(wl.model), "_edge_sides", lambda self: [])
    x = torch.from_numpy(wl.x).float()
    target = torch.from_numpy(synthetic.gamma_targets(3, wl.N, 3))
    _training_step(wl, x, target, engine, DEV)
    built = []
    original = engine._from_pathways
    monkeypatch.setattr(engine, "_from_pathways",
                        lambda *a, **k: built.append(1) or original(*a, **k))
    with torch.no_grad():  # new values, same nonzero pattern
        for name, p in wl.model.named_parameters():
            if name.endswith("log_weights"):
                p.mul_(1.05)
    s_gpu, l_gpu, g_gpu = _training_step(wl, x, target, engine, DEV)
    assert not built, "the dense pathways were compressed again"
    s_ref, l_ref, g_ref = _training_step(wl, x, target, oracle_engine, "cpu")
    differs = (s_gpu != s_ref).any(axis=(0, 2))
    assert not differs.any(), f"rasters differ from step {int(np.argmax(differs))}"
    np.testing.assert_allclose(l_gpu, l_ref, rtol=1e-5)
    for key, value in g_ref.items():
        scale = np.abs(value).max()
        np.testing.assert_allclose(g_gpu[key], value, rtol=0, atol=1e-4 * scale, err_msg=key)
    # back on the GPU (new tensors: a new layout), then one synapse fewer: a new nonzero
    # pattern under the same structure, compressed anew
    _training_step(wl, x, target, engine, DEV)
    built.clear()
    with torch.no_grad():
        mask = dict(wl.model.named_buffers())["rec_projections.E__E.mask"]
        flat = mask.view(-1)
        flat[int(torch.nonzero(flat)[0])] = 0.0
    s_gpu, _, _ = _training_step(wl, x, target, engine, DEV)
    assert built, "a changed nonzero pattern kept the old layout"
    s_ref, _, _ = _training_step(wl, x, target, oracle_engine, "cpu")
    assert np.array_equal(s_gpu, s_ref)


def test_learnt_weights_by_synapse_follow_the_mask(monkeypatch):
    """The network's synapse-by-synapse form of learnt recurrent weights (what the HIP
    engine is given for config 3): one synapse fewer in a mask rebuilds the plan; the
    training step then gives the dense path's raster, loss and gradients (the same
    per-synapse gradient kernel: equal to float32 rounding) and the oracle's raster and
    loss."""
    wl = synthetic.config3(B=2, T=60)
    x = torch.from_numpy(wl.x).float()
    target = torch.from_numpy(synthetic.gamma_targets(3, wl.N, 3))
    model = wl.model
    _training_step(wl, x, target, engine, DEV)
    side = model._edge_sides()
    assert side, "config 3's recurrent side is not formed synapse by synapse"
    before = model._edge_connectome(side[0]).n_edges
    with torch.no_grad():
        mask = dict(model.named_buffers())["rec_projections.E__E.mask"]
        flat = mask.view(-1)
        flat[int(torch.nonzero(flat)[0])] = 0.0
    s_gpu, l_gpu, g_gpu = _training_step(wl, x, target, engine, DEV)
    assert model._edge_connectome(side[0]).n_edges == before - 1
    with monkeypatch.context() as m:
        m.setattr(type(model), "_edge_sides", lambda self: [])
        s_dense, l_dense, g_dense = _training_step(wl, x, target, engine, DEV)
    assert np.array_equal(s_gpu, s_dense)
    np.testing.assert_allclose(l_gpu, l_dense, rtol=1e-6)
    assert g_gpu.keys() == g_dense.keys()
    for key, value in g_dense.items():
        scale = np.abs(value).max()
        np.testing.assert_allclose(g_gpu[key], value, rtol=0, atol=1e-6 * scale, err_msg=key)
    s_ref, l_ref, _ = _training_step(wl, x, target, oracle_engine, "cpu")
    differs = (s_gpu != s_ref).any(axis=(0, 2))
    assert not differs.any(), f"rasters differ from step {int(np.argmax(differs))}"
    np.testing.assert_allclose(l_gpu, l_ref, rtol=1e-5)


# ---------------------------------------------------------------------------------
# The launch geometries the benchmarks run
# ---------------------------------------------------------------------------------


def _plan(B, N, K=3):
    n_cu, lds = engine._device_info(torch.device(DEV))
    return engine.geometry(B, N, K, n_cu, lds)


def _to(obj, device):
    """A ``Drive`` or ``Physiology`` with every tensor copied to ``device`` (differentiably:
    gradients flow back to the originals)."""
    import dataclasses

    def move(value):
        if torch.is_tensor(value):
            return value.to(device)
        if isinstance(value, Connectome):
            return value.to(device)
        if isinstance(value, list):
            return [move(v) for v in value]
        if isinstance(value, tuple):
            return tuple(move(v) for v in value)
        return value

    return dataclasses.replace(obj, **{f.name: move(getattr(obj, f.name))
                                       for f in dataclasses.fields(obj)})


def _engine_training_step(wl, x, target, eng, device):
    """One training step through ``simulate`` itself, on tables built once on the CPU by
    the network (so both engines integrate bit-identical physiology; a network on the GPU
    recomputes its learnt decays there, with torch's GPU ``exp``, which differs from its
    CPU ``exp`` in the last place)."""
    model = wl.model
    model.reset_state()
    model.zero_grad(set_to_none=True)
    drive, p = model._drive(), model._physiology()
    run = eng.simulate(model.v.to(device), model._synaptic.to(device), x.to(device),
                       _to(drive, device), _to(p, device),
                       refractory=model.refractory.to(device))
    loss = synthetic.binned_rate_loss(run.spikes, target.to(device), model.dt.item())
    loss.backward()
    grads = {n: q.grad.detach().cpu().numpy() for n, q in model.named_parameters()
             if q.grad is not None}
    return run.spikes.detach().cpu().numpy(), float(loss.detach()), grads


def test_config3_bench_geometry_training_step(monkeypatch):
    """Configuration 3's benchmarked batch (64 trials: 64 groups of 4 workgroups, 2,528
    targets each, three items per thread, the training kernel with saved tensors) over
    50 steps through ``simulate``: raster, loss and all six gradients against the oracle
    with exactly rounded sums (``SUMS = "exact"``, what the kernel computes). At 32M
    neuron-steps with ~12k spikes per step, a last-place difference in any input flips a
    spike within the 50 steps: the float32 BLAS rounding of the oracle's default product
    does, and so does torch's GPU ``exp`` in the learnt membrane decay (one place off from
    its CPU ``exp`` for every neuron here) — so the network's tables are built once, on
    the CPU, for both engines."""
    monkeypatch.setattr(oracle_engine, "SUMS", "exact")
    wl = synthetic.config3(B=64, T=50)
    groups, R, range_n = _plan(64, wl.N)
    assert (groups, R) == (64, 4) and -(-range_n // engine.BLOCK) == 3, (groups, R, range_n)
    x = torch.from_numpy(wl.x).float()
    target = torch.from_numpy(synthetic.gamma_targets(3, wl.N, 2))
    s_ref, l_ref, g_ref = _engine_training_step(wl, x, target, oracle_engine, "cpu")
    s_gpu, l_gpu, g_gpu = _engine_training_step(wl, x, target, engine, DEV)
    assert s_ref.sum() > 0
    differs = (s_gpu != s_ref).any(axis=(0, 2))
    assert not differs.any(), f"rasters differ from step {int(np.argmax(differs))}"
    np.testing.assert_allclose(l_gpu, l_ref, rtol=1e-5)
    assert g_ref.keys() == g_gpu.keys() and len(g_ref) == 6
    for key, value in g_ref.items():
        scale = np.abs(value).max()
        assert scale > 0, key
        np.testing.assert_allclose(g_gpu[key], value, rtol=0, atol=1e-4 * scale, err_msg=key)


def test_config1_bench_geometry():
    """Configuration 1's benchmarked batch (32 trials: 32 groups of 8 workgroups, 1,280
    targets each, two items per thread) over 200 steps: the raster equal to the oracle's,
    voltages within 1e-5 relative."""
    wl = synthetic.config1(T=200, B=32)
    groups, R, range_n = _plan(32, wl.N)
    assert (groups, R) == (32, 8) and -(-range_n // engine.BLOCK) == 2, (groups, R, range_n)
    x = torch.from_numpy(wl.x).float()
    s_ref, v_ref = _forward(wl.model, x, oracle_engine)
    wl.model.to(DEV)
    s_gpu, v_gpu = _forward(wl.model, x.to(DEV), engine)
    assert s_ref.sum() > 0
    differs = (s_gpu != s_ref).any(axis=(0, 2))
    assert not differs.any(), f"rasters differ from step {int(np.argmax(differs))}"
    np.testing.assert_allclose(v_gpu, v_ref, rtol=1e-5, atol=1e-5 * 65)


# ---------------------------------------------------------------------------------
# Beyond the chaotic-divergence horizon
# ---------------------------------------------------------------------------------

LONG_B, LONG_T = 8, 2000


def _free_run(model, x, eng, v0=None):
    sc.use_engine(model, eng)
    model.track_variables = False
    model.reset_state()
    if v0 is not None:
        model.v = v0.to(model.v.device)
    with torch.no_grad():
        return model(x).cpu().numpy() > 0.5


def test_config1_long_horizon_rates():
    """Configuration 1 (8 trials) over 2,000 steps, the north star's per-neuron rate
    criterion. Should the GPU's and the oracle's rasters part (a last-place difference
    flipping a spike; none did on the MI355X, where all 2,000 steps agree), rates are
    compared as firing statistics:

    * the population's and each cell type's mean rate within 1%;
    * per neuron, over the whole run: the GPU-oracle discrepancy (mean over neurons of
      the absolute rate difference, and the counting-noise chi-square of the per-neuron
      spike counts) no larger than that between two GPU runs that differ by one spike
      at step 0 in each trial, plus 1% of the mean rate: a flipped spike is what a
      rounding difference eventually causes, so this is the discrepancy chaos alone
      produces (each neuron's count over 0.2 s carries a Poisson error of ~15%, so a
      literal 1% per neuron could only hold between identical trajectories);
    * per neuron, before the rasters part: identical counts."""
    wl = synthetic.config1(T=LONG_T, B=LONG_B)
    x = torch.from_numpy(wl.x).float()
    s_ref = _free_run(wl.model, x, oracle_engine)
    wl.model.to(DEV)
    xd = x.to(DEV)
    s_gpu = _free_run(wl.model, xd, engine)
    # one neuron per trial (a different one in each) starts above threshold
    v0 = torch.full((LONG_B, wl.N), synthetic.U_RESET)
    v0[torch.arange(LONG_B), torch.arange(LONG_B) * 997 + 13] = synthetic.THETA + 1.0
    s_pert = _free_run(wl.model, xd, engine, v0)

    differs = (s_gpu != s_ref).any(axis=(0, 2))
    horizon = int(np.argmax(differs)) if differs.any() else LONG_T
    print(f"rasters part at step {horizon} of {LONG_T}")
    assert horizon >= 200, horizon
    early = slice(0, horizon)
    assert np.array_equal(s_gpu[:, early].sum(axis=(0, 1)), s_ref[:, early].sum(axis=(0, 1)))

    to_hz = 1000.0 / (LONG_B * LONG_T * 0.1)
    c_gpu, c_ref, c_pert = (s.sum(axis=(0, 1)).astype(np.float64) for s in (s_gpu, s_ref, s_pert))
    r_gpu, r_ref, r_pert = c_gpu * to_hz, c_ref * to_hz, c_pert * to_hz
    mean = r_ref.mean()
    assert abs(r_gpu.mean() - mean) <= 0.01 * mean, (r_gpu.mean(), mean)
    types = wl.structure["types"]
    for t in np.unique(types):
        a, b = r_gpu[types == t].mean(), r_ref[types == t].mean()
        assert abs(a - b) <= 0.01 * b, (t, a, b)

    def chi2(a, b):
        both = a + b
        keep = both > 0
        return float(((a - b)[keep] ** 2 / both[keep]).mean())

    d_ref, d_pert = np.abs(r_gpu - r_ref).mean(), np.abs(r_gpu - r_pert).mean()
    x_ref, x_pert = chi2(c_gpu, c_ref), chi2(c_gpu, c_pert)
    print(f"mean rate {mean:.3f} Hz; per-neuron |dr| {d_ref:.3f} Hz against {d_pert:.3f} Hz "
          f"(chaos alone); chi2 {x_ref:.3f} against {x_pert:.3f}")
    assert d_ref <= d_pert + 0.01 * mean, (d_ref, d_pert)
    assert x_ref <= x_pert * 1.05 + 0.01, (x_ref, x_pert)
