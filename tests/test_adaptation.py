"""Spike-frequency adaptation in conductance networks, on the CPU oracle (reference
``tests/test_adaptation.py``): a cell type with ``adapt > 0`` gives each neuron a
conductance by ``E_adapt`` (part of the state) that decays with ``tau_adapt`` and rises
by ``adapt`` at each of the neuron's spikes (``conductance/dynamics.py:13-19,136-139,
200-202``).

These pin the oracle's restatement: the tracked adaptation follows its recursion from
the spikes (computed here in float64, independently), it lengthens the intervals under
constant drive, ``adapt = 0`` is the former network bit for bit, the state carries across
chunks and checkpoints, and the parameters are validated. The GPU's forward and
gradients are checked against the oracle in ``test_gpu_adaptation.py``.
"""

import math

import numpy as np
import pytest
import torch

import oracle.dynamics as oracle_engine
import scenarios as sc
from wiretorch_amd.network import FeedforwardConductanceLIFNetwork
from wiretorch_amd.projections import FrozenProjection

ADAPT = 2.0  # nS per spike
TAU_ADAPT = 150.0
LEARN_ADAPT = {"adapt": ["excitatory"], "tau_adapt": ["excitatory"]}


def _driven(adapt, n=3, batch_size=2):
    """``n`` uncoupled neurons under a constant strong input, adapting by ``adapt``."""
    cell = dict(name="e", cell_id=0, tau_mem=20.0, adapt=adapt, tau_adapt=TAU_ADAPT,
                theta=-50.0, U_reset=-65.0, E_L=-65.0, g_L=1.0, E_adapt=-90.0)
    synapse = dict(tau_rise=0.1, tau_decay=1.0, E_syn=0.0, g_bar=1.0)
    model = FeedforwardConductanceLIFNetwork(
        dt=1.0, projections={("in", "e"): FrozenProjection(np.full((1, n), 3.0))},
        cell_type_indices=np.zeros(n, dtype=np.int64),
        cell_type_indices_FF=np.zeros(1, dtype=np.int64), cell_params=[cell],
        cell_params_FF=[dict(name="in", cell_id=0)],
        synapse_params_FF=[dict(synapse_id=0, cell_id=0, name="s", **synapse)],
        surrgrad_scale=5.0, batch_size=batch_size, track_variables=True,
    )  # fmt: skip
    sc.use_engine(model, oracle_engine)
    return model


def _oracle(built):
    sc.use_engine(built.model, oracle_engine)
    return built.model


def test_adaptation_follows_the_spikes():
    """Each step it decays by exp(-dt / tau_adapt) and rises by adapt at the spike."""
    model = _driven(ADAPT)
    out = model(torch.ones((2, 400, 1)))
    spikes = out["spikes"].numpy().astype(np.float64)
    decay = math.exp(-1.0 / TAU_ADAPT)
    a, expected = np.zeros(spikes[:, 0].shape), []
    for t in range(spikes.shape[1]):
        a = a * decay + ADAPT * spikes[:, t]
        expected.append(a)
    np.testing.assert_allclose(out["adaptation"].numpy(), np.stack(expected, 1), rtol=1e-5,
                               atol=1e-6)
    assert spikes.sum() > 10
    torch.testing.assert_close(model.adaptation, out["adaptation"][:, -1])


def test_membrane_term_is_the_closed_form():
    """With no input and below threshold, each step of the exponential-Euler update with
    the adaptation conductance g_a(t) held over the step is the exact solution of
    C dv/dt = -g_L (v - E_L) - g_a (v - E_adapt): v_inf + (v - v_inf) exp(-dt (g_L + g_a) / C)
    with v_inf = (g_L E_L + g_a E_adapt) / (g_L + g_a), and g_a(t) = g_a(0) decay^t.
    Evaluated in float64 from the physiology tables; a dropped term of the conductance or
    a wrong sign of the current fails it."""
    model = _driven(ADAPT, n=1, batch_size=1)
    model.reset_state()
    with torch.no_grad():
        model.v.fill_(-60.0)
        model.adaptation.fill_(5.0)
    p = model._physiology()
    C, beta = float(p.C_m[0]), float(p.beta[0])
    E_L, E_a, dt = float(p.E_L[0]), float(p.E_adapt[0]), float(p.dt)
    decay = float(p.adapt_decay[0])
    g_L = C * -math.log(beta) / dt
    out = model(torch.zeros((1, 20, 1)))
    assert not out["spikes"].any()
    v, g_a = -60.0, 5.0
    for t in range(20):
        v_inf = (g_L * E_L + g_a * E_a) / (g_L + g_a)
        v = v_inf + (v - v_inf) * math.exp(-dt * (g_L + g_a) / C)
        g_a *= decay
        assert abs(float(out["voltages"][0, t, 0]) - v) < 1e-4, t
        assert abs(float(out["adaptation"][0, t, 0]) - g_a) < 1e-5, t


def test_intervals_lengthen():
    """Under constant drive the intervals lengthen as the adaptation builds up; without it
    they are regular."""
    intervals = {}
    for adapt in (0.0, ADAPT):
        spikes = _driven(adapt)(torch.ones((2, 600, 1)))["spikes"][0, :, 0]
        intervals[adapt] = torch.diff(torch.nonzero(spikes).flatten())
    regular, adapting = intervals[0.0], intervals[ADAPT]
    assert regular.max() - regular.min() <= 1
    assert adapting[-1] > 1.5 * adapting[0] and len(adapting) < len(regular)


def test_no_adaptation_is_the_former_network():
    runs = []
    for adapt in (None, 0.0):
        built = sc.recurrent(sc.BATCH_SIZE, sc.SEED, adapt=adapt)
        model = _oracle(built)
        assert not model._adapting
        runs.append(model(torch.from_numpy(built.input_spikes[:, :60])))
    torch.testing.assert_close(runs[0], runs[1], rtol=0, atol=0)
    built = sc.recurrent(sc.BATCH_SIZE, sc.SEED, adapt=ADAPT)
    assert not torch.equal(_oracle(built)(torch.from_numpy(built.input_spikes[:, :60])),
                           runs[0])


def test_state_carries_across_chunks_and_checkpoints():
    runs = []
    for mode in ("one", "chunks", "checkpoints"):
        built = sc.recurrent(sc.BATCH_SIZE, sc.SEED, adapt=ADAPT)
        model = _oracle(built)
        x = torch.from_numpy(built.input_spikes[:, :60])
        if mode == "one":
            runs.append((model(x), model.adaptation.clone()))
            continue
        chunks = []
        for start in range(0, 60, 10):
            if mode == "checkpoints":
                state = model.get_checkpoint_state()
                assert "adaptation" in state
                model.reset_state()
                assert not model.adaptation.any()
                model.load_checkpoint_state(state)
            chunks.append(model(x[:, start:start + 10]))
        runs.append((torch.cat(chunks, dim=1), model.adaptation.clone()))
    assert runs[0][1].any()
    for run in runs[1:]:
        torch.testing.assert_close(run, runs[0], rtol=0, atol=1e-5)


def test_checkpoints_without_adaptation_load():
    built = sc.recurrent(sc.BATCH_SIZE, sc.SEED, adapt=ADAPT)
    model = _oracle(built)
    model(torch.from_numpy(built.input_spikes[:, :30]))
    state = model.get_checkpoint_state()
    del state["adaptation"]
    model.load_checkpoint_state(state)
    assert not model.adaptation.any()
    assert "adaptation" not in sc.recurrent(sc.BATCH_SIZE, sc.SEED).model.get_checkpoint_state()


def test_validation():
    with pytest.raises(AssertionError, match="adapt"):
        _driven(-1.0)
    with pytest.raises(AssertionError, match="positive"):  # inhibitory types: adapt 0
        sc.recurrent(sc.BATCH_SIZE, sc.SEED, learn={"adapt": True}, adapt=ADAPT)
    model = sc.recurrent(sc.BATCH_SIZE, sc.SEED, learn=LEARN_ADAPT, adapt=ADAPT).model
    assert {"cell_parameters.log_adapt", "cell_parameters.log_tau_adapt"} <= set(
        dict(model.named_parameters()))
