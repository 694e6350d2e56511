"""Presynaptic dynamics of feedforward pathways in the oracle (reference
``network_simulators/network.py:186-250``, ``tests/test_stp.py``): short-term plasticity's
factors against the event-by-event map of Markram, Wang & Tsodyks (1998) in float64 —
each spike's input is its release over ``U``, a first spike from rest exactly 1 — and
receptor saturation driven by those releases against its recursion restated in float64
(the reference's ``test_release_drives_saturation``): each release opens ``c f`` of the
closed receptors, at most all of them."""

import math

import numpy as np
import pytest
import torch

import oracle.dynamics as od
from wiretorch_amd.network import Drive, Gate

DT = 1.0


def markram(times, U, tau_D, tau_F):
    """Release at each spike: ``r_n = u_n R_n``, ``u_{n+1} = U + u_n (1 - U) e^{-dt/tau_F}``,
    ``R_{n+1} = R_n (1 - u_n) e^{-dt/tau_D} + 1 - e^{-dt/tau_D}`` (``u_1 = U``, ``R_1 = 1``)."""
    u, R, out = U, 1.0, []
    for n, t in enumerate(times):
        if n:
            gap = (t - times[n - 1]) * DT
            fac = math.exp(-gap / tau_F) if tau_F > 0 else 0.0
            rec = math.exp(-gap / tau_D)
            u, R = U + u * (1 - U) * fac, R * (1 - u) * rec + 1 - rec
        out.append(u * R)
    return np.array(out)


def _gate(U, tau_D, tau_F, c=0.0, tau=1.0, stp=True, saturates=False, n=1):
    d_F = math.exp(-DT / tau_F) if tau_F > 0 else 0.0
    params = torch.tensor([c, math.exp(-DT / tau), U, math.exp(-DT / tau_D), d_F],
                          dtype=torch.float32)
    return Gate(params, stp, saturates, 0, n)


def _rest(gate, B):
    parts = []
    if gate.stp:
        parts += [torch.full((B, gate.n), float(gate.params[2])), torch.ones((B, gate.n))]
    if gate.saturates:
        parts.append(torch.zeros((B, gate.n)))
    return torch.cat(parts, dim=1)


def _one_input(gate):
    W = torch.ones((1, 2))
    return Drive(made=torch.ones((1, 1), dtype=torch.bool), scale=torch.ones((1, 2)),
                 feedforward=[(torch.tensor([0]), W)], gates=[gate])


def _train(seed, steps=400, p=0.06):
    rng = np.random.default_rng(seed)
    x = (rng.random((2, steps, 1)) < p).astype(np.float32)
    x[:, 0] = 1.0  # a first spike from rest
    return torch.from_numpy(x)


@pytest.mark.parametrize("U, tau_D, tau_F", [(0.5, 800.0, 0.0), (0.03, 130.0, 530.0),
                                            (0.2, 300.0, 150.0)],
                         ids=["depressing", "facilitating", "both"])
def test_release_follows_markram(U, tau_D, tau_F):
    gate = _gate(U, tau_D, tau_F)
    x = _train(0)
    factors, state = od.gate_feedforward(_one_input(gate), x, _rest(gate, 2))
    f = factors[0][..., 0].numpy()
    for trial in range(2):
        times = np.flatnonzero(x[trial, :, 0].numpy())
        expected = markram(times.tolist(), U, tau_D, tau_F) / U
        assert f[trial, times[0]] == 1.0  # exactly its weight from rest
        np.testing.assert_allclose(f[trial, times], expected, rtol=1e-4)  # the reference's
    assert state.shape == (2, 2)


def test_release_drives_saturation():
    U, tau_D, tau_F, c, tau = 0.03, 130.0, 530.0, 0.4, 20.0
    gate = _gate(U, tau_D, tau_F, c=c, tau=tau, saturates=True)
    x = _train(1, steps=300, p=0.08)
    factors, state = od.gate_feedforward(_one_input(gate), x, _rest(gate, 2))
    xs = x[:, :, 0].double().numpy()
    d_D, d_F, d = math.exp(-DT / tau_D), math.exp(-DT / tau_F), math.exp(-DT / tau)
    u, r = np.full(2, U), np.ones(2)
    g, want = np.zeros(2), []
    for t in range(x.shape[1]):
        r = 1 - (1 - r) * d_D
        u = U + (u - U) * d_F
        release = u * r / U
        r = r - xs[:, t] * u * r
        u = u + xs[:, t] * U * (1 - u)
        g = g * d
        f = np.minimum(c * release * (1 - g), 1 - g)
        g = np.minimum(g + xs[:, t] * f, 1.0)
        want.append(f)
    np.testing.assert_allclose(factors[0][..., 0].double().numpy(), np.stack(want, 1),
                               rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(state[:, 2].double().numpy(), g, rtol=1e-4, atol=1e-6)
    assert max(float(np.max(w)) for w in want) > 0  # it opened receptors


def test_saturation_alone_opens_at_most_the_closed():
    """Without STP a release opens ``c (1 - g)`` of what its decay left closed; a
    saturation of 1 opens all of it."""
    gate = _gate(1.0, 1.0, 0.0, c=1.0, tau=5.0, stp=False, saturates=True)
    x = torch.zeros((1, 6, 1))
    x[0, [0, 1, 4]] = 1.0
    factors, state = od.gate_feedforward(_one_input(gate), x, torch.zeros((1, 1)))
    f = factors[0][0, :, 0]
    d = math.exp(-DT / 5.0)
    assert f[0] == 1.0  # all open after the first spike
    assert torch.allclose(f[1], torch.tensor(1 - d), rtol=1e-6)  # what one step's decay closed
    assert torch.allclose(f[4], torch.tensor(1 - d ** 3), rtol=1e-5)  # three steps' after t = 1
    assert float(state[0, 0]) == pytest.approx(d)  # open again after t = 4, one decay since


# =====================================================================
# The network layer (reference tests/test_stp.py, tests/test_saturation.py), on the oracle
# =====================================================================

import scenarios as sc  # noqa: E402
from wiretorch_amd import stp as wt_stp  # noqa: E402
from wiretorch_amd.network import FeedforwardConductanceLIFNetwork  # noqa: E402
from wiretorch_amd.projections import FrozenProjection  # noqa: E402


def _inputs_onto_one(weights, saturation, tau_decay, dt, batch_size, **kwargs):
    """One neuron driven by ``len(weights)`` inputs through one saturating synapse type
    (reference ``tests/test_saturation.py:36-72``)."""
    return FeedforwardConductanceLIFNetwork(
        dt=dt, projections={("in", "e"): FrozenProjection(np.asarray(weights)[:, None])},
        cell_type_indices=np.zeros(1, dtype=np.int64),
        cell_type_indices_FF=np.zeros(len(weights), dtype=np.int64),
        cell_params=[dict(name="e", cell_id=0, tau_mem=20.0, theta=50.0, U_reset=-60.0,
                          E_L=-60.0, g_L=1.0)],
        cell_params_FF=[dict(name="in", cell_id=0)],
        synapse_params_FF=[dict(name="NMDA", synapse_id=0, cell_id=0, tau_rise=0.5,
                                tau_decay=tau_decay, E_syn=0.0, g_bar=2.0,
                                saturation=saturation)],
        surrgrad_scale=5.0, batch_size=batch_size, **kwargs)


def test_conductance_follows_the_gating():
    """Each step the saturating type's decay component is ``g_bar sum_j w_j u_j``, ``u_j``
    the gating recursion over input ``j``'s spikes in float64 — the kernel of a
    saturating type unnormalised (``g_bar``: every receptor open)."""
    weights = [0.5, 1.0, 2.0]
    model = _inputs_onto_one(weights, 0.4, 20.0, 1.0, 2, track_variables=True)
    sc.use_engine(model, od)
    rng = np.random.default_rng(0)
    x = (rng.random((2, 300, 3)) < 0.08).astype(np.float32)
    out = model(torch.from_numpy(x))
    u, us, decay = np.zeros((2, 3)), [], math.exp(-1.0 / 20.0)
    for t in range(x.shape[1]):
        u = u * decay
        u = np.minimum(u + x[:, t] * 0.4 * (1 - u), 1.0)
        us.append(u)
    u = np.stack(us, axis=1)
    got = out["conductances_feedforward"][:, :, 0, 1, 0].numpy()
    np.testing.assert_allclose(got, 2.0 * u @ np.asarray(weights), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(model.gating.numpy(), u[:, -1], atol=1e-6)


def test_pathways_and_rest_state():
    """The mitral source type: depressing onto excitatory, facilitating onto inhibitory
    targets, each with its plain and its saturating (NMDA) synapses — four pathways over
    its rows; the state starts at rest (u = U, x = 1, g = 0)."""
    model = sc.feedforward(sc.BATCH_SIZE, sc.SEED, stp=True, saturation=0.63).model
    mitral = [p for p in model.pathways if p.cell_type == 0]
    assert len(mitral) == 4 and len({p.owner for p in mitral}) == 1
    assert {(p.stp, p.targets) for p in mitral} == {(wt_stp.DEPRESSING, (0,)),
                                                   (wt_stp.FACILITATING, (1,))}
    assert sorted(p.gate is not None for p in mitral) == [False, False, True, True]
    model.reset_state()
    for p in mitral:
        start, n = model._gate_columns[p.index]
        u, x = model.gating[:, start:start + n], model.gating[:, start + n:start + 2 * n]
        assert (u == p.stp.U).all() and (x == 1).all()
        if p.gate is not None:
            assert (model.gating[:, start + 2 * n:start + 3 * n] == 0).all()
    plain = sc.feedforward(sc.BATCH_SIZE, sc.SEED).model
    assert [p.presynaptic for p in plain.pathways] == [False] * 3 and plain.n_gating == 0


def _oracle_run(stp, saturation, chunks=1, checkpoints=False, T=60):
    built = sc.feedforward(sc.BATCH_SIZE, sc.SEED, stp=stp, saturation=saturation)
    model = built.model
    sc.use_engine(model, od)
    model.reset_state()
    x = torch.from_numpy(built.input_spikes[:, :T]).float()
    out = []
    with torch.no_grad():
        for xc in x.split(T // chunks, dim=1):
            if checkpoints:
                state = model.get_checkpoint_state()
                model.reset_state()
                model.load_checkpoint_state(state)
            out.append(model(xc))
    return torch.cat(out, dim=1), model.gating.clone()


def test_presynaptic_dynamics_change_the_network_and_carry_across_chunks():
    plain, _ = _oracle_run(False, None)
    one = _oracle_run(True, 0.63)
    assert not torch.equal(plain, one[0])
    for kwargs in (dict(chunks=3), dict(chunks=3, checkpoints=True)):
        again = _oracle_run(True, 0.63, **kwargs)
        assert torch.equal(again[0], one[0]) and torch.equal(again[1], one[1]), kwargs


def test_validation():
    with pytest.raises(ValueError, match="U must be"):
        wt_stp.STP(U=0.0, tau_D=100.0)
    with pytest.raises(ValueError, match="tau_D"):
        wt_stp.STP(U=0.5, tau_D=0.0)
    with pytest.raises(ValueError, match="no projection"):
        _inputs_onto_one([1.0], 0.0, 20.0, 1.0, 1, stp={("in", "x"): wt_stp.DEPRESSING})
    model = _inputs_onto_one([1.0], 0.0, 20.0, 1.0, 1, stp={("in", "e"): dict(U=0.4, tau_D=200.0)})
    assert model.pathways[0].stp == wt_stp.STP(U=0.4, tau_D=200.0)
    with pytest.raises(AssertionError, match="saturation"):
        _inputs_onto_one([1.0], 1.5, 20.0, 1.0, 1)
    with pytest.raises(ValueError, match="tau_decay"):
        _inputs_onto_one([1.0], 0.5, 20.0, 1.0, 1, learn={"tau_decay": True})
    with pytest.raises(NotImplementedError, match="feedforward"):
        sc.recurrent(sc.BATCH_SIZE, sc.SEED, saturation=0.63)
