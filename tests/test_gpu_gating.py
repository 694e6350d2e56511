"""Presynaptic dynamics of feedforward pathways on the GPU against the oracle (reference
``tests/test_stp.py:302-312``, ``tests/test_saturation.py:332-347``): the gate scan
(``wt_gate_scan``) gives the oracle's factors and gating state bit for bit — short-term
plasticity, saturation, both, on spikes and on real-valued inputs — and a feed-forward
network whose input pathways have them (one of them a second pathway over the same
source rows with dynamics of its own) gives the oracle's spikes, voltages within 1e-5
and the gradients of its weights (at the synapses) and input within 1e-4 of their
scale; two chunks that
carry the gating state equal one call. Recurrent pathways with presynaptic dynamics
raise."""

import copy
import math
from dataclasses import replace

import numpy as np
import pytest
import torch

import oracle.dynamics as oracle_engine
import scenarios as sc
from wiretorch_amd import engine
from wiretorch_amd.network import Gate

pytestmark = pytest.mark.gpu
DEV = "cuda"
KINDS = [(True, False), (False, True), (True, True)]  # (stp, saturates) by pathway


def _gated(drive, dt, B, device, extra=True):
    """The drive's feedforward pathways with presynaptic dynamics (cycling KINDS), plus
    (``extra``) a second pathway over the first one's rows with half its weights and
    facilitating STP; the gating state at rest."""
    ff, made, scale = list(drive.feedforward), drive.made, drive.scale
    if extra:
        rows, W = ff[0]
        ff.append((rows, 0.5 * W))
        made = torch.cat([made, made[drive.K_rec: drive.K_rec + 1]])
        scale = torch.cat([scale, scale[drive.K_rec: drive.K_rec + 1]])
    gates, rest, start = [None] * drive.K_rec, [], 0
    for k, (rows, _) in enumerate(ff):
        stp, sat = KINDS[k % len(KINDS)] if k < len(drive.feedforward) else (True, False)
        U, tau_D, tau_F = (0.2, 300.0, 150.0) if k < len(drive.feedforward) else (0.03, 130.0, 530.0)
        params = torch.tensor([0.4, math.exp(-dt / 20.0), U, math.exp(-dt / tau_D),
                               math.exp(-dt / tau_F)], dtype=torch.float32, device=device)
        gate = Gate(params, stp, sat, start, rows.numel())
        gates.append(gate)
        start += gate.width
        if stp:
            rest += [np.full(gate.n, U), np.ones(gate.n)]
        if sat:
            rest.append(np.zeros(gate.n))
    gating = torch.from_numpy(np.concatenate(rest).astype(np.float32)).to(device)
    drive = replace(drive, feedforward=ff, made=made, scale=scale, gates=gates)
    return drive, gating.expand(B, -1).clone()


def _setup(device, T, real_valued=False):
    built = sc.feedforward(sc.BATCH_SIZE, sc.SEED)
    model = built.model.to(device)
    model.reset_state()
    x = torch.from_numpy(built.input_spikes[:, :T]).float().to(device)
    if real_valued:
        x = x * torch.linspace(0.5, 1.5, x.shape[-1], device=device)
    drive, gating = _gated(model._drive(), float(model.dt), x.shape[0], device)
    return model, x, drive, gating


@pytest.mark.parametrize("real_valued", [False, True], ids=["spikes", "values"])
def test_gate_scan_equals_oracle(real_valued):
    _, x, drive, gating = _setup(DEV, 150, real_valued)
    got_x, _, got_gating = engine._gate_inputs(drive, x, gating)
    cpu = replace(drive, feedforward=[(r.cpu(), W.cpu()) for r, W in drive.feedforward],
                  gates=[None if g is None else replace(g, params=g.params.cpu())
                         for g in drive.gates])
    factors, want_gating = oracle_engine.gate_feedforward(cpu, x.cpu(), gating.cpu())
    want_x = torch.cat([x.cpu()[:, :, rows] * f for (rows, _), f in zip(cpu.feedforward, factors)],
                       dim=2)
    torch.cuda.synchronize()
    assert torch.equal(got_gating.cpu(), want_gating)
    assert torch.equal(got_x.cpu(), want_x)
    assert (want_gating != gating.cpu()).any()  # the state moved


def _run(device, eng, T=100, chunks=1):
    torch.manual_seed(0)
    model, x, drive, gating = _setup(device, T)
    p = model._physiology()
    weights = [W.detach().clone().requires_grad_(True) for _, W in drive.feedforward]
    drive = replace(drive, feedforward=[(r, W) for (r, _), W in zip(drive.feedforward, weights)])
    x = x.clone().requires_grad_(True)
    v, g = model.v, model._synaptic
    spikes = []
    for xc in x.split(T // chunks, dim=1):
        run = eng.simulate(v, g, xc, drive, p, gating=gating)
        v, g, gating = run.v, run.syn, run.gating
        spikes.append(run.spikes)
    spikes = torch.cat(spikes, dim=1)
    R = torch.from_numpy(np.random.default_rng(3).standard_normal(spikes.shape)
                         .astype(np.float32)).to(device)
    (spikes * R).sum().backward()
    # on the support: the engine's weight gradient is dL/dW at the synapses (the
    # reference's learnt projections mask the rest, projections.py:164,216)
    grads = {f"W{k}": (W.grad * (W != 0)).detach().cpu().double()
             for k, W in enumerate(weights)}
    grads["x"] = x.grad.detach().cpu().double()
    return spikes.detach().cpu(), v.detach().cpu().double(), gating.detach().cpu(), grads


def test_gated_feedforward_network_matches_oracle():
    s_k, v_k, gt_k, g_k = _run(DEV, engine)
    s_r, v_r, gt_r, g_r = _run("cpu", oracle_engine)
    assert s_r.sum() > 0
    differs = (s_k != s_r).any(dim=0).any(dim=-1)
    assert not differs.any(), f"spikes differ from step {int(differs.nonzero()[0])}"
    torch.testing.assert_close(v_k, v_r, rtol=1e-5, atol=1e-5)
    assert torch.equal(gt_k, gt_r)
    for key in g_r:
        scale = g_r[key].abs().max().item() or 1.0
        err = (g_k[key] - g_r[key]).abs().max().item()
        assert err <= 1e-4 * scale, (key, err, scale)


def test_gating_carries_across_chunks():
    one = _run(DEV, engine)
    two = _run(DEV, engine, chunks=2)
    assert torch.equal(one[0], two[0]) and torch.equal(one[2], two[2])
    torch.testing.assert_close(one[1], two[1], rtol=0, atol=0)


def test_recurrent_presynaptic_dynamics_raise():
    built = sc.recurrent(sc.BATCH_SIZE, sc.SEED)
    model = built.model.to(DEV)
    model.reset_state()
    drive = model._drive()
    gate = Gate(torch.zeros(5, device=DEV), True, False, 0, int(drive.recurrent[0][0].numel()))
    drive = replace(drive, gates=[gate] + [None] * (drive.K_rec + drive.K_ff - 1))
    x = torch.from_numpy(built.input_spikes[:, :10]).to(DEV)
    with pytest.raises(NotImplementedError, match="recurrent"):
        engine.simulate(model.v, model._synaptic, x, drive, model._physiology(),
                        gating=torch.zeros((x.shape[0], 2 * gate.n), device=DEV))
    ff_only = replace(drive, gates=[None] * drive.K_rec + [gate] * drive.K_ff)
    with pytest.raises(ValueError, match="gating state"):
        engine.simulate(model.v, model._synaptic, x, ff_only, model._physiology())


def test_network_with_presynaptic_dynamics_matches_oracle():
    """Through the network API (reference ``tests/test_stp.py:302-312``,
    ``tests/test_saturation.py:332-347``): a feed-forward network whose input sources
    have depressing and facilitating STP onto different targets and saturating NMDA
    synapses, every physiology parameter learnt but the saturating types' tau_decay,
    spike probabilities in the loss — the oracle's spikes, voltages and gradients
    (``test_gpu_nmda._engine_vs_oracle``)."""
    from test_gpu_nmda import LEARN, _engine_vs_oracle

    learn = {**LEARN, "tau_decay": ["AMPA", "GABA_A"]}
    _engine_vs_oracle(lambda: sc.feedforward(sc.BATCH_SIZE, sc.SEED, probabilities=True,
                                             learn=learn, stp=True, saturation=0.63))


@pytest.mark.parametrize("recurrent_gradients", [False, True], ids=["off", "on"])
def test_recurrent_network_with_plastic_inputs_matches_oracle(recurrent_gradients):
    """A recurrent network whose input source has depressing and facilitating STP onto
    its two target types (its recurrent pathways have none), scaling factors and the
    physiology learnt: the oracle's spikes, voltages and gradients through both backward
    passes."""
    from test_gpu_nmda import LEARN, _engine_vs_oracle, _with_flag

    builder = lambda: sc.recurrent(sc.BATCH_SIZE, sc.SEED, scaling_factors=True,  # noqa: E731
                                   learn=LEARN, stp="feedforward")
    _engine_vs_oracle(_with_flag(builder, recurrent_gradients))
