"""The voltage-dependent Mg block of NMDA synapse types, on the CPU (reference
``tests/test_nmda.py``): a type with ``mg > 0`` scales its current by
``B(v) = 1 / (1 + (mg / mg_k) exp(-mg_slope v))`` (Jahr & Stevens).

These pin the oracle's restatement (``oracle.dynamics.mg_block`` / ``membrane``): the
tables follow the published defaults, ``mg = 0`` leaves the network bit for bit as it
was, the block changes the spikes, and every tracked current equals ``B G (v - E)``
evaluated in float64 from the tracked voltages and conductances entering the step (a
closed form independent of the restatement's code). The GPU's forward and gradients are
checked against the oracle in ``test_gpu_nmda.py``.
"""

import numpy as np
import pytest
import torch

import oracle.dynamics as oracle_engine
import scenarios as sc
from wiretorch_amd.synapses import MG_K, MG_SLOPE

MG = 1.0  # mM, the physiological concentration


def _run(built, steps=60, track=False):
    model = built.model
    sc.use_engine(model, oracle_engine)
    model.reset_state()
    model.track_variables, model.track_batch_idx = track, None
    with torch.no_grad():
        return model(torch.from_numpy(built.input_spikes[:, :steps]))


def test_block_tables():
    """``mg_c = mg / mg_k`` and ``mg_a = mg_slope`` with the Jahr-Stevens defaults; a type
    without ``mg`` has no block."""
    model = sc.recurrent(sc.BATCH_SIZE, sc.SEED, mg=MG).model
    names = [s["name"] for s in model.registry.synapses]
    nmda = torch.tensor([name == "NMDA" for name in names])
    torch.testing.assert_close(model.mg_c, torch.where(nmda, MG / MG_K, 0.0))
    torch.testing.assert_close(model.mg_a, torch.full((len(names),), MG_SLOPE))
    assert (MG_K, MG_SLOPE) == (3.57, 0.062)
    assert model._mg_block and model._physiology().mg_c is not None
    plain = sc.recurrent(sc.BATCH_SIZE, sc.SEED).model
    assert not plain._mg_block and plain._physiology().mg_c is None


@pytest.mark.parametrize("build", [sc.recurrent, sc.feedforward], ids=["rec", "ff"])
def test_no_block_is_the_former_network(build):
    """``mg = 0`` (and absent) changes nothing, bit for bit."""
    runs = []
    for mg in (None, 0.0):
        built = build(sc.BATCH_SIZE, sc.SEED, mg=mg)
        spikes = _run(built)
        runs.append((spikes, built.model.v.clone()))
    torch.testing.assert_close(runs[0], runs[1], rtol=0, atol=0)


def test_block_changes_the_network():
    off, on = (_run(sc.recurrent(sc.BATCH_SIZE, sc.SEED, mg=mg), 150) for mg in (None, MG))
    assert on.sum() > 0 and not torch.equal(off, on)


def test_tracked_currents_follow_the_formula():
    """Step t's tracked current of type s is B_s(v) clip(g_s) (v - E_s) at the voltage
    and conductances entering the step (step t - 1's tracked ones), B = 1 for the types
    without a block; the block binds on most NMDA currents at these voltages."""
    built = sc.recurrent(sc.BATCH_SIZE, sc.SEED, mg=MG)
    model = built.model
    out = _run(built, 60, track=True)
    v = out["voltages"][:, :-1].double()
    G = out["conductances"][:, :-1].sum(dim=3).double()  # (B, T, N, S)
    G = torch.minimum(G.clamp(min=0.0), model.g_clip.double())
    E, c, a = (getattr(model, k).double() for k in ("E_syn", "mg_c", "mg_a"))
    B = 1 / (1 + c * torch.exp(-a * v[..., None]))
    expected = B * G * (v[..., None] - E)
    actual = out["currents"][:, 1:].double()
    scale = expected.abs().max().item()
    torch.testing.assert_close(actual, expected, rtol=1e-5, atol=1e-6 * scale)
    nmda = torch.tensor([s["name"] == "NMDA" for s in model.registry.synapses])
    assert (B[..., nmda] < 0.5).double().mean() > 0.5
    assert bool((B[..., ~nmda] == 1).all())


def test_block_at_the_limits():
    """sigmoid(mg_a v - log mg_c): exactly 1 without a block, and the closed form's
    values at a few voltages (in float32, within rounding)."""
    v = torch.tensor([[-90.0, -60.0, -20.0, 0.0, 40.0]])
    c = torch.tensor([0.0, MG / MG_K])
    a = torch.tensor([MG_SLOPE, MG_SLOPE])
    B = oracle_engine.mg_block(v, c, a)
    assert bool((B[..., 0] == 1).all())
    closed = 1 / (1 + (MG / MG_K) * np.exp(-MG_SLOPE * v.double().numpy()[0]))
    np.testing.assert_allclose(B[0, :, 1].numpy(), closed, rtol=1e-6)


def test_checkpoints_load_either_way():
    """The block comes from the synapse parameters, not the saved module."""
    without, with_block = (sc.recurrent(sc.BATCH_SIZE, sc.SEED, mg=mg).model for mg in (None, MG))
    with_block.load_state_dict(without.state_dict())
    without.load_state_dict(with_block.state_dict())
    assert with_block._mg_block and not without._mg_block
