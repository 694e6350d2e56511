"""Spike-frequency adaptation on the GPU against the oracle (reference
``tests/test_adaptation.py:199-248``): spikes, final voltages and every gradient — the
adaptation's rise (``log_adapt``), time constant (``log_tau_adapt``) and reversal
potential (``E_adapt``) among them — through both backward passes, with the refractory
period and the Mg block together, with learnt recurrent weights, and for the
feed-forward network with spike probabilities in the loss; the comparison is
``test_gpu_nmda._engine_vs_oracle`` (the reference's ``_kernels_vs_reference``
protocol).

Beside the oracle: the GPU's tracked adaptation follows its recursion from the GPU's own
spikes (float64, computed here), and the state carries across chunks and checkpoints
bit for bit.
"""

import math

import numpy as np
import pytest
import torch

import oracle.dynamics as oracle_engine
import scenarios as sc
from test_adaptation import ADAPT, LEARN_ADAPT, TAU_ADAPT, _driven
from test_gpu_nmda import LEARN, _engine_vs_oracle, _with_flag
from wiretorch_amd import engine

pytestmark = pytest.mark.gpu
DEV = "cuda"
LEARN_ALL = {**LEARN, **LEARN_ADAPT, "E_adapt": ["excitatory"]}


@pytest.mark.parametrize("recurrent_gradients", [False, True], ids=["off", "on"])
def test_recurrent_matches_oracle(recurrent_gradients):
    builder = lambda: sc.recurrent(  # noqa: E731
        sc.BATCH_SIZE, sc.SEED, scaling_factors=True, learn=LEARN_ALL, adapt=ADAPT)
    grads = _engine_vs_oracle(_with_flag(builder, recurrent_gradients))
    for name in ("log_adapt", "log_tau_adapt", "E_adapt"):
        assert grads[f"cell_parameters.{name}"].abs().sum() > 0, name


@pytest.mark.parametrize("recurrent_gradients", [False, True], ids=["off", "on"])
def test_mechanisms_together_match_oracle(recurrent_gradients):
    """Adaptation, the Mg block and a refractory period at once (the reference's
    ``test_every_mechanism_together`` without presynaptic dynamics)."""
    learn = {**LEARN_ALL, "tau_decay": ["AMPA", "GABA_A"]}
    builder = lambda: sc.recurrent(  # noqa: E731
        sc.BATCH_SIZE, sc.SEED, scaling_factors=True, learn=learn, adapt=ADAPT,
        tau_ref=3.0, mg=1.0)
    _engine_vs_oracle(_with_flag(builder, recurrent_gradients))


def test_learnt_weights_match_oracle():
    builder = lambda: sc.recurrent(sc.BATCH_SIZE, sc.SEED, learnt_weights=True,  # noqa: E731
                                   adapt=ADAPT)
    _engine_vs_oracle(_with_flag(builder, True))


def test_feedforward_matches_oracle():
    _engine_vs_oracle(lambda: sc.feedforward(sc.BATCH_SIZE, sc.SEED, probabilities=True,
                                             learn=LEARN_ALL, adapt=ADAPT))


def test_free_run_matches_oracle():
    """200 steps: the raster equals the oracle's, voltages and the tracked adaptation
    within 1e-5."""
    built = sc.recurrent(sc.BATCH_SIZE, sc.SEED, adapt=ADAPT, tau_ref=3.0)
    x = torch.from_numpy(built.input_spikes)
    runs = []
    for device, eng in (("cpu", oracle_engine), (DEV, engine)):
        model = built.model.to(device)
        sc.use_engine(model, eng)
        model.reset_state()
        model.track_variables, model.track_batch_idx = True, None
        with torch.no_grad():
            out = model(x.to(device))
        runs.append({k: out[k].cpu().numpy() for k in ("spikes", "voltages", "adaptation")}
                    | {"final": model.adaptation.cpu().numpy()})
    ref, gpu = runs
    assert ref["spikes"].sum() > 0 and ref["final"].any()
    differs = (gpu["spikes"] != ref["spikes"]).any(axis=(0, 2))
    assert not differs.any(), f"rasters differ from step {int(np.argmax(differs))}"
    np.testing.assert_allclose(gpu["voltages"], ref["voltages"], rtol=1e-5, atol=65e-5)
    np.testing.assert_allclose(gpu["adaptation"], ref["adaptation"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(gpu["final"], gpu["adaptation"][:, -1], rtol=0, atol=0)


def test_adaptation_follows_the_gpu_spikes():
    """The GPU's tracked adaptation is its recursion from the GPU's own spikes, and it
    lengthens the intervals under constant drive."""
    model = _driven(ADAPT).to(DEV)
    sc.use_engine(model, engine)
    with torch.no_grad():
        out = model(torch.ones((2, 400, 1), device=DEV))
    spikes = out["spikes"].cpu().numpy().astype(np.float64)
    decay = math.exp(-1.0 / TAU_ADAPT)
    a, expected = np.zeros(spikes[:, 0].shape), []
    for t in range(spikes.shape[1]):
        a = a * decay + ADAPT * spikes[:, t]
        expected.append(a)
    np.testing.assert_allclose(out["adaptation"].cpu().numpy(), np.stack(expected, 1),
                               rtol=1e-5, atol=1e-6)
    intervals = torch.diff(torch.nonzero(out["spikes"][0, :, 0].cpu()).flatten())
    assert len(intervals) > 3 and intervals[-1] > 1.5 * intervals[0]


def test_state_carries_across_chunks_and_checkpoints():
    """One launch of 60 steps, six chunks of 10, and six chunks through checkpoints give
    the same spikes and adaptation, bit for bit."""
    runs = []
    for mode in ("one", "chunks", "checkpoints"):
        built = sc.recurrent(sc.BATCH_SIZE, sc.SEED, adapt=ADAPT)
        model = built.model.to(DEV)
        sc.use_engine(model, engine)
        model.reset_state()
        x = torch.from_numpy(built.input_spikes[:, :60]).to(DEV)
        with torch.no_grad():
            if mode == "one":
                runs.append((model(x).cpu(), model.adaptation.cpu().clone()))
                continue
            chunks = []
            for start in range(0, 60, 10):
                if mode == "checkpoints":
                    state = model.get_checkpoint_state()
                    model.reset_state()
                    model.load_checkpoint_state(state)
                chunks.append(model(x[:, start:start + 10]).cpu())
        runs.append((torch.cat(chunks, dim=1), model.adaptation.cpu().clone()))
    assert runs[0][1].any()
    for run in runs[1:]:
        torch.testing.assert_close(run, runs[0], rtol=0, atol=0)
