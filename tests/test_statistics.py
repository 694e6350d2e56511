"""Long-horizon firing statistics against the reference's recording.

``tests/golden/reference/statistics.npz`` (the reference's ``tests/fixtures/statistics.npz``)
holds, for a 2000-neuron recurrent network run 3000 steps and a 1000-neuron feedforward
network run 2000 steps (4 trials, the first 500 steps discarded), per-neuron rates for
two independent inputs and the feedforward spike trains of the first input
(reference ``tests/fixtures/generate.py:201-271``).

Recurrent networks are chaotic, so after a few tens of steps any difference in rounding
gives different spike trains; the recurrent network is compared statistically, with the
recording's own input-to-input variability as the yardstick, as in the reference's
``tests/test_statistics.py:50-76``. The feedforward network is not chaotic: its spike
trains agree almost exactly (``tests/test_statistics.py:79-86``).

Both the oracle (CPU) and the HIP engine (GPU) are held to these criteria.
"""

import numpy as np
import pytest
import torch

import oracle.dynamics as oracle_engine
import scenarios as sc

BATCH, BURN_IN, CHUNK = 4, 500, 250
INPUT_SEEDS = (0, 1)
NETWORKS = {  # name: (builder, sizes, steps)
    "recurrent": (sc.recurrent, dict(n=2000, n_ff=600), 3000),
    "feedforward": (sc.feedforward, dict(n=1000, n_ff=400), 2000),
}


@pytest.fixture(scope="module")
def recorded():
    return sc.load_fixture("statistics")


def build(name, input_seed):
    builder, sizes, steps = NETWORKS[name]
    return builder(BATCH, sc.SEED, n_steps=steps, input_seed=input_seed, **sizes)


def stats_run(name, input_seed, engine, device):
    """Free run in chunks of 250 steps (the state carried across calls); the spikes
    after the burn-in, as a bool array on the host."""
    built = build(name, input_seed)
    model = built.model.to(device)
    sc.use_engine(model, engine)
    x = torch.from_numpy(built.input_spikes).float().to(device)
    out = []
    with torch.no_grad():
        for start in range(0, x.shape[1], CHUNK):
            out.append(sc.unpack_output(model(x[:, start : start + CHUNK]))["spikes"])
    spikes = torch.cat(out, dim=1)[:, BURN_IN:]
    return built, (spikes > 0.5).cpu().numpy()


def population_means(rates, types):
    return np.array([rates[types == t].mean() for t in np.unique(types)])


def check_recurrent(built, spikes, recorded):
    types = built.structure["types"]
    rates = spikes.mean(axis=(0, 1)) * 1000.0
    rec_a = recorded["recurrent.rates.0"]
    rec_b = recorded["recurrent.rates.1"]
    reference = population_means(rec_a, types)
    allowed = np.maximum(2 * np.abs(population_means(rec_b, types) - reference), 0.02 * reference)
    got = population_means(rates, types)
    assert np.all(np.abs(got - reference) <= allowed), (got, reference, allowed)
    floor = np.corrcoef(rec_a, rec_b)[0, 1]
    assert np.corrcoef(rates, rec_a)[0, 1] >= floor - 0.01


def check_feedforward(spikes, recorded):
    reference = recorded["feedforward.spikes"]
    assert spikes.shape == reference.shape
    mismatched = (spikes != reference).sum() / reference.sum()
    assert mismatched < 1e-3, f"{mismatched:.3%} of spikes differ from the recording"


@pytest.mark.parametrize("name", list(NETWORKS))
@pytest.mark.parametrize("input_seed", INPUT_SEEDS)
def test_statistics_fingerprints(name, input_seed, recorded):
    """The networks and inputs rebuilt here are the recorded ones."""
    _, meta = recorded
    assert sc.fingerprint(build(name, input_seed)) == meta["fingerprints"][f"{name}.{input_seed}"]


@pytest.mark.slow
def test_oracle_recurrent_rates(recorded):
    built, spikes = stats_run("recurrent", 0, oracle_engine, "cpu")
    check_recurrent(built, spikes, recorded[0])


def test_oracle_feedforward_spikes(recorded):
    _, spikes = stats_run("feedforward", 0, oracle_engine, "cpu")
    check_feedforward(spikes, recorded[0])


@pytest.mark.gpu
def test_gpu_recurrent_rates(recorded):
    from wiretorch_amd import engine

    built, spikes = stats_run("recurrent", 0, engine, "cuda")
    check_recurrent(built, spikes, recorded[0])


@pytest.mark.gpu
def test_gpu_feedforward_spikes(recorded):
    from wiretorch_amd import engine

    _, spikes = stats_run("feedforward", 0, engine, "cuda")
    check_feedforward(spikes, recorded[0])
