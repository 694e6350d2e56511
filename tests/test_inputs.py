"""On-device Poisson input, host side (CPU): the numpy Philox4x32-10 replay against the
generator's published known-answer vectors, and the replayed spikes' rates and windows."""

import numpy as np
import pytest
import torch

from wiretorch_amd.inputs import PoissonInput, firing_probability, philox4x32_10

# Philox4x32-10 known-answer vectors (counter, key) -> output, as published with the
# generator (Random123's kat_vectors: zero, all-ones, and the digits of pi).
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("counter, key, want", KAT)
def test_philox_known_answers(counter, key, want):
    got = philox4x32_10(*[np.uint32(c) for c in counter], *key)
    assert tuple(int(w) for w in got) == want


def test_firing_probability_is_the_references_float32_product():
    rates = np.array([5.0, 10.0, 17.3, 250.0], dtype=np.float32)
    p = firing_probability(rates, 0.1)
    assert p.dtype == torch.float32
    assert torch.equal(p, torch.from_numpy(rates) * 0.1 * 1e-3)


def test_replayed_spikes_have_the_rates_and_windows_continue_the_stream():
    rates = np.linspace(5.0, 50.0, 40)
    x = PoissonInput(rates, dt=1.0, batch_size=16, n_steps=2000, seed=1234, device="cpu")
    spikes = x.replay()
    assert spikes.shape == (16, 2000, 40) and spikes.dtype == bool
    p = firing_probability(rates, 1.0).numpy()
    got = spikes.mean(axis=(0, 1))
    sd = np.sqrt(p * (1 - p) / (16 * 2000))
    assert np.all(np.abs(got - p) < 5 * sd), (got, p)
    # channels and trials are not correlated: pairwise coincidence at the product rate
    both = (spikes[:, :, 0] & spikes[:, :, 39]).mean()
    assert abs(both - p[0] * p[39]) < 5 * np.sqrt(p[0] * p[39] / (16 * 2000))
    assert np.array_equal(x.window(700, 1300).replay(), spikes[:, 700:1300])
    other = PoissonInput(rates, dt=1.0, batch_size=16, n_steps=2000, seed=1235, device="cpu")
    assert not np.array_equal(other.replay(), spikes)
