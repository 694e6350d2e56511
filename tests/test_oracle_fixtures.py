"""The CPU oracle against the reference's recorded fixtures.

The fixtures (``tests/golden/reference/*.npz``, copied from the reference's
``tests/fixtures/``) were recorded from the reference's PyTorch CPU step. The oracle
restates that step, and the networks are rebuilt through this package's API, so the
reference's own criteria apply (``tests/test_lockstep.py:23-101``,
``tests/test_free_run.py:24-52``, ``tests/test_gradients.py:19-38`` of the reference):
fingerprints equal, spikes exact, voltages to 1e-4 mV in lockstep and 1e-5 of the
range in a free run, gradients to 1e-4 of each gradient's scale.

This pins the oracle (``oracle.dynamics``) and this package's table builders
(``wiretorch_amd.network``) together.
"""

import numpy as np
import pytest
import torch

import oracle.dynamics as oracle_engine
import scenarios as sc

NAMES = list(sc.SCENARIOS)
TRAINABLE = [n for n in NAMES if n != "recurrent_frozen"]


def build(name):
    built = sc.SCENARIOS[name].build(sc.BATCH_SIZE)
    sc.use_engine(built.model, oracle_engine)
    return built


@pytest.mark.parametrize("name", NAMES)
def test_fingerprint(name):
    _, meta = sc.load_fixture(name)
    assert sc.fingerprint(build(name)) == meta["fingerprint"]


@pytest.mark.parametrize("name", NAMES)
def test_lockstep(name):
    scenario = sc.SCENARIOS[name]
    recorded, _ = sc.load_fixture(name)
    built = build(name)
    model = built.model
    model.track_variables, model.track_batch_idx = True, None
    theta = model.theta.numpy()
    x = torch.from_numpy(built.input_spikes)
    excused = []
    for w, start in enumerate(range(0, x.shape[1], sc.WINDOW)):
        stop = start + sc.WINDOW
        model.load_checkpoint_state({k: recorded[f"state.{k}"][w] for k in scenario.state_keys})
        with torch.no_grad():
            out = sc.unpack_output(model(x[:, start:stop]))
        spikes = out["spikes"].numpy() > 0.5
        v_enter = np.concatenate(
            [recorded["state.v"][w][:, None], recorded["voltages"][:, start : stop - 1]], axis=1
        )
        ok = np.ones(sc.BATCH_SIZE, dtype=bool)
        for b, t, n in zip(*np.nonzero(spikes != recorded["spikes"][:, start:stop])):
            if ok[b]:
                assert abs(v_enter[b, t, n] - theta[n]) < 1e-3
                ok[b] = False
                excused.append((w, b))
        np.testing.assert_allclose(
            out["voltages"].numpy()[ok], recorded["voltages"][ok, start:stop], rtol=0, atol=1e-4
        )
        for key, value in model.get_checkpoint_state().items():
            np.testing.assert_allclose(
                value[ok], recorded[f"state.{key}"][w + 1][ok], rtol=1e-4, atol=1e-5
            )
        if scenario.returns_probabilities:
            np.testing.assert_allclose(
                out["probabilities"].numpy()[ok], recorded["probabilities"][ok, start:stop],
                rtol=0, atol=1e-4,
            )
    assert len(excused) <= 0.01 * (x.shape[1] // sc.WINDOW) * sc.BATCH_SIZE


@pytest.mark.parametrize("name", NAMES)
def test_free_run_exact(name):
    recorded, _ = sc.load_fixture(name)
    scenario = sc.SCENARIOS[name]
    run = sc.free_run(scenario, build(name))
    assert np.array_equal(run["spikes"], recorded["spikes"])
    atol = 1e-5 * np.ptp(recorded["voltages"])
    np.testing.assert_allclose(run["voltages"], recorded["voltages"], rtol=0, atol=atol)
    if scenario.returns_probabilities:
        np.testing.assert_allclose(
            run["probabilities"], recorded["probabilities"], rtol=0, atol=1e-5
        )


@pytest.mark.parametrize("track", [False, True], ids=["plain", "tracking"])
@pytest.mark.parametrize("name", TRAINABLE)
def test_gradients(name, track):
    recorded, _ = sc.load_fixture(name)
    loss, grads = sc.gradients(build(name), track=track)
    expected = {k[len("grad."):]: v for k, v in recorded.items() if k.startswith("grad.")}
    assert grads.keys() == expected.keys()
    np.testing.assert_allclose(loss, recorded["loss"], rtol=1e-4)
    for key, value in expected.items():
        scale = np.abs(value).max() or 1.0
        np.testing.assert_allclose(grads[key], value, rtol=0, atol=1e-4 * scale, err_msg=key)
